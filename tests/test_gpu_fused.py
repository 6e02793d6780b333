"""GPU parity of the fused GEMV forms through the C ABI.

Contract ops (reference gpu/backend/vulkan/root.zig:150-194):
  * matVecGateUpResidentBurstAsync: out[r] = act(gate_r . x, up_r . x), against
    the oracle's fusedGateUpRows restatement (matvec/form/fused.zig:27-86);
  * matVecMlpResidentBurstAsync / matVecMlpPairResidentBurstAsync: the SwiGLU
    MLP down . act(gate . x, up . x) (fused.zig:387-413), against the oracle's
    gate_up followed by its production GEMV.
Device-level forms used by the decode step: RMSNorm folded into the GEMV
(norm.zig:26-37, restated here in float64), the residual epilogue and the
normed gate_up.  Bar: relative L2 <= 1e-3 (the reference GPU tests' shapes
and activation, gpu/root_test.zig:180-326, use the same kernels).
"""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import ref_x, rel_l2
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu

TYPES = [synth.Q4_0, synth.Q8_0, synth.Q4_K, synth.Q6_K, synth.Q4_1, synth.F32, synth.F16, synth.BF16]
NAMES = synth.TYPE_NAMES
REL_L2 = 1e-3


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _rmsnorm(x, w, eps):
    """norm.zig:26-37 in float64: x * (1/sqrt(mean(x^2) + eps)) * w."""
    x64 = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(x64 * x64) + eps)
    return (x64 * inv * w.astype(np.float64)).astype(np.float32)


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("rows,k", [(64, 256), (333, 4096), (130, 3840), (70, 5120), (96, 8192), (40, 12288)])
@pytest.mark.parametrize("act", [zd.SILU, zd.GELU], ids=["silu", "gelu"])
def test_gate_up_matches_oracle(dev, qt, rows, k, act):
    if k % synth.BLOCK_ELEMS[qt]:
        pytest.skip("k not a multiple of the block")
    _say(f"gate_up {NAMES[qt]} rows={rows} k={k} act={act}")
    wg = synth.weights(qt, rows, k, seed=rows + k)
    wu = synth.weights(qt, rows, k, seed=rows + k + 1)
    x = synth.activation(k + 3, k)
    want = oracle.gate_up(qt, wg, wu, k, rows, x, act)
    rg, ru = dev.upload_resident(wg), dev.upload_resident(wu)
    h = dev.mat_vec_gate_up_resident_burst_async(rg, ru, zd.quant(qt), rows, k, x, act, zd.PLAIN, True)
    assert h is not None, dev.last_error()
    out = np.full(rows, np.nan, np.float32)
    assert dev.wait_resident(h, out, rows), dev.last_error()
    assert rel_l2(out, want) <= REL_L2
    dev.free_resident(rg)
    dev.free_resident(ru)


# GpuVariant codes select the fused kernel's row tile (u4/u8 four output rows
# per wave tile, un2/un4 two, the others one) for the quants the reference
# grid lists gate_up variants for; ragged row counts leave partial tiles.
@pytest.mark.parametrize("qt", [synth.Q4_0, synth.Q4_1, synth.Q8_0], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("variant", [zd.PLAIN, zd.UN2, zd.U4, zd.SUB], ids=["plain", "un2", "u4", "sub"])
@pytest.mark.parametrize("rows,k", [(333, 4096), (320, 1024), (41, 8192), (5, 256), (12288, 4096)])
def test_gate_up_variants_match_oracle(dev, qt, variant, rows, k):
    _say(f"gate_up variant {variant} {NAMES[qt]} rows={rows} k={k}")
    wg = synth.weights(qt, rows, k, seed=3 * rows + k)
    wu = synth.weights(qt, rows, k, seed=3 * rows + k + 1)
    x = synth.activation(k + 9, k)
    want = oracle.gate_up(qt, wg, wu, k, rows, x, zd.GELU)
    rg, ru = dev.upload_resident(wg), dev.upload_resident(wu)
    h = dev.mat_vec_gate_up_resident_burst_async(rg, ru, zd.quant(qt), rows, k, x, zd.GELU, variant, True)
    assert h is not None, dev.last_error()
    out = np.full(rows, np.nan, np.float32)
    assert dev.wait_resident(h, out, rows), dev.last_error()
    assert rel_l2(out, want) <= REL_L2
    # the MLP op applies the variant to its gate_up: the down GEMV (64 rows,
    # k = ffn = rows) over the gate_up result
    if rows % 32 == 0 and rows <= 4096:
        wd = synth.weights(qt, 64, rows, seed=7)
        rd = dev.upload_resident(wd)
        h = dev.mat_vec_mlp_resident_burst_async(rg, ru, rd, zd.quant(qt), 64, k, rows, x, zd.GELU, variant, True)
        got = np.zeros(64, np.float32)
        assert h is not None and dev.wait_resident(h, got, 64), dev.last_error()
        assert rel_l2(got, oracle.matvec(qt, wd, rows, 64, want)) <= REL_L2
        dev.free_resident(rd)
    dev.free_resident(rg)
    dev.free_resident(ru)


def test_gate_up_reference_shape(dev):
    """The reference GPU test's gate_up case: 64 rows x k=256 q4_0, x[i] = (i%11)*0.1-0.5."""
    rows, k = 64, 256
    wg = synth.weights(synth.Q4_0, rows, k, seed=5)
    wu = synth.weights(synth.Q4_0, rows, k, seed=6)
    x = ref_x(k)
    for act in (zd.SILU, zd.GELU):
        want = oracle.gate_up(synth.Q4_0, wg, wu, k, rows, x, act)
        rg, ru = dev.upload_resident(wg), dev.upload_resident(wu)
        h = dev.mat_vec_gate_up_resident_burst_async(rg, ru, zd.quant(zd.Q4_0), rows, k, x, act, zd.U4, True)
        out = np.zeros(rows, np.float32)
        assert h is not None and dev.wait_resident(h, out, rows), dev.last_error()
        assert np.all(np.abs(out - want) <= 1e-4 + 1e-4 * np.abs(want))
        dev.free_resident(rg)
        dev.free_resident(ru)


@pytest.mark.parametrize("gq,dq,rows,k,ffn", [
    (synth.Q4_0, synth.Q4_0, 64, 256, 512),
    (synth.Q4_0, synth.Q4_0, 4096, 4096, 12288),
    (synth.Q8_0, synth.Q4_0, 256, 1024, 3072),
    (synth.Q4_K, synth.Q6_K, 128, 3840, 15360),
    (synth.Q6_K, synth.Q8_0, 96, 2048, 768),
    (synth.Q4_1, synth.Q4_1, 256, 4096, 1024),
    (synth.F16, synth.BF16, 128, 1024, 2048),
    (synth.F32, synth.Q4_1, 64, 512, 1536),
])
def test_mlp_pair_matches_oracle(dev, gq, dq, rows, k, ffn):
    _say(f"mlp {NAMES[gq]}/{NAMES[dq]} rows={rows} k={k} ffn={ffn}")
    wg = synth.weights(gq, ffn, k, seed=ffn + 1)
    wu = synth.weights(gq, ffn, k, seed=ffn + 2)
    wd = synth.weights(dq, rows, ffn, seed=ffn + 3)
    x = synth.activation(k + 7, k)
    mid = oracle.gate_up(gq, wg, wu, k, ffn, x, zd.SILU)
    want = oracle.matvec(dq, wd, ffn, rows, mid)
    rg, ru, rd = dev.upload_resident(wg), dev.upload_resident(wu), dev.upload_resident(wd)
    h = dev.mat_vec_mlp_pair_resident_burst_async(rg, ru, rd, zd.quant(gq), zd.quant(dq), rows, k, ffn, x,
                                                  zd.SILU, zd.PLAIN, True)
    assert h is not None, dev.last_error()
    out = np.full(rows, np.nan, np.float32)
    assert dev.wait_resident(h, out, rows), dev.last_error()
    assert rel_l2(out, want) <= REL_L2
    if gq == dq:
        h = dev.mat_vec_mlp_resident_burst_async(rg, ru, rd, zd.quant(gq), rows, k, ffn, x, zd.SILU, zd.PLAIN,
                                                 True)
        out2 = np.zeros(rows, np.float32)
        assert h is not None and dev.wait_resident(h, out2, rows), dev.last_error()
        np.testing.assert_array_equal(out2, out)
    for r in (rg, ru, rd):
        dev.free_resident(r)


def test_fused_ops_share_the_burst_activation(dev):
    """A burst: a plain GEMV stages x (first), then gate_up and the MLP reuse it."""
    rows, k, ffn = 128, 1024, 2048
    w = synth.weights(synth.Q4_0, rows, k, seed=1)
    wg = synth.weights(synth.Q4_0, ffn, k, seed=2)
    wu = synth.weights(synth.Q4_0, ffn, k, seed=3)
    wd = synth.weights(synth.Q4_0, rows, ffn, seed=4)
    x = synth.activation(9, k)
    r, rg, ru, rd = (dev.upload_resident(a) for a in (w, wg, wu, wd))
    q = zd.quant(zd.Q4_0)
    h0 = dev.mat_vec_resident_burst_async(r, q, rows, k, x, True)
    h1 = dev.mat_vec_gate_up_resident_burst_async(rg, ru, q, ffn, k, x, zd.SILU, zd.PLAIN, False)
    h2 = dev.mat_vec_mlp_resident_burst_async(rg, ru, rd, q, rows, k, ffn, x, zd.SILU, zd.PLAIN, False)
    assert None not in (h0, h1, h2), dev.last_error()
    o0, o1, o2 = np.zeros(rows, np.float32), np.zeros(ffn, np.float32), np.zeros(rows, np.float32)
    assert dev.wait_resident(h2, o2, rows) and dev.wait_resident(h0, o0, rows) and dev.wait_resident(h1, o1, ffn)
    assert rel_l2(o0, oracle.matvec(synth.Q4_0, w, k, rows, x)) <= REL_L2
    mid = oracle.gate_up(synth.Q4_0, wg, wu, k, ffn, x, zd.SILU)
    assert rel_l2(o1, mid) <= REL_L2
    assert rel_l2(o2, oracle.matvec(synth.Q4_0, wd, ffn, rows, mid)) <= REL_L2
    # a member with another activation than the burst's is refused
    other = x.copy()
    assert dev.mat_vec_gate_up_resident_burst_async(rg, ru, q, ffn, k, other, zd.SILU, zd.PLAIN, False) is None
    for res in (r, rg, ru, rd):
        dev.free_resident(res)


def test_fused_ops_reject_bad_arguments(dev):
    rows, k = 32, 256
    wg = synth.weights(synth.Q4_0, rows, k, seed=1)
    x = synth.activation(1, k)
    rg, ru = dev.upload_resident(wg), dev.upload_resident(wg)
    q = zd.quant(zd.Q4_0)
    assert dev.mat_vec_gate_up_resident_burst_async(rg, ru, q, rows, k, x, 2, zd.PLAIN, True) is None  # act
    assert dev.mat_vec_gate_up_resident_burst_async(rg, ru, q, rows + 1, k, x, zd.SILU, zd.PLAIN, True) is None
    short = dev.upload_resident(wg[: len(wg) // 2].copy())
    assert dev.mat_vec_mlp_resident_burst_async(rg, ru, short, q, rows, k, k, x, zd.SILU, zd.PLAIN, True) is None
    h = dev.mat_vec_gate_up_resident_burst_async(rg, ru, q, rows, k, x, zd.SILU, zd.PLAIN, True)
    out = np.zeros(rows, np.float32)
    assert h is not None and dev.wait_resident(h, out, rows)  # still healthy
    for r in (rg, ru, short):
        dev.free_resident(r)


def _dev_vec(dev, a):
    p = dev.dev_malloc(a.nbytes)
    dev.dev_upload(p, a)
    return p


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("rows,k", [(256, 4096), (100, 3840), (64, 2048), (5000, 4096), (4133, 12288), (77, 11264),
                                    (72, 5120), (40, 8192)])
def test_device_forms_match_oracle(dev, qt, rows, k):
    """norm / resid / normpair forms on device buffers (the decode step's ops);
    the larger shapes give the prefetching instances several row tiles per
    wave and a ragged last tile."""
    if k % synth.BLOCK_ELEMS[qt]:
        pytest.skip("k not a multiple of the block")
    _say(f"forms {NAMES[qt]} rows={rows} k={k}")
    eps = 1e-6
    w = synth.weights(qt, rows, k, seed=k + 11)
    wu = synth.weights(qt, rows, k, seed=k + 12)
    x = synth.activation(k + 13, k) * np.float32(3.0)
    nw = (1.0 + 0.1 * synth.activation(k + 14, k)).astype(np.float32)
    res = synth.activation(k + 15, rows)
    rw, ru = dev.upload_resident(w), dev.upload_resident(wu)
    xd, nwd, resd, yd = _dev_vec(dev, x), _dev_vec(dev, nw), _dev_vec(dev, res), dev.dev_malloc(rows * 4)
    q = zd.quant(qt)
    xn = _rmsnorm(x, nw, eps)
    cases = [
        (zd.FORM_NORM, dict(norm_w=nwd, eps=eps), oracle.matvec(qt, w, k, rows, xn)),
        (zd.FORM_RESID, dict(res=resd), res + oracle.matvec(qt, w, k, rows, x)),
        (zd.FORM_NORMPAIR, dict(norm_w=nwd, eps=eps, w_up=ru, act=zd.SILU),
         oracle.gate_up(qt, w, wu, k, rows, xn, zd.SILU)),
        (zd.FORM_PAIR, dict(w_up=ru, act=zd.GELU), oracle.gate_up(qt, w, wu, k, rows, x, zd.GELU)),
        (zd.FORM_PLAIN, dict(), oracle.matvec(qt, w, k, rows, x)),
    ]
    for form, kw, want in cases:
        assert dev.gemv_op_enqueue(form, q, rw, rows, k, xd, yd, **kw), dev.last_error()
        got = np.zeros(rows, np.float32)
        dev.dev_download(got, yd)
        assert rel_l2(got, want) <= REL_L2, form
    # the residual form in place (res aliases y), as the decode step uses it
    dev.dev_upload(yd, res)
    assert dev.gemv_op_enqueue(zd.FORM_RESID, q, rw, rows, k, xd, yd, res=yd), dev.last_error()
    got = np.zeros(rows, np.float32)
    dev.dev_download(got, yd)
    assert rel_l2(got, res + oracle.matvec(qt, w, k, rows, x)) <= REL_L2
    # missing buffers are refused
    assert not dev.gemv_op_enqueue(zd.FORM_NORM, q, rw, rows, k, xd, yd)
    assert not dev.gemv_op_enqueue(zd.FORM_PAIR, q, rw, rows, k, xd, yd)
    for p in (xd, nwd, resd, yd):
        dev.dev_free(p)
    dev.free_resident(rw)
    dev.free_resident(ru)


# Row counts around the split-K kernels' tile and grid sizes (2-row tiles for
# q8_0 and the K-quants, 4-row for q4_0, one workgroup per CU): fewer rows than a tile, a
# ragged last tile, fewer tiles than CUs, one tile past a whole grid, and
# several ring turns per workgroup.
SPLIT_ROWS = [1, 3, 5, 255, 513, 1028, 2051, 3000]


@pytest.mark.parametrize("qt,k", [(synth.Q8_0, 12288), (synth.Q4_0, 12288), (synth.Q4_K, 15360), (synth.Q6_K, 15360)],
                         ids=["q8_0", "q4_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("rows", SPLIT_ROWS)
def test_split_k_shapes_match_oracle(dev, qt, k, rows):
    """The down-projection shapes run split-K (q8_0 / q4_0 at k = 12288, the
    K-quants at k = 15360, whose 480 chunks per row leave the last wave half
    idle): the plain form and the residual form (also in place, res aliasing
    y) against the oracle, and two launches agree bit for bit (the waves'
    partials meet in a fixed order)."""
    _say(f"split-k {NAMES[qt]} rows={rows}")
    w = synth.weights(qt, rows, k, seed=rows + 901)
    x = synth.activation(rows + 902, k)
    res = synth.activation(rows + 903, rows)
    rw = dev.upload_resident(w)
    xd, resd, yd = _dev_vec(dev, x), _dev_vec(dev, res), dev.dev_malloc(rows * 4)
    q = zd.quant(qt)
    want = oracle.matvec(qt, w, k, rows, x)
    got = np.zeros(rows, np.float32)
    again = np.zeros(rows, np.float32)
    assert dev.gemv_op_enqueue(zd.FORM_PLAIN, q, rw, rows, k, xd, yd), dev.last_error()
    dev.dev_download(got, yd)
    assert rel_l2(got, want) <= REL_L2
    assert dev.gemv_op_enqueue(zd.FORM_PLAIN, q, rw, rows, k, xd, yd), dev.last_error()
    dev.dev_download(again, yd)
    np.testing.assert_array_equal(again.view(np.uint32), got.view(np.uint32))
    assert dev.gemv_op_enqueue(zd.FORM_RESID, q, rw, rows, k, xd, yd, res=resd), dev.last_error()
    dev.dev_download(got, yd)
    assert rel_l2(got, res + want) <= REL_L2
    dev.dev_upload(yd, res)
    assert dev.gemv_op_enqueue(zd.FORM_RESID, q, rw, rows, k, xd, yd, res=yd), dev.last_error()
    dev.dev_download(again, yd)
    np.testing.assert_array_equal(again.view(np.uint32), got.view(np.uint32))
    for p in (xd, resd, yd):
        dev.dev_free(p)
    dev.free_resident(rw)


# Row lengths just below the split-K shapes: q4_k / q6_k at 58 super-blocks
# (464 chunks: the split-K instance's last wave holds 16 valid chunks and
# clamps the rest), q8_0 / q4_0 one block short of 12288 (no exact split-K
# instance: the one-wave-per-row kernels run).
@pytest.mark.parametrize("qt,k", [(synth.Q4_K, 14848), (synth.Q6_K, 14848), (synth.Q8_0, 12256), (synth.Q4_0, 12256)],
                         ids=["q4_k", "q6_k", "q8_0", "q4_0"])
@pytest.mark.parametrize("rows", [3, 515])
def test_split_k_ragged_rows_match_oracle(dev, qt, k, rows):
    _say(f"split-k ragged {NAMES[qt]} rows={rows} k={k}")
    w = synth.weights(qt, rows, k, seed=rows + k)
    x = synth.activation(rows + 7, k)
    res = synth.activation(rows + 8, rows)
    rw = dev.upload_resident(w)
    xd, resd, yd = _dev_vec(dev, x), _dev_vec(dev, res), dev.dev_malloc(rows * 4)
    q = zd.quant(qt)
    want = oracle.matvec(qt, w, k, rows, x)
    got = np.zeros(rows, np.float32)
    assert dev.gemv_op_enqueue(zd.FORM_PLAIN, q, rw, rows, k, xd, yd), dev.last_error()
    dev.dev_download(got, yd)
    assert rel_l2(got, want) <= REL_L2
    assert dev.gemv_op_enqueue(zd.FORM_RESID, q, rw, rows, k, xd, yd, res=resd), dev.last_error()
    dev.dev_download(got, yd)
    assert rel_l2(got, res + want) <= REL_L2
    for p in (xd, resd, yd):
        dev.dev_free(p)
    dev.free_resident(rw)


def test_contract_timing_helpers_run_the_contract_ops(dev):
    """The contract-path timers (burst + waitResident per GEMV; a decode token
    in the executor's burst pattern) run on small shapes and report positive
    times; a layer whose weights are too short for the shapes is refused."""
    hidden, qr, kvr, ffn, vocab = 256, 256, 128, 512, 1000
    shapes = [(qr, hidden), (kvr, hidden), (kvr, hidden), (hidden, qr), (ffn, hidden), (ffn, hidden), (hidden, ffn)]
    layers = []
    for i in range(2):
        layers.append([dev.upload_resident(synth.weights(synth.Q4_0, r, k, seed=10 * i + j))
                       for j, (r, k) in enumerate(shapes)])
    lm = dev.upload_resident(synth.weights(synth.Q8_0, vocab, hidden, seed=99))
    assert dev.time_contract_gemv(layers[0][:1], zd.quant(zd.Q4_0), qr, hidden, 5) > 0.0
    assert dev.time_contract_decode(layers, zd.quant(zd.Q4_0), hidden, qr, kvr, ffn, lm, zd.quant(zd.Q8_0), vocab,
                                    2) > 0.0
    with pytest.raises(RuntimeError):
        dev.time_contract_decode(layers, zd.quant(zd.Q4_0), hidden, qr, kvr, 2 * ffn, lm, zd.quant(zd.Q8_0), vocab, 1)
    for layer in layers:
        for r in layer:
            dev.free_resident(r)
    dev.free_resident(lm)


# Shapes on the kernel pickers' boundaries: the row classes (<= 8192 rows
# takes the residual form's two-row q4_0 tiles, >= 65536 the tall instances --
# here quants without one), chunk-step counts that are not a whole number of
# 64-chunk steps (k = 4352, 2304, 8448, 12544), the widest generic x and k at
# its maximum.  (A wider sweep of these boundaries -- 8 quants x 20 k x the row
# classes x all forms, 4000 checks -- passed the same bar.)
BOUNDARY_SHAPES = [
    (synth.Q4_0, 8192, 4096), (synth.Q4_0, 8193, 4096), (synth.Q8_0, 8193, 4352), (synth.F16, 65537, 2048),
    (synth.Q4_1, 65537, 2048), (synth.Q4_K, 255, 2304), (synth.Q6_K, 3, 8448), (synth.Q4_0, 255, 12544),
    (synth.F32, 8193, 4352), (synth.BF16, 3, 24576), (synth.Q8_0, 3, 32768),
]


# The lm_head instances from 65536 rows at row lengths past 4096 (prefetching
# 8-wave workgroups, plain and RMSNorm-fused), at 65573 rows (a ragged last
# tile): each form against the oracle and the route in the launch log.
TALL_FORM_SHAPES = [(synth.Q6_K, 5120), (synth.Q8_0, 5120), (synth.Q8_0, 6144), (synth.Q8_0, 7168), (synth.Q8_0, 8192),
                    (synth.Q4_0, 5120), (synth.Q4_0, 8192), (synth.Q4_K, 5120), (synth.Q4_K, 8192), (synth.Q4_1, 5120),
                    (synth.Q4_1, 8192)]


@pytest.mark.parametrize("qt,k", TALL_FORM_SHAPES, ids=[f"{NAMES[q]}-{k}" for q, k in TALL_FORM_SHAPES])
def test_tall_forms_match_oracle(dev, qt, k):
    rows = 65536 + 37
    _say(f"tall forms {NAMES[qt]} rows={rows} k={k}")
    eps = 1e-6
    w = synth.weights(qt, rows, k, seed=rows + 5 * k + qt)
    x = synth.activation(k + 2, k) * np.float32(2.0)
    nw = (1.0 + 0.1 * synth.activation(k + 8, k)).astype(np.float32)
    rw = dev.upload_resident(w)
    assert rw is not None, dev.last_error()
    xd, nwd, yd = _dev_vec(dev, x), _dev_vec(dev, nw), dev.dev_malloc(rows * 4)
    try:
        cases = [(zd.FORM_PLAIN, dict(), oracle.matvec(qt, w, k, rows, x)),
                 (zd.FORM_NORM, dict(norm_w=nwd, eps=eps), oracle.matvec(qt, w, k, rows, _rmsnorm(x, nw, eps)))]
        for form, kw, want in cases:
            assert dev.gemv_op_enqueue(form, zd.quant(qt), rw, rows, k, xd, yd, **kw), dev.last_error()
            dev.sync()
            assert dev.launch_log(True)
            try:
                assert dev.gemv_op_enqueue(form, zd.quant(qt), rw, rows, k, xd, yd, **kw), dev.last_error()
                dev.sync()
                log = dev.launch_log_read()
            finally:
                dev.launch_log(False)
            assert [r["block"] for r in log] == [512], (form, log)
            got = np.zeros(rows, np.float32)
            dev.dev_download(got, yd)
            assert np.isfinite(got).all() and rel_l2(got, want) <= REL_L2, form
    finally:
        for p in (xd, nwd, yd):
            dev.dev_free(p)
        dev.free_resident(rw)


@pytest.mark.parametrize("qt,rows,k", BOUNDARY_SHAPES,
                         ids=[f"{NAMES[q]}-{r}x{k}" for q, r, k in BOUNDARY_SHAPES])
def test_picker_boundary_shapes_match_oracle(dev, qt, rows, k):
    _say(f"boundary shape {NAMES[qt]} rows={rows} k={k}")
    eps = 1e-6
    w = synth.weights(qt, rows, k, seed=rows + 3 * k + qt)
    x = synth.activation(k + 1, k) * np.float32(2.0)
    nw = (1.0 + 0.1 * synth.activation(k + 7, k)).astype(np.float32)
    res = synth.activation(k + 5, rows)
    rw = dev.upload_resident(w)
    assert rw is not None, dev.last_error()
    xd, nwd, resd, yd = _dev_vec(dev, x), _dev_vec(dev, nw), _dev_vec(dev, res), dev.dev_malloc(rows * 4)
    base = oracle.matvec(qt, w, k, rows, x)
    cases = [(zd.FORM_PLAIN, dict(), base), (zd.FORM_RESID, dict(res=resd), res + base),
             (zd.FORM_NORM, dict(norm_w=nwd, eps=eps), oracle.matvec(qt, w, k, rows, _rmsnorm(x, nw, eps)))]
    for form, kw, want in cases:
        assert dev.gemv_op_enqueue(form, zd.quant(qt), rw, rows, k, xd, yd, **kw), dev.last_error()
        got = np.zeros(rows, np.float32)
        dev.dev_download(got, yd)
        assert np.isfinite(got).all() and rel_l2(got, want) <= REL_L2, form
    out = np.full(rows, np.nan, np.float32)
    assert dev.mat_vec_resident(rw, zd.quant(qt), rows, k, x, out), dev.last_error()
    assert rel_l2(out, base) <= REL_L2
    for p in (xd, nwd, resd, yd):
        dev.dev_free(p)
    dev.free_resident(rw)
