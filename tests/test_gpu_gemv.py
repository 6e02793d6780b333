"""GPU parity of the HIP GEMV path against the CPU oracle, through the C ABI.

Bars (from the task's north star and the reference's own GPU tests):
  * dequantized blocks: bit-exact against the oracle's codecs;
  * GEMV outputs: relative L2 <= 1e-3 against the oracle's production sweep,
    and the reference's per-element check |c-g| <= 1e-4 + 1e-4|c| at k=256
    (5e-3 + 1e-4|c| at k=8192) on its fillWeights-style inputs
    (reference gpu/root_test.zig:33-50, :52-128);
  * the activation quantizer: bit-exact (qx, dx, sums).
"""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import assert_close_ref, fill_weights, ref_x, rel_l2
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu

TYPES = [synth.Q4_0, synth.Q8_0, synth.Q4_K, synth.Q6_K, synth.Q4_1, synth.F32, synth.F16, synth.BF16]
NAMES = synth.TYPE_NAMES
REL_L2 = 1e-3


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: NAMES[t])
def test_dequant_bit_exact(dev, qt):
    rows, k = 48, 512
    _say(f"dequant {NAMES[qt]} rows={rows} k={k}")
    w = synth.weights(qt, rows, k, seed=11)
    res = dev.upload_resident(w)
    assert res is not None, dev.last_error()
    got = dev.dequant_resident(res, zd.quant(qt), rows * k)
    assert got is not None, dev.last_error()
    want = oracle.dequant(qt, w, rows * k)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    dev.free_resident(res)


# Row lengths of the configs, every x tier, and the long rows of other models'
# FFN down projections and hidden sizes (5120, 7168, 10240, 11008, 14336,
# 17408, 18944: the split-K instances of 5-10 chunk steps for the 32-element
# chunk quants and 9-19 for q8_0, plus its exact 5- and 7-step instances).
SHAPES = [(64, 256), (37, 512), (333, 4096), (129, 3840), (64, 8192), (257, 12288), (40, 15360), (16, 32768),
          (70, 5120), (41, 7168), (33, 10240), (67, 11008), (130, 14336), (29, 17408), (65, 18944)]


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("rows,k", SHAPES)
def test_gemv_matches_oracle(dev, qt, rows, k):
    if k % synth.BLOCK_ELEMS[qt]:
        pytest.skip("k not a multiple of the block")
    _say(f"gemv {NAMES[qt]} rows={rows} k={k}")
    w = synth.weights(qt, rows, k, seed=rows * 7 + k)
    x = synth.activation(k + 1, k)
    want = oracle.matvec(qt, w, k, rows, x)
    res = dev.upload_resident(w)
    assert res is not None, dev.last_error()
    for variant in (zd.PLAIN, zd.U4, zd.UN2):
        out = np.full(rows, np.nan, np.float32)
        assert dev.mat_vec_resident(res, zd.quant(qt, variant), rows, k, x, out), dev.last_error()
        err = rel_l2(out, want)
        assert err <= REL_L2, f"variant {variant}: rel-L2 {err:.3e}"
    dev.free_resident(res)


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: NAMES[t])
def test_reference_style_parity(dev, qt):
    """The reference's expectMatVecParity / expectAxisParity inputs and tolerances."""
    for rows, k, abs_tol in ((64, 256, 1e-4), (64, 8192, 5e-3)):
        _say(f"reference-style {NAMES[qt]} rows={rows} k={k}")
        w = fill_weights(qt, rows, k)
        x = ref_x(k)
        cpu = oracle.matvec(qt, w, k, rows, x)
        gpu = np.zeros(rows, np.float32)
        assert dev.mat_vec(zd.quant(qt), w, rows, k, x, gpu), dev.last_error()
        assert_close_ref(cpu, gpu, abs_tol=abs_tol)
        res = dev.upload_resident(w)
        out = np.zeros(rows, np.float32)
        assert dev.mat_vec_resident(res, zd.quant(qt), rows, k, x, out)
        assert_close_ref(cpu, out, abs_tol=abs_tol)
        h = dev.mat_vec_resident_burst_async(res, zd.quant(qt), rows, k, x, True)
        assert h is not None, dev.last_error()
        burst = np.zeros(rows, np.float32)
        assert dev.wait_resident(h, burst, rows)
        assert_close_ref(cpu, burst, abs_tol=abs_tol)
        dev.free_resident(res)


def test_async_burst_batch_agree(dev):
    """Every resident path returns the same bits for the same inputs."""
    qt, k = synth.Q4_0, 4096
    shapes = [4096, 1024, 1024]  # q, k, v projections sharing x
    ws = [synth.weights(qt, r, k, seed=100 + i) for i, r in enumerate(shapes)]
    x = synth.activation(5, k)
    ress = [dev.upload_resident(w) for w in ws]
    ref = []
    for r, res in zip(shapes, ress):
        o = np.zeros(r, np.float32)
        assert dev.mat_vec_resident(res, zd.quant(qt), r, k, x, o)
        ref.append(o)
    # plain async
    hs = [dev.mat_vec_resident_async(res, zd.quant(qt), r, k, x) for r, res in zip(shapes, ress)]
    assert all(h is not None for h in hs)
    for h, r, o in zip(hs, shapes, ref):
        got = np.zeros(r, np.float32)
        assert dev.wait_resident(h, got, r)
        np.testing.assert_array_equal(got, o)
    # burst: first stages x, the rest reuse it
    hs = [dev.mat_vec_resident_burst_async(res, zd.quant(qt), r, k, x, i == 0)
          for i, (r, res) in enumerate(zip(shapes, ress))]
    assert all(h is not None for h in hs)
    for h, r, o in zip(hs, shapes, ref):
        got = np.zeros(r, np.float32)
        assert dev.wait_resident(h, got, r)
        np.testing.assert_array_equal(got, o)
    # batch: one x upload, one wait
    outs = [np.zeros(r, np.float32) for r in shapes]
    ops = [zd.ResidentOp(res, zd.quant(qt), r, o) for res, r, o in zip(ress, shapes, outs)]
    assert dev.mat_vec_resident_batch(k, x, ops), dev.last_error()
    for o, want in zip(outs, ref):
        np.testing.assert_array_equal(o, want)
    # oracle agreement of the q projection
    assert rel_l2(ref[0], oracle.matvec(qt, ws[0], k, shapes[0], x)) <= REL_L2
    for res in ress:
        dev.free_resident(res)


@pytest.mark.parametrize("qt,k", [(synth.Q8_0, 4096), (synth.Q4_K, 3840), (synth.F16, 1024), (synth.Q4_1, 12288),
                                  (synth.Q8_0, 12288), (synth.Q4_0, 12288), (synth.Q4_1, 5120), (synth.Q6_K, 5120),
                                  (synth.Q4_0, 8192), (synth.Q8_0, 14336)],
                         ids=["q8_0", "q4_k", "f16", "q4_1", "q8_0_split", "q4_0_split", "q4_1_g8k", "q6_k_g8k",
                              "q4_0_split_mid", "q8_0_split_long"])
def test_batch_one_launch_matches_single_ops(dev, qt, k):
    """A same-quant batch runs as one launch of the batch kernel (op by op
    where the single op sums in another order: split-K at k = 12288 for
    q8_0 / q4_0, int8-plane x for q4_k at k = 3840); every op's
    rows equal the single-op GEMV's bit for bit (same per-lane order and
    reduction), including eight ops of ragged row counts."""
    _say(f"batch {NAMES[qt]} k={k}")
    shapes = [1, 77, 4096, 130, 33, 1024, 2, 513]
    ws = [synth.weights(qt, r, k, seed=300 + i) for i, r in enumerate(shapes)]
    x = synth.activation(31, k)
    ress = [dev.upload_resident(w) for w in ws]
    ref = []
    for r, res in zip(shapes, ress):
        o = np.zeros(r, np.float32)
        assert dev.mat_vec_resident(res, zd.quant(qt), r, k, x, o), dev.last_error()
        ref.append(o)
    outs = [np.full(r, np.nan, np.float32) for r in shapes]
    ops = [zd.ResidentOp(res, zd.quant(qt), r, o) for res, r, o in zip(ress, shapes, outs)]
    assert dev.mat_vec_resident_batch(k, x, ops), dev.last_error()
    for o, want in zip(outs, ref):
        np.testing.assert_array_equal(o, want)
    assert rel_l2(outs[2], oracle.matvec(qt, ws[2], k, shapes[2], x)) <= REL_L2
    # a mixed-quant batch runs op by op and agrees too
    wq = synth.weights(synth.Q4_0, 64, k, seed=399)
    rq = dev.upload_resident(wq)
    oq = np.zeros(64, np.float32)
    assert dev.mat_vec_resident(rq, zd.quant(zd.Q4_0), 64, k, x, oq)
    mixed = [np.zeros(shapes[0], np.float32), np.zeros(64, np.float32)]
    ops = [zd.ResidentOp(ress[0], zd.quant(qt), shapes[0], mixed[0]), zd.ResidentOp(rq, zd.quant(zd.Q4_0), 64, mixed[1])]
    assert dev.mat_vec_resident_batch(k, x, ops), dev.last_error()
    np.testing.assert_array_equal(mixed[0], ref[0])
    np.testing.assert_array_equal(mixed[1], oq)
    for res in ress + [rq]:
        dev.free_resident(res)


def test_ring_refuses_ninth_inflight_and_stale_handles(dev):
    qt, rows, k = synth.Q8_0, 128, 256
    w = synth.weights(qt, rows, k, seed=3)
    x = synth.activation(4, k)
    res = dev.upload_resident(w)
    hs = [dev.mat_vec_resident_async(res, zd.quant(qt), rows, k, x) for _ in range(zd.RING_SIZE)]
    assert all(h is not None for h in hs)
    assert dev.mat_vec_resident_async(res, zd.quant(qt), rows, k, x) is None  # ring full
    want = oracle.matvec(qt, w, k, rows, x)
    out = np.zeros(rows, np.float32)
    for h in hs:
        assert dev.wait_resident(h, out, rows)
        assert rel_l2(out, want) <= REL_L2
    assert not dev.wait_resident(hs[0], out, rows)  # drained handle is stale
    # after draining, the ring accepts again (more than 8 submits in total)
    for _ in range(3):
        h = dev.mat_vec_resident_async(res, zd.quant(qt), rows, k, x)
        assert h is not None
        assert dev.wait_resident(h, out, rows)
    dev.free_resident(res)


def test_burst_member_must_share_first_activation(dev):
    qt, rows, k = synth.Q4_0, 64, 256
    w = synth.weights(qt, rows, k, seed=8)
    x = synth.activation(1, k)
    other = x.copy()
    res = dev.upload_resident(w)
    out = np.zeros(rows, np.float32)
    h = dev.mat_vec_resident_burst_async(res, zd.quant(qt), rows, k, x, True)
    assert h is not None
    assert dev.mat_vec_resident_burst_async(res, zd.quant(qt), rows, k, other, False) is None
    h2 = dev.mat_vec_resident_burst_async(res, zd.quant(qt), rows, k, x, False)
    assert h2 is not None
    assert dev.wait_resident(h, out, rows) and dev.wait_resident(h2, out, rows)
    dev.free_resident(res)


def test_rejections_fall_back(dev):
    """Unsupported quant or shape, short buffers: False, never a crash
    (reference pipeline.zig:1256-1262)."""
    rows, k = 16, 256
    w = synth.weights(synth.Q4_0, rows, k, seed=1)
    x = synth.activation(1, k)
    out = np.zeros(rows, np.float32)
    assert not dev.mat_vec(6, np.zeros(rows * 8 * 22, np.uint8), rows, k, x, out)  # q5_0: no kernel
    xf = synth.activation(2, 40)  # float rows must be a multiple of 32 elements (16-byte rows)
    assert not dev.mat_vec(zd.quant(zd.F32), np.zeros(rows * 40 * 4, np.uint8), rows, 40, xf, out)
    assert not dev.mat_vec(zd.quant(zd.Q4_0), w, rows, k + 16, np.zeros(k + 16, np.float32), out)  # k % 32
    assert not dev.mat_vec(zd.quant(zd.Q4_0), w[:-1], rows, k, x, out)  # short weight
    assert not dev.mat_vec(zd.quant(zd.Q4_0), w, 0, k, x, out)  # rows == 0
    assert not dev.mat_vec(zd.quant(zd.Q4_0), w, rows, k, x, np.zeros(rows - 1, np.float32))  # short out
    assert not dev.mat_vec(zd.quant(zd.Q4_0), w, rows, k, x[:-1].copy(), out)  # x length
    res = dev.upload_resident(w)
    assert not dev.mat_vec_resident(res, zd.quant(zd.Q4_0), rows + 1, k, x, out)  # resident too short
    # a resident keeps one layout: a later different quant is refused
    assert dev.mat_vec_resident(res, zd.quant(zd.Q4_0), rows, k, x, out)
    assert not dev.mat_vec_resident(res, zd.quant(zd.Q8_0), rows // 2, k, x, out)
    dev.free_resident(res)
    # ...and the device is still healthy
    res = dev.upload_resident(w)
    assert dev.mat_vec_resident(res, zd.quant(zd.Q4_0), rows, k, x, out)
    dev.free_resident(res)


def test_quantizer_bit_exact(dev):
    _say("quantize_act_q8")
    x = synth.activation(21, 4096 * 4)
    x[:32] = 0.0  # an all-zero block: d = 0, inv = 0
    x[32:64] = np.float32(127.0) * np.linspace(-1, 1, 32, dtype=np.float32)
    got = dev.quantize_act_q8(x)
    assert got is not None, dev.last_error()
    want = oracle.quantize_act_q8(x)
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[1].view(np.uint32), want[1].view(np.uint32))
    np.testing.assert_array_equal(got[2], want[2])


CONFIG_SHAPES = [
    ("c0_q4_0", synth.Q4_0, 4096, 4096),
    ("tall_q6_k", synth.Q6_K, 65536 + 37, 3840),  # the lm_head kernels (from 65536 rows)
    ("tall_q6_k_5120", synth.Q6_K, 65536 + 37, 5120),  # the two-row 3-step lm_head instance
    # the other lm_head instances (prefetching 8-wave workgroups from 65536 rows)
    ("tall_q4_0_4096", synth.Q4_0, 65536 + 37, 4096),
    ("tall_q4_0_5120", synth.Q4_0, 65536 + 37, 5120),
    ("tall_q4_0_8192", synth.Q4_0, 65536 + 37, 8192),
    ("tall_q4_k_4096", synth.Q4_K, 65536 + 37, 4096),
    ("tall_q4_k_5120", synth.Q4_K, 65536 + 37, 5120),
    ("tall_q4_k_8192", synth.Q4_K, 65536 + 37, 8192),
    ("tall_q4_1_4096", synth.Q4_1, 65536 + 37, 4096),
    ("tall_q4_1_6144", synth.Q4_1, 65536 + 37, 6144),
    ("tall_q4_1_8192", synth.Q4_1, 65536 + 37, 8192),
    ("tall_q8_0_5120", synth.Q8_0, 65536 + 37, 5120),
    ("tall_q8_0_6144", synth.Q8_0, 65536 + 37, 6144),
    ("tall_q8_0_7168", synth.Q8_0, 65536 + 37, 7168),
    ("tall_q8_0_8192", synth.Q8_0, 65536 + 37, 8192),
    ("tall_q8_0", synth.Q8_0, 65536 + 37, 4096),
    ("c1_gate_q8_0", synth.Q8_0, 12288, 4096),
    ("c1_down_q8_0", synth.Q8_0, 4096, 12288),
    ("c3_gate_q4_k", synth.Q4_K, 15360, 3840),
    ("c3_down_q4_k", synth.Q4_K, 3840, 15360),
    ("c3_gate_q6_k", synth.Q6_K, 15360, 3840),
    ("c3_down_q6_k", synth.Q6_K, 3840, 15360),
]


@pytest.mark.parametrize("name,qt,rows,k", CONFIG_SHAPES, ids=[c[0] for c in CONFIG_SHAPES])
def test_benchmark_shapes_match_oracle(dev, name, qt, rows, k):
    """The full benchmark-config GEMVs against the oracle at their real size."""
    _say(f"config shape {name}")
    w = synth.weights(qt, rows, k, seed=0x5A4C4D00 + rows)
    x = synth.activation(0x5A4C4D09, k)
    want = oracle.matvec(qt, w, k, rows, x)
    res = dev.upload_resident(w)
    out = np.zeros(rows, np.float32)
    assert dev.mat_vec_resident(res, zd.quant(qt), rows, k, x, out), dev.last_error()
    assert rel_l2(out, want) <= REL_L2
    dev.free_resident(res)


TALL_ROUTES = [(synth.Q6_K, 3840), (synth.Q6_K, 5120), (synth.Q8_0, 4096), (synth.Q8_0, 5120), (synth.Q8_0, 8192),
               (synth.Q4_0, 4096), (synth.Q4_0, 5120), (synth.Q4_0, 8192), (synth.Q4_K, 5120), (synth.Q4_K, 8192),
               (synth.Q4_1, 4096), (synth.Q4_1, 8192)]


@pytest.mark.parametrize("qt,k", TALL_ROUTES, ids=[f"{synth.TYPE_NAMES[q]}_{k}" for q, k in TALL_ROUTES])
@pytest.mark.parametrize("rows", [65536 + 37, 65535])
def test_tall_route(dev, qt, k, rows):
    """GEMVs of 65536 rows and more take the prefetching lm_head instances
    (8-wave workgroups) where the quant has one for the row length (q4_k's
    k <= 4096 keeps its 16-wave instance); one row fewer keeps the 4- or
    16-wave (or split-K) instances."""
    _say(f"tall route quant={qt} {rows}x{k}")
    w = synth.weights(qt, rows, k, seed=0x5A4C4D50 + k)
    res = dev.upload_resident(w)
    xs = synth.activation(0x5A4C4D51, k)
    x = dev.dev_malloc(xs.nbytes)
    y = dev.dev_malloc(rows * 4)
    try:
        dev.dev_upload(x, xs)
        assert dev.mat_vec_enqueue(res, zd.quant(qt), rows, k, x, y), dev.last_error()
        dev.sync()
        assert dev.launch_log(True)
        try:
            assert dev.mat_vec_enqueue(res, zd.quant(qt), rows, k, x, y), dev.last_error()
            dev.sync()
            log = dev.launch_log_read()
        finally:
            dev.launch_log(False)
        assert [r["what"] for r in log] == ["gemv"]
        assert (log[0]["block"] == 512) == (rows >= 65536), log[0]
    finally:
        dev.dev_free(x)
        dev.dev_free(y)
        dev.free_resident(res)
