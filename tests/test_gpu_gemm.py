"""GPU parity of the matrix products (matMulBatch / matMulResident) through the C ABI.

From 3 tokens on the device runs zlm's int path (q8 activations; the int8
MFMA GEMM, or at 3-4 tokens the int-path token GEMV);
its oracle is the int path of the reference (matvec/kernels/quantized.zig:49-55
for Q4_0, :79-87 for Q4_1, :111-123 for Q4_K, :149-156 for Q8_0, over the
activation quantizer of matvec/layout.zig:458-476) applied per token: relative
L2 <= 1e-3 (the block dots are exact integers; only fp32 scaling and summation
order differ).  Against the fp32 GEMM the reference's own int-vs-fp bound
applies, |int - fp| <= 0.02 * sum|w*x| (kernels/quantized_test.zig:61).  One
or two tokens run the fp GEMV (two tokens in one pass over the weights, more
cases in test_gpu_few_tokens.py), checked against the oracle's fp matMulRows
(form/single.zig:213-292), relative L2 <= 1e-3.
"""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import rel_l2
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


SHAPES = [(64, 256, 4), (100, 512, 37), (64, 1024, 64), (130, 4096, 70), (48, 16384, 3), (70, 4096, 129),
          (64, 4096, 1)]
GEMM_QUANTS = [(synth.Q4_0, zd.Q4_0), (synth.Q8_0, zd.Q8_0), (synth.Q4_1, zd.Q4_1), (synth.Q4_K, zd.Q4_K)]


# Token counts up to this run the fp GEMV path (the host's kGemmGemvM).
GEMV_M = 2


def _oracle(qt, w, k, rows, m, x):
    """The arithmetic the device runs for m tokens: fp GEMVs or the int path."""
    if m <= GEMV_M:
        return oracle.matmul_rows(qt, w, k, rows, m, x)
    return oracle.matmul_int(qt, w, k, rows, m, x)


@pytest.mark.parametrize("qt,zq", GEMM_QUANTS, ids=["q4_0", "q8_0", "q4_1", "q4_k"])
@pytest.mark.parametrize("rows,k,m", SHAPES)
def test_gemm_matches_int_oracle(dev, qt, zq, rows, k, m):
    _say(f"gemm type={qt} rows={rows} k={k} m={m}")
    w = synth.weights(qt, rows, k, seed=rows + k + m)
    x = synth.activation(m + 5, m * k)
    want = _oracle(qt, w, k, rows, m, x)
    out = np.full(m * rows, np.nan, np.float32)
    assert dev.mat_mul_batch(zd.quant(zq), w, rows, k, m, x, out), dev.last_error()
    got = out.reshape(m, rows)
    assert rel_l2(got, want) <= 1e-3
    if m > GEMV_M:
        # the block dots are exact integers, so only the fp32 scaling and
        # summation order may differ (~1e-7); one quantized activation off by
        # one unit moves its token's outputs by ~1e-4
        assert rel_l2(got, want) <= 1e-5
    res = dev.upload_resident(w)
    out2 = np.zeros(m * rows, np.float32)
    assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, m, x, out2), dev.last_error()
    np.testing.assert_array_equal(out2, out)
    # the int path stays within the reference's bound of the fp32 GEMM
    fp = oracle.matmul_rows(qt, w, k, rows, m, x)
    dq = np.abs(oracle.dequant(qt, w, rows * k).reshape(rows, k).astype(np.float64))
    mag = np.abs(x.reshape(m, k).astype(np.float64)) @ dq.T
    assert np.all(np.abs(got - fp) <= 0.02 * mag + 1e-6)
    dev.free_resident(res)


# The small-token paths (m = 3, 4 at k <= 8192: the int-path token GEMV;
# otherwise up to 32: the small-M kernel, one 32-token tile; the workgroup's waves
# split the row's blocks in pairs -- 16 waves and 32-block split steps for
# q4_0 / q8_0, 8 waves and 16-block steps for q4_1 / q4_k): odd block counts
# (a pair's second block past the end), block counts not a multiple of a split
# step (k = 3840 and 288), ragged row tiles, one token, a full tile, and the
# first m past it (a second, one-token tile).  Two more shapes past one token
# tile reach the tiled GEMM split over wave groups (four for q4_0 / q8_0, two
# for q4_1 / q4_k) with an odd block count (k = 288: 9 blocks) and with fewer
# blocks than groups have pairs (k = 96: 3 blocks; the last groups get none).
# A k that is not whole super-blocks for q4_k is rounded up to the next one.
SMALL_M = [(33, 4096, 2), (64, 4096, 9), (96, 3840, 32), (40, 12288, 31), (37, 288, 5), (64, 256, 33),
           (32, 512, 1), (4096 + 17, 4096, 8), (50, 4096, 3), (37, 288, 64), (40, 96, 40)]


@pytest.mark.parametrize("qt,zq", GEMM_QUANTS, ids=["q4_0", "q8_0", "q4_1", "q4_k"])
@pytest.mark.parametrize("rows,k,m", SMALL_M)
def test_small_m_gemm_matches_int_oracle(dev, qt, zq, rows, k, m):
    be = synth.BLOCK_ELEMS[qt]
    k = (k + be - 1) // be * be
    _say(f"small-m gemm type={qt} rows={rows} k={k} m={m}")
    w = synth.weights(qt, rows, k, seed=rows * 3 + k + m)
    x = synth.activation(m + 11, m * k)
    want = _oracle(qt, w, k, rows, m, x)
    res = dev.upload_resident(w)
    out = np.full(m * rows, np.nan, np.float32)
    assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, m, x, out), dev.last_error()
    assert rel_l2(out.reshape(m, rows), want) <= 1e-3
    again = np.full(m * rows, np.nan, np.float32)
    assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, m, x, again), dev.last_error()
    np.testing.assert_array_equal(again.view(np.uint32), out.view(np.uint32))  # fixed summation order
    # From 3 tokens the device runs the int path, where the reference's
    # matMulResident is fp32: the reference's own int-vs-fp bound
    # (kernels/quantized_test.zig:61) holds against the oracle's fp matMulRows
    fp = oracle.matmul_rows(qt, w, k, rows, m, x)
    dq = np.abs(oracle.dequant(qt, w, rows * k).reshape(rows, k).astype(np.float64))
    mag = np.abs(x.reshape(m, k).astype(np.float64)) @ dq.T
    assert np.all(np.abs(out.reshape(m, rows) - fp) <= 0.02 * mag + 1e-6)
    dev.free_resident(res)


def _route(dev, res, zq, rows, k, m, x_dev, out_dev):
    """The launches of one matMul on device buffers (after a first call that
    builds the layouts)."""
    assert dev.mat_mul_enqueue(res, zd.quant(zq), rows, k, m, x_dev, out_dev), dev.last_error()
    dev.sync()
    assert dev.launch_log(True)
    try:
        assert dev.mat_mul_enqueue(res, zd.quant(zq), rows, k, m, x_dev, out_dev), dev.last_error()
        dev.sync()
        return dev.launch_log_read()
    finally:
        dev.launch_log(False)


# Past one 32-token tile the host picks, by a cost model, the small-M kernel
# (one workgroup per 32-row x 32-token tile, grid.y = token tiles) or the
# 128 x 64 tiled GEMM, whose tiles' blocks are split over four 4-wave groups
# (q4_0 / q8_0 at up to one workgroup per CU), two (q4_0 / q8_0 at two per
# CU, q4_1 / q4_k at one) or none (larger grids).  These shapes sit well
# inside each choice: the small-M kernel over four token tiles (the last
# partial); 0.76 workgroups per CU (three 128-token tiles): four groups for
# q4_0 / q8_0, two for q4_1 / q4_k; 1.5 workgroups per CU (two 128-token
# tiles and a ragged row tile): two groups for q4_0 / q8_0, unsplit for
# q4_1 / q4_k; and 2.3 workgroups per CU (three 128-token tiles, the last
# partial): unsplit.  All over a row prefix of a resident holding 64 rows
# more.
MULTI_TILE = [("small", 4096 + 17, 4096, 100), ("split", 4096 + 17, 4096, 384), ("two", 12288 + 40, 4096, 256),
              ("large", 12288 + 40, 4096, 300)]


@pytest.mark.parametrize("qt,zq", GEMM_QUANTS, ids=["q4_0", "q8_0", "q4_1", "q4_k"])
@pytest.mark.parametrize("route,rows,k,m", MULTI_TILE, ids=["small", "split", "two", "large"])
def test_gemm_past_one_token_tile(dev, qt, zq, route, rows, k, m):
    _say(f"gemm past one token tile type={qt} route={route} rows={rows} k={k} m={m}")
    rb = synth.row_bytes(qt, k)
    w = synth.weights(qt, rows + 64, k, seed=rows + m)
    xs = synth.activation(m + 13, m * k)
    res = dev.upload_resident(w)
    x_dev = dev.dev_malloc(xs.nbytes)
    out_dev = dev.dev_malloc(m * rows * 4)
    try:
        dev.dev_upload(x_dev, xs)
        log = _route(dev, res, zq, rows, k, m, x_dev, out_dev)
        gemm = [r for r in log if r["what"].startswith("gemm")]
        assert len(gemm) == 1
        if route == "small":
            assert gemm[0]["what"] == "gemm small"
            assert (gemm[0]["grid_x"], gemm[0]["grid_y"]) == ((rows + 31) // 32, (m + 31) // 32)
        else:
            plain = zq in (zd.Q4_0, zd.Q8_0)
            groups = {"split": 4 if plain else 2, "two": 2 if plain else 1, "large": 1}[route]
            what = {4: "gemm k4", 2: "gemm k2", 1: "gemm"}[groups]
            assert (gemm[0]["what"], gemm[0]["block"]) == (what, 256 * groups)
            assert (gemm[0]["grid_x"], gemm[0]["grid_y"]) == ((rows + 63) // 64, (m + 127) // 128)
        out = np.zeros(m * rows, np.float32)
        dev.dev_download(out, out_dev)
        got = out.reshape(m, rows)
        for r0, r1 in ((0, 64), (rows // 2, rows // 2 + 32), (rows - 48, rows)):
            want = oracle.matmul_int(qt, w[r0 * rb:r1 * rb], k, r1 - r0, m, xs)
            assert rel_l2(got[:, r0:r1], want) <= 1e-5, (r0, r1)
        if route == "small":
            # each 32-token tile is its own workgroup column: the first tile's
            # tokens come out bit for bit as in a one-tile call
            assert dev.mat_mul_enqueue(res, zd.quant(zq), rows, k, 32, x_dev, out_dev), dev.last_error()
            one = np.zeros(32 * rows, np.float32)
            dev.dev_download(one, out_dev)
            np.testing.assert_array_equal(one.view(np.uint32), out[:32 * rows].view(np.uint32))
    finally:
        dev.dev_free(x_dev)
        dev.dev_free(out_dev)
        dev.free_resident(res)


# The split tiled GEMMs' block ranges on rows of few or odd 32-element block
# counts (a group's range is an even number of blocks, the last one short or
# empty): nb = 7 over four groups is 2 + 2 + 2 + 1, nb = 3 is 2 + 1 + 0 + 0,
# nb = 9 over two groups (two workgroups per CU) 6 + 3; q4_k rows are whole
# 256-element super-blocks, so it runs nb = 8 only (4 + 4 over two groups).
# (case, rows, k, m, what the host picks for q4_0 / q8_0 and for q4_1 /
# q4_k.)
SPLIT_RANGES = [("nb7", 4096 + 17, 224, 384, "gemm k4", "gemm k2"),
                ("nb3", 4096 + 17, 96, 384, "gemm k4", "gemm k2"),
                ("nb9", 12288 + 40, 288, 256, "gemm k2", "gemm"),
                ("nb8", 4096 + 17, 256, 384, "gemm k4", "gemm k2")]


SPLIT_RANGE_CASES = [(qt, zq) + c for c in SPLIT_RANGES for qt, zq in GEMM_QUANTS
                     if c[2] % synth.BLOCK_ELEMS[qt] == 0]
GEMM_QUANT_IDS = {synth.Q4_0: "q4_0", synth.Q8_0: "q8_0", synth.Q4_1: "q4_1", synth.Q4_K: "q4_k"}


@pytest.mark.parametrize("qt,zq,case,rows,k,m,plain_what,min_what", SPLIT_RANGE_CASES,
                         ids=[f"{c[2]}-{GEMM_QUANT_IDS[c[0]]}" for c in SPLIT_RANGE_CASES])
def test_gemm_split_block_ranges(dev, qt, zq, case, rows, k, m, plain_what, min_what):
    _say(f"gemm split block ranges type={qt} case={case} rows={rows} k={k} m={m}")
    rb = synth.row_bytes(qt, k)
    w = synth.weights(qt, rows, k, seed=rows + k + m)
    xs = synth.activation(k + m, m * k)
    res = dev.upload_resident(w)
    x_dev = dev.dev_malloc(xs.nbytes)
    out_dev = dev.dev_malloc(m * rows * 4)
    try:
        dev.dev_upload(x_dev, xs)
        log = _route(dev, res, zq, rows, k, m, x_dev, out_dev)
        gemm = [r for r in log if r["what"].startswith("gemm")]
        want_what = plain_what if zq in (zd.Q4_0, zd.Q8_0) else min_what
        assert [r["what"] for r in gemm] == [want_what]
        out = np.zeros(m * rows, np.float32)
        dev.dev_download(out, out_dev)
        got = out.reshape(m, rows)
        for r0, r1 in ((0, 64), (rows // 2, rows // 2 + 32), (rows - 48, rows)):
            want = oracle.matmul_int(qt, w[r0 * rb:r1 * rb], k, r1 - r0, m, xs)
            assert rel_l2(got[:, r0:r1], want) <= 1e-5, (r0, r1)
    finally:
        dev.dev_free(x_dev)
        dev.dev_free(out_dev)
        dev.free_resident(res)


def test_gemm_config4_rows_subset(dev):
    """configs[4] at full size (12288 x 4096 Q4_0 x 512 tokens); rows checked
    against the oracle on a slice of the weight (a GEMM row depends only on its
    own weight row)."""
    rows, k, m = 12288, 4096, 512
    _say("gemm config4 full")
    w = synth.weights(synth.Q4_0, rows, k, seed=0x5A4C4D04)
    x = synth.activation(0x5A4C4D0D, m * k)
    res = dev.upload_resident(w)
    out = np.zeros(m * rows, np.float32)
    assert dev.mat_mul_resident(res, zd.quant(zd.Q4_0), rows, k, m, x, out), dev.last_error()
    got = out.reshape(m, rows)
    rb = synth.row_bytes(synth.Q4_0, k)
    for r0, r1 in ((0, 256), (6000, 6128), (12160, 12288)):
        want = oracle.matmul_int(synth.Q4_0, w[r0 * rb:r1 * rb], k, r1 - r0, m, x)
        assert rel_l2(got[:, r0:r1], want) <= 1e-3, (r0, r1)
    dev.free_resident(res)


def test_gemm_unsupported_quants_fall_back(dev):
    rows, k, m = 32, 256, 4
    x = synth.activation(1, m * k)
    out = np.zeros(m * rows, np.float32)
    for qt in (synth.Q6_K, synth.F32, synth.F16):
        w = synth.weights(qt, rows, k, seed=2)
        assert not dev.mat_mul_batch(zd.quant(qt), w, rows, k, m, x, out)
    w = synth.weights(synth.Q4_0, rows, k, seed=2)
    assert not dev.mat_mul_batch(zd.quant(zd.Q4_0), w, rows, k, m, x[:-1].copy(), out)  # x length
    assert not dev.mat_mul_batch(zd.quant(zd.Q4_0), w, rows, k, m, x, out[:-1].copy())  # short out
    assert dev.mat_mul_batch(zd.quant(zd.Q4_0), w, rows, k, m, x, out)  # still healthy


def test_gemm_q4_k_c3_shape_rows_subset(dev):
    """A configs[3]-shaped Q4_K prefill (15360 x 3840, 96 tokens): row slices
    against the int oracle."""
    rows, k, m = 15360, 3840, 96
    _say("gemm q4_k 15360x3840 m=96")
    w = synth.weights(synth.Q4_K, rows, k, seed=0x5A4C4D03)
    x = synth.activation(0x5A4C4D0C, m * k)
    res = dev.upload_resident(w)
    out = np.zeros(m * rows, np.float32)
    assert dev.mat_mul_resident(res, zd.quant(zd.Q4_K), rows, k, m, x, out), dev.last_error()
    got = out.reshape(m, rows)
    rb = synth.row_bytes(synth.Q4_K, k)
    for r0, r1 in ((0, 96), (7000, 7064), (15296, 15360)):
        want = oracle.matmul_int(synth.Q4_K, w[r0 * rb:r1 * rb], k, r1 - r0, m, x)
        assert rel_l2(got[:, r0:r1], want) <= 1e-3, (r0, r1)
    dev.free_resident(res)


def test_resident_device_bytes_follow_the_conversions(dev):
    """The HBM a resident holds: its raw bytes after upload, the device layout
    after the first op (the token GEMVs of up to 4 tokens read it too), plus
    the GEMM tiled copy after a tiled GEMM (zlm_gpu_layout_bytes' estimate),
    and the layout again after zlm_gpu_release_gemm_tiles (a later GEMM
    rebuilds the copy)."""
    rows, k, m = 96, 4096, 9
    for qt, zq in GEMM_QUANTS:
        w = synth.weights(qt, rows, k, seed=77)
        x = synth.activation(78, m * k)
        res = dev.upload_resident(w)
        assert dev.resident_device_bytes(res) == w.size
        out = np.zeros(rows, np.float32)
        assert dev.mat_vec_resident(res, zd.quant(zq), rows, k, x[:k], out), dev.last_error()
        layout = zd.layout_bytes(zd.quant(zq), rows, k, False)
        assert dev.resident_device_bytes(res) == layout
        for few in (2, 4):
            outf = np.zeros(few * rows, np.float32)
            assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, few, x[:few * k], outf), dev.last_error()
            assert dev.resident_device_bytes(res) == layout
        outm = np.zeros(m * rows, np.float32)
        assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, m, x, outm), dev.last_error()
        assert dev.resident_device_bytes(res) == zd.layout_bytes(zd.quant(zq), rows, k, True) > layout
        assert dev.release_gemm_tiles(res)
        assert dev.resident_device_bytes(res) == layout
        again = np.zeros(m * rows, np.float32)
        assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, m, x, again), dev.last_error()
        np.testing.assert_array_equal(again, outm)
        dev.free_resident(res)
