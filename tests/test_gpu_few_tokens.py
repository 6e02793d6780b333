"""matMul at m = 2, 3 and 4: every token in one pass over the weights.

m = 2 (the fp path):

Two tokens run zlm's fp path (the oracle's matMulRows, form/single.zig:213-292:
the batched q4_0 / q8_0 forms, per-token production GEMVs for q4_1 / q4_k),
relative L2 <= 1e-3.  The device's two-token GEMV (zlm_gemv_<quant>_tok2_g<T>,
two-row wave tiles at the 4096- and 8192-float tiers, four rows for q4_k at
4096) loads every weight fragment once and sums it against both tokens' x
tiles; k beyond its 16384-float tier runs one GEMV per token.  Checked here:

* every tier (k <= 4096, 8192, 16384), a k that ends inside a step group
  (k = 256 and the q4_k k = 3840), row counts that end inside a wave tile
  (odd, and 65573 rows: many tiles per wave), and k = 20480 past the last
  tier, for the four matMul quants, resident and streamed;
* the route: the launch log shows one two-token launch up to k = 16384 and two
  GEMV launches past it;
* each token's row equals the one-token product to fp32 rounding (the same
  per-lane fragments, the same x, a different summation grouping).

m = 3, 4 (zlm's int path: q8 activations, exact integer block dots,
kernels/quantized.zig:49-55, :79-87, :111-123, :149-156 over the quantizer of
matvec/layout.zig:458-476): the int-path token GEMV (zlm_gemv_<quant>_q8tok4_
g<T>, two-row tiles for the nibble quants from 32768 rows) quantizes the
activations in its own prologue; m = 5..8 its eight-slot form for q4_1 at k
<= 4096 and q4_k there up to 8192 rows, the small-M GEMM otherwise (both
checked here at m = 5 and 8).  Against the oracle's int
path (orc_matmul_int) at relative L2 <= 1e-5, which one activation off by one
quantization unit would exceed, with activations that stress the quantizer
(a zero block, a block with one nonzero, values near rounding ties and a
block of tiny values; a denormal amax is left out: its 1/d overflows and the
float-to-int conversion of the infinite product is undefined in the reference
and the oracle alike); repeatable bit for bit; the route (one launch, no
tiled copy) up to k = 8192 and the quantizer + GEMM past it or from 5 tokens.
"""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import rel_l2
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu

QUANTS = [(synth.Q4_0, zd.Q4_0), (synth.Q8_0, zd.Q8_0), (synth.Q4_1, zd.Q4_1), (synth.Q4_K, zd.Q4_K)]
IDS = ["q4_0", "q8_0", "q4_1", "q4_k"]
SHAPES = [(1, 256), (67, 3840), (4097, 4096), (301, 6144), (300, 8192), (129, 12288), (64, 16384), (33, 20480),
          (65536 + 37, 3840)]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("qt,zq", QUANTS, ids=IDS)
@pytest.mark.parametrize("rows,k", SHAPES)
def test_two_tokens_match_oracle(dev, qt, zq, rows, k):
    be = synth.BLOCK_ELEMS[qt]
    k = (k + be - 1) // be * be
    _say(f"two tokens {IDS[QUANTS.index((qt, zq))]} rows={rows} k={k}")
    w = synth.weights(qt, rows, k, seed=rows + 7 * k)
    x = synth.activation(rows + 3, 2 * k)
    want = oracle.matmul_rows(qt, w, k, rows, 2, x)
    res = dev.upload_resident(w)
    assert res is not None, dev.last_error()
    try:
        out = np.full(2 * rows, np.nan, np.float32)
        assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, 2, x, out), dev.last_error()
        assert rel_l2(out.reshape(2, rows), want) <= 1e-3
        # streamed weights take the same route
        out2 = np.full(2 * rows, np.nan, np.float32)
        assert dev.mat_mul_batch(zd.quant(zq), w, rows, k, 2, x, out2), dev.last_error()
        np.testing.assert_array_equal(out2.view(np.uint32), out.view(np.uint32))
        # each token against its own one-token product
        for t in range(2):
            one = np.full(rows, np.nan, np.float32)
            assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, 1, x[t * k:(t + 1) * k].copy(), one)
            assert rel_l2(out[t * rows:(t + 1) * rows], one) <= 1e-5
    finally:
        dev.free_resident(res)


@pytest.mark.parametrize("k,launches", [(4096, ["gemv two tokens"]), (8192, ["gemv two tokens"]),
                                        (16384, ["gemv two tokens"]), (20480, ["gemv", "gemv"])])
def test_two_token_route(dev, k, launches):
    rows = 96
    w = synth.weights(synth.Q4_0, rows, k, seed=k)
    res = dev.upload_resident(w)
    x = dev.dev_malloc(2 * k * 4)
    out = dev.dev_malloc(2 * rows * 4)
    try:
        dev.dev_upload(x, synth.activation(5, 2 * k))
        assert dev.mat_mul_enqueue(res, zd.quant(zd.Q4_0), rows, k, 2, x, out), dev.last_error()  # layout
        dev.sync()
        assert dev.launch_log(True)
        assert dev.mat_mul_enqueue(res, zd.quant(zd.Q4_0), rows, k, 2, x, out), dev.last_error()
        dev.sync()
        log = dev.launch_log_read()
        assert [r["what"] for r in log] == launches
        if launches == ["gemv two tokens"]:
            # the workgroup grows with the x tier: 4, 8 or 16 waves
            assert log[0]["block"] == 64 * {4096: 4, 8192: 8, 16384: 16}[k]
    finally:
        dev.launch_log(False)
        dev.dev_free(x)
        dev.dev_free(out)
        dev.free_resident(res)


# (32768 + 37, 1024) and (32768 + 1, 5120): the two-row tiles of the nibble
# quants (from 32768 rows), ending inside a tile, at both x tiers; (129,
# 12288) and (65, 15360): the 16384-float tier of q4_1 / q4_k (the GEMM for
# the others)
INT_SHAPES = [(1, 256), (67, 3840), (4097, 4096), (300, 8192), (129, 12288), (65, 15360), (32768 + 37, 1024),
              (32768 + 1, 5120)]


def _stress_x(m, k, seed):
    """Activations whose q8 blocks hit the quantizer's edge cases."""
    x = synth.activation(seed, m * k).reshape(m, k).copy()
    x[0, 0:32] = 0.0                     # amax 0: d = 0, every q = 0
    x[0, 32:64] = 0.0
    x[0, 40] = -3.0                      # one nonzero: q = -127 there, 0 elsewhere
    d = 2.0 / 127.0                      # ties: v / d = n + 1/2 for a block with amax 2
    x[1, 64:96] = (np.arange(32) % 5 - 2 + 0.5) * d
    x[1, 64] = 2.0
    x[-1, 96:128] = np.float32(1e-30)    # a tiny (normal) amax
    return x.reshape(-1).astype(np.float32)


@pytest.mark.parametrize("qt,zq", QUANTS, ids=IDS)
@pytest.mark.parametrize("rows,k", INT_SHAPES)
@pytest.mark.parametrize("m", [3, 4, 5, 8])
def test_int_tokens_match_oracle(dev, qt, zq, rows, k, m):
    be = synth.BLOCK_ELEMS[qt]
    k = (k + be - 1) // be * be
    _say(f"int tokens {IDS[QUANTS.index((qt, zq))]} rows={rows} k={k} m={m}")
    w = synth.weights(qt, rows, k, seed=rows + 5 * k + m)
    x = _stress_x(m, k, rows + m)
    want = oracle.matmul_int(qt, w, k, rows, m, x)
    res = dev.upload_resident(w)
    assert res is not None, dev.last_error()
    try:
        out = np.full(m * rows, np.nan, np.float32)
        assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, m, x, out), dev.last_error()
        assert rel_l2(out.reshape(m, rows), want) <= 1e-5
        again = np.full(m * rows, np.nan, np.float32)
        assert dev.mat_mul_resident(res, zd.quant(zq), rows, k, m, x, again), dev.last_error()
        np.testing.assert_array_equal(again.view(np.uint32), out.view(np.uint32))
        # the reference's int-vs-fp bound (kernels/quantized_test.zig:61) against its fp matMulRows
        fp = oracle.matmul_rows(qt, w, k, rows, m, x)
        dq = np.abs(oracle.dequant(qt, w, rows * k).reshape(rows, k).astype(np.float64))
        mag = np.abs(x.reshape(m, k).astype(np.float64)) @ dq.T
        assert np.all(np.abs(out.reshape(m, rows) - fp) <= 0.02 * mag + 1e-6)
    finally:
        dev.free_resident(res)


@pytest.mark.parametrize("k,m,launches", [(4096, 3, ["gemv int tokens"]), (8192, 4, ["gemv int tokens"]),
                                          (12288, 3, ["quantize tiled", "gemm small"]),
                                          (4096, 5, ["quantize tiled", "gemm small"])])
def test_int_token_route(dev, k, m, launches):
    rows = 96
    w = synth.weights(synth.Q4_0, rows, k, seed=k + m)
    res = dev.upload_resident(w)
    x = dev.dev_malloc(m * k * 4)
    out = dev.dev_malloc(m * rows * 4)
    try:
        dev.dev_upload(x, synth.activation(7, m * k))
        assert dev.mat_mul_enqueue(res, zd.quant(zd.Q4_0), rows, k, m, x, out), dev.last_error()  # layouts
        dev.sync()
        tiled = dev.resident_device_bytes(res) > zd.layout_bytes(zd.quant(zd.Q4_0), rows, k, False)
        assert tiled == (launches != ["gemv int tokens"])
        assert dev.launch_log(True)
        assert dev.mat_mul_enqueue(res, zd.quant(zd.Q4_0), rows, k, m, x, out), dev.last_error()
        dev.sync()
        assert [r["what"] for r in dev.launch_log_read()] == launches
    finally:
        dev.launch_log(False)
        dev.dev_free(x)
        dev.dev_free(out)
        dev.free_resident(res)


@pytest.mark.parametrize("m", [2, 3, 4])
def test_token_routes_replay_from_a_graph(dev, m):
    """The token routes allocate nothing, so they capture into a HIP graph;
    replays (with eager work between them) equal the eager result bit for
    bit."""
    rows, k = 300, 4096
    w = synth.weights(synth.Q4_K, rows, k, seed=m)
    res = dev.upload_resident(w)
    x = dev.dev_malloc(m * k * 4)
    out = dev.dev_malloc(m * rows * 4)
    other = dev.dev_malloc(m * rows * 4)
    graph = None
    try:
        dev.dev_upload(x, synth.activation(9 + m, m * k))
        q = zd.quant(zd.Q4_K)
        assert dev.mat_mul_enqueue(res, q, rows, k, m, x, out), dev.last_error()
        eager = np.zeros(m * rows, np.float32)
        dev.dev_download(eager, out)
        assert dev.capture_begin(), dev.last_error()
        try:
            ok = dev.mat_mul_enqueue(res, q, rows, k, m, x, out)
        finally:
            graph = dev.capture_end()
        assert ok and graph is not None, dev.last_error()
        for rep in range(3):
            dev.dev_upload(out, np.full(m * rows, np.nan, np.float32))
            dev.graph_launch(graph, 1)
            got = np.zeros(m * rows, np.float32)
            dev.dev_download(got, out)
            np.testing.assert_array_equal(got.view(np.uint32), eager.view(np.uint32), err_msg=f"replay {rep}")
            assert dev.mat_mul_enqueue(res, q, rows, k, m, x, other), dev.last_error()  # eager work between
            dev.sync()
    finally:
        if graph is not None:
            dev.graph_destroy(graph)
        for p in (x, out, other):
            dev.dev_free(p)
        dev.free_resident(res)


@pytest.mark.parametrize("qt,rows,k,m,launches", [
    (zd.Q4_K, 96, 4096, 5, ["gemv int tokens"]), (zd.Q4_K, 96, 4096, 8, ["gemv int tokens"]),
    (zd.Q4_1, 12288, 4096, 8, ["gemv int tokens"]), (zd.Q4_K, 12288, 4096, 8, ["quantize tiled", "gemm small"]),
    (zd.Q4_K, 96, 8192, 5, ["quantize tiled", "gemm small"]), (zd.Q4_1, 96, 4096, 9, ["quantize tiled", "gemm small"]),
    (zd.Q4_0, 96, 4096, 8, ["quantize tiled", "gemm small"]),
    (zd.Q4_K, 96, 15360, 3, ["gemv int tokens"]), (zd.Q4_1, 96, 16384, 4, ["gemv int tokens"]),
    (zd.Q4_K, 96, 20480, 3, ["quantize tiled", "gemm small"]), (zd.Q4_0, 96, 12288, 4, ["quantize tiled", "gemm small"])],
    ids=lambda v: str(v) if not isinstance(v, list) else "")
def test_min_quant_token_routes(dev, qt, rows, k, m, launches):
    """The int-path token GEMV's extra routes for the quants whose small-M
    GEMM carries a min term: m = 5..8 the eight-slot form for q4_1 at k <=
    4096 and q4_k there up to 8192 rows; m = 3, 4 the 16384-float tier for
    both at k 8193-16384.  Everything else past 4 tokens, or past k = 8192
    for q4_0 / q8_0, runs the small-M GEMM."""
    sq = {zd.Q4_K: synth.Q4_K, zd.Q4_1: synth.Q4_1, zd.Q4_0: synth.Q4_0}[qt]
    w = synth.weights(sq, rows, k, seed=k + m + rows)
    res = dev.upload_resident(w)
    x = dev.dev_malloc(m * k * 4)
    out = dev.dev_malloc(m * rows * 4)
    try:
        dev.dev_upload(x, synth.activation(9, m * k))
        assert dev.mat_mul_enqueue(res, zd.quant(qt), rows, k, m, x, out), dev.last_error()  # layouts
        dev.sync()
        assert dev.launch_log(True)
        assert dev.mat_mul_enqueue(res, zd.quant(qt), rows, k, m, x, out), dev.last_error()
        dev.sync()
        assert [r["what"] for r in dev.launch_log_read()] == launches
    finally:
        dev.launch_log(False)
        dev.dev_free(x)
        dev.dev_free(out)
        dev.free_resident(res)

