"""matMul at m = 2: both tokens in one pass over the weights.

Two tokens run zlm's fp path (the oracle's matMulRows, form/single.zig:213-292:
the batched q4_0 / q8_0 forms, per-token production GEMVs for q4_1 / q4_k),
relative L2 <= 1e-3.  The device's two-token GEMV (zlm_gemv_<quant>_tok2_g<T>)
loads every weight fragment once and sums it against both tokens' x tiles;
k beyond its 16384-float tier runs one GEMV per token.  Checked here:

* every tier (k <= 4096, 8192, 16384), a k that ends inside a step group
  (k = 256 and the q4_k k = 3840), ragged row counts, and k = 20480 past the
  last tier, for the four matMul quants, resident and streamed;
* the route: the launch log shows one two-token launch up to k = 16384 and two
  GEMV launches past it;
* each token's row equals the one-token product to fp32 rounding (the same
  per-lane fragments, the same x, a different summation grouping).
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
SHAPES = [(1, 256), (67, 3840), (4097, 4096), (300, 8192), (129, 12288), (64, 16384), (33, 20480)]


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
