"""Resident ops over a row prefix of a larger resident.

zlm's executor runs a resident op over `rows = min(row_count, m)` of a tensor
(reference runtime/executor.zig:246, :794), and the tuner's split probe runs
the async GEMV over rows [0, m/2) of an m-row resident while CPU threads take
the rest (tuner/calibrate.zig:778-834).  Every resident op here runs over rows
[0, r) of a resident holding more rows, against the oracle on those rows
(relative L2 <= 1e-3 for the fp GEMVs; the int path's 1e-5 for matMul past two
tokens), and leaves the output past r untouched:

* matVecResident and matVecResidentAsync + waitResident, all eight GEMV types;
* matVecResidentBatch over prefixes of two residents;
* the fused gate_up and the MLP ops (a prefix of the gate/up rows; a prefix
  of the down rows);
* matMulResident for the four GEMM types at m = 1, 2 (the fp GEMV and the
  two-token GEMV), 3 (the int-path token GEMV), 5 and 40 (the small-M kernel
  over one and two token tiles; test_gpu_gemm.py runs the tiled GEMM over a
  row prefix).
"""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import rel_l2
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu

TYPES = [synth.Q4_0, synth.Q8_0, synth.Q4_K, synth.Q6_K, synth.Q4_1, synth.F32, synth.F16, synth.BF16]
NAMES = synth.TYPE_NAMES
TOTAL = 300  # rows the resident holds


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _prefix(qt, w, k, r):
    return w[:r * synth.row_bytes(qt, k)]


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("k", [1024, 4096])
def test_gemv_over_a_row_prefix(dev, qt, k):
    w = synth.weights(qt, TOTAL, k, seed=11 * k + qt)
    x = synth.activation(k + qt, k)
    res = dev.upload_resident(w)
    assert res is not None, dev.last_error()
    q = zd.quant(qt)
    try:
        for r in (1, 37, TOTAL // 2, TOTAL - 1, TOTAL):
            _say(f"row prefix {NAMES[qt]} k={k} rows={r} of {TOTAL}")
            want = oracle.matvec(qt, _prefix(qt, w, k, r), k, r, x)
            out = np.full(TOTAL, -7.0, np.float32)
            assert dev.mat_vec_resident(res, q, r, k, x, out), dev.last_error()
            assert rel_l2(out[:r], want) <= 1e-3
            assert np.all(out[r:] == -7.0)
            h = dev.mat_vec_resident_async(res, q, r, k, x)
            assert h is not None, dev.last_error()
            out2 = np.full(TOTAL, -7.0, np.float32)
            assert dev.wait_resident(h, out2, r), dev.last_error()
            np.testing.assert_array_equal(out2[:r].view(np.uint32), out[:r].view(np.uint32))
            assert np.all(out2[r:] == -7.0)
        # a prefix longer than the resident is refused
        assert not dev.mat_vec_resident(res, q, TOTAL + 1, k, x, np.zeros(TOTAL + 1, np.float32))
    finally:
        dev.free_resident(res)


@pytest.mark.parametrize("qt", [synth.Q4_0, synth.Q8_0, synth.Q4_K], ids=lambda t: NAMES[t])
def test_batch_over_row_prefixes(dev, qt):
    k = 1024
    wa = synth.weights(qt, TOTAL, k, seed=21)
    wb = synth.weights(qt, TOTAL, k, seed=22)
    x = synth.activation(23, k)
    ra, rb = dev.upload_resident(wa), dev.upload_resident(wb)
    try:
        oa, ob = np.zeros(100, np.float32), np.zeros(233, np.float32)
        ops = [zd.ResidentOp(ra, zd.quant(qt), 100, oa), zd.ResidentOp(rb, zd.quant(qt), 233, ob)]
        assert dev.mat_vec_resident_batch(k, x, ops), dev.last_error()
        assert rel_l2(oa, oracle.matvec(qt, _prefix(qt, wa, k, 100), k, 100, x)) <= 1e-3
        assert rel_l2(ob, oracle.matvec(qt, _prefix(qt, wb, k, 233), k, 233, x)) <= 1e-3
    finally:
        dev.free_resident(ra)
        dev.free_resident(rb)


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: NAMES[t])
def test_fused_ops_over_row_prefixes(dev, qt):
    k, ffn, hidden = 1024, 512, 256
    wg = synth.weights(qt, ffn, k, seed=31)
    wu = synth.weights(qt, ffn, k, seed=32)
    x = synth.activation(33, k)
    rg, ru = dev.upload_resident(wg), dev.upload_resident(wu)
    q = zd.quant(qt)
    try:
        for r in (1, 99, 511):
            _say(f"gate_up prefix {NAMES[qt]} rows={r} of {ffn}")
            want = oracle.gate_up(qt, _prefix(qt, wg, k, r), _prefix(qt, wu, k, r), k, r, x, zd.SILU)
            h = dev.mat_vec_gate_up_resident_burst_async(rg, ru, q, r, k, x, zd.SILU, zd.PLAIN, True)
            out = np.full(ffn, -7.0, np.float32)
            assert h is not None and dev.wait_resident(h, out, r), dev.last_error()
            assert rel_l2(out[:r], want) <= 1e-3 and np.all(out[r:] == -7.0)
        # the MLP with a down resident of more rows than the op's `rows`
        wd = synth.weights(qt, hidden, ffn, seed=34)
        rd = dev.upload_resident(wd)
        mid = oracle.gate_up(qt, wg, wu, k, ffn, x, zd.SILU)
        for r in (3, 200):
            h = dev.mat_vec_mlp_resident_burst_async(rg, ru, rd, q, r, k, ffn, x, zd.SILU, zd.PLAIN, True)
            out = np.full(hidden, -7.0, np.float32)
            assert h is not None and dev.wait_resident(h, out, r), dev.last_error()
            want = oracle.matvec(qt, _prefix(qt, wd, ffn, r), ffn, r, mid)
            assert rel_l2(out[:r], want) <= 1e-3 and np.all(out[r:] == -7.0)
        dev.free_resident(rd)
    finally:
        dev.free_resident(rg)
        dev.free_resident(ru)


GEMM_TYPES = [synth.Q4_0, synth.Q8_0, synth.Q4_1, synth.Q4_K]


@pytest.mark.parametrize("qt", GEMM_TYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 40])
def test_matmul_over_a_row_prefix(dev, qt, m):
    k = 1024
    w = synth.weights(qt, TOTAL, k, seed=41 + m)
    x = synth.activation(42 + m, m * k)
    res = dev.upload_resident(w)
    try:
        for r in (7, 129, TOTAL - 1):
            _say(f"matMul prefix {NAMES[qt]} m={m} rows={r} of {TOTAL}")
            wp = _prefix(qt, w, k, r)
            want = oracle.matmul_rows(qt, wp, k, r, m, x) if m <= 2 else oracle.matmul_int(qt, wp, k, r, m, x)
            out = np.full(m * r, np.nan, np.float32)
            assert dev.mat_mul_resident(res, zd.quant(qt), r, k, m, x, out), dev.last_error()
            assert rel_l2(out.reshape(m, r), want) <= (1e-3 if m <= 2 else 1e-5)
    finally:
        dev.free_resident(res)
