"""Pins the CPU oracle (oracle/zlm_oracle.c) before it is trusted as the checker.

Each check is chosen so a plausible restatement mistake fails it:
  * the reference's own known-answer tests (quant/root_test.zig, gguf/format.zig);
  * float64 closed forms of the codecs (a missing fma, a wrong nibble half, a
    wrong scale index or sign changes bits);
  * float64 brute force of every GEMV/GEMM form;
  * invariants the reference tests assert: row-split invariance
    (matvec/test.zig:273), lane-width agreement (matvec/test.zig:19-79),
    GEMM = repeated GEMV (fixtures.zig:90-124), int vs fp within
    0.02*sum|w*x| (kernels/quantized_test.zig:61);
  * textbook facts: round-half-away-from-zero, f16 decoding for all 65536 codes.
"""
import json
import os

import numpy as np
import pytest

import oracle
from tests.helpers import rel_l2
from zlm_amd import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")
TYPES = [synth.Q4_0, synth.Q8_0, synth.Q4_K, synth.Q6_K, synth.Q4_1, synth.F32, synth.F16, synth.BF16]


def f16b(v: float) -> list:
    return list(np.frombuffer(np.float16(v).tobytes(), np.uint8))


@pytest.fixture(scope="module")
def kats():
    with open(GOLDEN) as f:
        return json.load(f)


# ---- reference known-answer tests --------------------------------------------------

def test_tensor_byte_length_kats(kats):
    for case in kats["tensor_byte_length"]:
        assert oracle.tensor_byte_length(case["type"], case["n"]) == case["bytes"], case


def test_dequant_q8_0_kat(kats):
    c = kats["dequant_q8_0"]
    qs = np.array(c["qs"], np.int8)
    block = np.concatenate([f16b(c["d"]), qs.view(np.uint8)]).astype(np.uint8)
    out = oracle.dequant(synth.Q8_0, block, 32)
    np.testing.assert_allclose(out, np.array(c["expected"], np.float32), atol=1e-6)


def test_dequant_q4_0_kat(kats):
    c = kats["dequant_q4_0"]
    block = np.concatenate([f16b(c["d"]), c["nibbles"]]).astype(np.uint8)
    out = oracle.dequant(synth.Q4_0, block, 32)
    np.testing.assert_allclose(out, np.array(c["expected"], np.float32), atol=1e-6)


def test_dequant_q4_k_block_layout_kat(kats):
    c = kats["dequant_q4_k"]
    block = np.zeros(144, np.uint8)
    block[0:2] = f16b(c["d"])
    block[2:4] = f16b(c["dmin"])
    block[4:16] = c["scales"]
    block[16:] = [(i * 17 + 3) & 0xFF for i in range(128)]
    out = oracle.dequant(synth.Q4_K, block, 256)
    for idx, val in c["expected"].items():
        assert abs(out[int(idx)] - val) <= 1e-5, (idx, out[int(idx)], val)


def test_dequant_q6_k_block_layout_kat(kats):
    c = kats["dequant_q6_k"]
    block = np.zeros(210, np.uint8)
    block[208:210] = f16b(c["d"])
    block[:128] = c["ql_byte"]
    block[128:192] = c["qh_byte"]
    block[192:208] = np.uint8(c["scale"])
    out = oracle.dequant(synth.Q6_K, block, 256)
    np.testing.assert_allclose(out[:32], np.float32(c["expected_first32"]), atol=1e-5)


def test_dequant_partial_tail_and_rejects(kats):
    c = kats["dequant_q8_0_tail"]
    block = np.concatenate([f16b(c["d"]), np.full(32, c["q"], np.int8).view(np.uint8)]).astype(np.uint8)
    out = oracle.dequant(synth.Q8_0, block, c["n"])
    np.testing.assert_allclose(out, np.float32(c["expected"]), atol=1e-6)
    with pytest.raises(oracle.OracleError) as e:
        oracle.dequant(synth.Q6_K, np.zeros(210, np.uint8), 100)
    assert e.value.name == "ShapeMismatch"
    with pytest.raises(oracle.OracleError) as e:
        oracle.dequant(synth.Q4_0, np.zeros(17, np.uint8), 32)
    assert e.value.name == "TruncatedData"


def test_f16_decode_all_codes():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(c)) for c in codes[::7]], np.float32)
    w = want[::7]
    finite = np.isfinite(w)
    np.testing.assert_array_equal(got[finite].view(np.uint32), w[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(w)]))


def test_f16_encode_round_trip():
    rng = np.random.default_rng(0)
    v = rng.normal(size=5000).astype(np.float32) * np.float32(3.0)
    got = np.array([oracle.f32_to_f16(float(a)) for a in v], np.uint16)
    np.testing.assert_array_equal(got, v.astype(np.float16).view(np.uint16))


# ---- codec closed forms in float64 ---------------------------------------------------

def _scale_min_k4(scales: np.ndarray, j: int):
    """The GGUF Q4_K 6-bit scale/min packing, from the format description."""
    if j < 4:
        return scales[j] & 63, scales[j + 4] & 63
    return (scales[j + 4] & 0x0F) | ((scales[j - 4] >> 6) << 4), (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4)


@pytest.mark.parametrize("qt", TYPES)
def test_dequant_closed_form_f64(qt):
    """Decode by the format description, in float64, rounding to f32 exactly
    where the reference rounds (products of f32 scales; the Q4_K fma once).
    For Q4_K, q*d1 is always exact in f32 (a 4-bit q times d*sc, an 11-bit f16
    mantissa times a 6-bit scale), so the fused and the two-rounding forms of
    q*d1 - dmin*mn coincide; what this test pins is the layout and scales."""
    nblk = 40
    w = synth.weights(qt, nblk, synth.BLOCK_ELEMS[qt], seed=5).reshape(nblk, -1)
    got = oracle.dequant(qt, w.reshape(-1), nblk * synth.BLOCK_ELEMS[qt]).reshape(nblk, -1)
    f32 = np.float32
    for b in range(nblk):
        blk = w[b]
        if qt == synth.Q4_0:
            d = f32(blk[0:2].view(np.float16)[0])
            q = np.concatenate([blk[2:18] & 15, blk[2:18] >> 4]).astype(np.int64) - 8
            want = (q.astype(f32) * d).astype(f32)
        elif qt == synth.Q8_0:
            d = f32(blk[0:2].view(np.float16)[0])
            want = (blk[2:34].view(np.int8).astype(f32) * d).astype(f32)
        elif qt == synth.Q4_1:
            # standard.zig:138-148: q*d + m, the product and the sum rounded
            d = f32(blk[0:2].view(np.float16)[0])
            m = f32(blk[2:4].view(np.float16)[0])
            q = np.concatenate([blk[4:20] & 15, blk[4:20] >> 4]).astype(f32)
            want = ((q * d).astype(f32) + m).astype(f32)
        elif qt == synth.F32:
            want = blk.view(np.float32).copy()
        elif qt == synth.F16:
            want = blk.view(np.float16).astype(f32)
        elif qt == synth.BF16:
            want = (blk.view(np.uint16).astype(np.uint32) << 16).view(f32)
        elif qt == synth.Q4_K:
            d = f32(blk[0:2].view(np.float16)[0])
            dm = f32(blk[2:4].view(np.float16)[0])
            sc = blk[4:16]
            want = np.zeros(256, f32)
            for g in range(4):
                s1, m1 = _scale_min_k4(sc, 2 * g)
                s2, m2 = _scale_min_k4(sc, 2 * g + 1)
                d1, mm1 = f32(d * f32(s1)), f32(dm * f32(m1))
                d2, mm2 = f32(d * f32(s2)), f32(dm * f32(m2))
                qq = blk[16 + 32 * g: 48 + 32 * g].astype(np.float64)
                # fma: the exact q*d1 - m1 rounded once
                want[64 * g: 64 * g + 32] = ((qq % 16) * np.float64(d1) - np.float64(mm1)).astype(f32)
                want[64 * g + 32: 64 * g + 64] = ((qq // 16) * np.float64(d2) - np.float64(mm2)).astype(f32)
        else:
            d = f32(blk[208:210].view(np.float16)[0])
            ql, qh, sc = blk[0:128], blk[128:192], blk[192:208].view(np.int8)
            want = np.zeros(256, f32)
            for n in range(2):
                for l in range(32):
                    is_ = l // 16
                    h = qh[32 * n + l]
                    vals = [
                        (ql[64 * n + l] & 15) | ((h >> 0) & 3) << 4,
                        (ql[64 * n + l + 32] & 15) | ((h >> 2) & 3) << 4,
                        (ql[64 * n + l] >> 4) | ((h >> 4) & 3) << 4,
                        (ql[64 * n + l + 32] >> 4) | ((h >> 6) & 3) << 4,
                    ]
                    for t in range(4):
                        s = f32(d * f32(sc[8 * n + is_ + 2 * t]))
                        want[128 * n + 32 * t + l] = f32(f32(int(vals[t]) - 32) * s)
        np.testing.assert_array_equal(got[b].view(np.uint32), want.view(np.uint32), err_msg=f"block {b}")


# ---- GEMV / GEMM forms ---------------------------------------------------------------

def _f64_ref(qt, w, rows, k, x):
    dq = oracle.dequant(qt, w, rows * k).reshape(rows, k).astype(np.float64)
    return dq @ x.astype(np.float64), np.abs(dq) @ np.abs(x.astype(np.float64))


@pytest.mark.parametrize("qt", TYPES)
@pytest.mark.parametrize("lanes", [4, 8, 16])
def test_matvec_f64_brute_force(qt, lanes):
    rows, k = 96, 1024
    w = synth.weights(qt, rows, k, seed=lanes)
    x = synth.activation(3, k)
    y = oracle.matvec(qt, w, k, rows, x, lanes=lanes)
    ref, mag = _f64_ref(qt, w, rows, k, x)
    assert rel_l2(y, ref) < 1e-5
    assert np.all(np.abs(y - ref) <= 1e-5 * mag + 1e-6)


@pytest.mark.parametrize("qt", TYPES)
def test_lane_widths_agree_and_row_split_invariance(qt):
    rows, k = 50, 2048
    w = synth.weights(qt, rows, k, seed=31)
    x = synth.activation(32, k)
    y8 = oracle.matvec(qt, w, k, rows, x, lanes=8)
    _, mag = _f64_ref(qt, w, rows, k, x)
    for lanes in (4, 16):
        y = oracle.matvec(qt, w, k, rows, x, lanes=lanes)
        assert np.all(np.abs(y - y8) <= 1e-5 * mag)
    parts = np.zeros(rows, np.float32)
    for i in range(3):
        b, e = oracle.range_of(rows, 3, i)
        parts[b:e] = oracle.matvec(qt, w, k, rows, x, begin=b, end=e)[b:e]
    np.testing.assert_array_equal(parts, y8)


def test_lm_head_rows_equals_production():
    for qt in (synth.Q8_0, synth.Q6_K):
        rows, k = 40, 512
        w = synth.weights(qt, rows, k, seed=2)
        x = synth.activation(2, k)
        np.testing.assert_array_equal(oracle.lm_head_rows(qt, w, k, rows, x), oracle.matvec(qt, w, k, rows, x))


def test_matvec_shape_errors():
    w = synth.weights(synth.Q4_0, 4, 64, seed=1)
    x = synth.activation(1, 64)
    with pytest.raises(oracle.OracleError):
        oracle.matvec(synth.Q4_0, w, 64, 5, x)  # truncated
    with pytest.raises(oracle.OracleError):
        oracle.matvec(synth.Q4_0, w, 64, 4, x, begin=3, end=2)  # range
    with pytest.raises(oracle.OracleError):
        oracle.matvec(synth.Q4_K, w, 64, 1, x)  # k % 256


# ---- activation quantizer and int path -----------------------------------------------

def test_quantizer_round_half_away_kat():
    x = np.zeros(64, np.float32)
    x[0] = 127.0  # amax = 127 -> d = 1, inv = 1: q = round(v)
    x[1:9] = [2.5, -2.5, 0.5, -0.5, 1.49, -1.5, 126.5, -127.0]
    qx, dx, sums = oracle.quantize_act_q8(x)
    assert dx[0] == np.float32(1.0) and dx[1] == 0.0
    assert list(qx[:9]) == [127, 3, -3, 1, -1, 1, -2, 127, -127]
    assert sums[0] == int(qx[:32].astype(np.int64).sum()) and sums[1] == 0
    assert np.all(qx[32:] == 0)


def test_quantizer_invariants():
    x = synth.activation(77, 32 * 500) * np.float32(3.0)
    qx, dx, sums = oracle.quantize_act_q8(x)
    xb = x.reshape(-1, 32)
    qb = qx.reshape(-1, 32).astype(np.int64)
    amax = np.abs(xb).max(axis=1)
    np.testing.assert_array_equal(dx, (amax / np.float32(127.0)).astype(np.float32))
    assert np.all(np.abs(qb) <= 127)
    assert np.all(np.abs(qb[np.arange(len(xb)), np.abs(xb).argmax(axis=1)]) == 127)
    err = np.abs(qb * dx[:, None].astype(np.float64) - xb)
    assert np.all(err <= dx[:, None] * 0.5 * (1 + 1e-5) + 1e-12)
    np.testing.assert_array_equal(sums, qb.sum(axis=1))


@pytest.mark.parametrize("qt", [synth.Q4_0, synth.Q8_0, synth.Q4_K, synth.Q4_1])
def test_int_path_exact_reconstruction_and_fp_bound(qt):
    rows, k = 64, 1024
    w = synth.weights(qt, rows, k, seed=12)
    x = synth.activation(13, k)
    y_int = oracle.matvec_int(qt, w, k, rows, x)
    qx, dx, _ = oracle.quantize_act_q8(x)
    # float64 reconstruction: dequantized weight times the q8 activation exactly
    xq = qx.astype(np.float64) * np.repeat(dx.astype(np.float64), 32)
    dq = oracle.dequant(qt, w, rows * k).reshape(rows, k).astype(np.float64)
    ref = dq @ xq
    assert rel_l2(y_int, ref) < 1e-5
    # the reference's int-vs-fp bound (kernels/quantized_test.zig:61)
    y_fp = oracle.matvec(qt, w, k, rows, x)
    mag = np.abs(dq) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y_int - y_fp) <= 0.02 * mag)


def test_matmul_equals_repeated_matvec():
    """GEMM = repeated GEMV within 1e-5 (reference matvec/fixtures.zig:90-124)."""
    for qt in (synth.Q4_0, synth.Q8_0, synth.Q4_K, synth.Q6_K):
        rows, k = 24, 512
        w = synth.weights(qt, rows, k, seed=4)
        for m in (2, 5, 33):
            x = synth.activation(m, m * k)
            got = oracle.matmul_rows(qt, w, k, rows, m, x)
            for t in range(m):
                want = oracle.matvec(qt, w, k, rows, x[t * k:(t + 1) * k])
                np.testing.assert_allclose(got[t], want, atol=1e-5 * max(1.0, float(np.abs(want).max())))
            ref = oracle.dequant(qt, w, rows * k).reshape(rows, k).astype(np.float64) @ \
                x.reshape(m, k).astype(np.float64).T
            assert rel_l2(got, ref.T) < 1e-5


def test_matmul_int_is_per_token_int_gemv():
    qt, rows, k, m = synth.Q4_0, 32, 512, 6
    w = synth.weights(qt, rows, k, seed=6)
    x = synth.activation(6, m * k)
    got = oracle.matmul_int(qt, w, k, rows, m, x)
    for t in range(m):
        np.testing.assert_array_equal(got[t], oracle.matvec_int(qt, w, k, rows, x[t * k:(t + 1) * k]))


# ---- fused gate_up and activations ----------------------------------------------------

def test_activation_closed_forms():
    for g in (-9.0, -1.25, 0.0, 0.5, 3.0, 12.0):
        u = 1.75
        silu = g / (1.0 + np.exp(-g)) * u
        gelu = 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))) * u
        assert abs(oracle.act_apply(0, g, u) - silu) <= 1e-6 * max(1.0, abs(silu))
        assert abs(oracle.act_apply(1, g, u) - gelu) <= 1e-6 * max(1.0, abs(gelu))


def test_gate_up_is_two_gemvs_and_act():
    qt, rows, k = synth.Q4_0, 48, 512
    wg = synth.weights(qt, rows, k, seed=1)
    wu = synth.weights(qt, rows, k, seed=2)
    x = synth.activation(3, k)
    g = oracle.matvec(qt, wg, k, rows, x)
    u = oracle.matvec(qt, wu, k, rows, x)
    for act in (0, 1):
        got = oracle.gate_up(qt, wg, wu, k, rows, x, act)
        want = np.array([oracle.act_apply(act, float(a), float(b)) for a, b in zip(g, u)], np.float32)
        np.testing.assert_array_equal(got, want)


# ---- the CPU-baseline row split ------------------------------------------------------

def test_range_of_ceil_first():
    assert [oracle.range_of(10, 3, i) for i in range(3)] == [(0, 4), (4, 7), (7, 10)]
    assert [oracle.range_of(2, 4, i) for i in range(4)] == [(0, 1), (1, 2), (2, 2), (2, 2)]
    assert oracle.range_of(5, 2, 7) == (5, 5)
    for total in (0, 1, 17, 4096):
        for parts in (1, 3, 8, 16):
            spans = [oracle.range_of(total, parts, i) for i in range(parts)]
            assert spans[0][0] == 0 and spans[-1][1] == total
            assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
            sizes = [e - b for b, e in spans]
            assert sizes == sorted(sizes, reverse=True) and sizes[0] - sizes[-1] <= 1


def test_threaded_timer_runs():
    qt, rows, k = synth.Q8_0, 256, 1024
    w = synth.weights(qt, rows, k, seed=1)
    x = synth.activation(1, k)
    assert oracle.time_matvec(qt, w, k, rows, x, threads=4, reps=2) > 0


# ---- the speed-faithful sweep (oracle/zlm_cpu_sweep.c) -------------------------------
# The CPU baseline runs zlm's production sweep the way zlm's ReleaseFast build
# does (compile-time lanes, per-type row loops, vector dequant).  It must be
# the oracle's arithmetic exactly: bit for bit at the same lane count, for
# every type, on odd row ranges and the boundary cases the sweeps share.

FAST_LANES = [L for L in (8, 16) if oracle.fast_native_lanes() >= L]


def _bits(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.uint32)


@pytest.mark.skipif(not FAST_LANES, reason="host has neither AVX2 nor AVX-512")
@pytest.mark.parametrize("lanes", FAST_LANES)
@pytest.mark.parametrize("qt", TYPES)
@pytest.mark.parametrize("rows,k", [(37, 256), (130, 4096), (9, 12288), (5, 3840)])
def test_fast_sweep_is_the_oracle_bit_for_bit(qt, lanes, rows, k):
    if k % synth.BLOCK_ELEMS[qt]:
        pytest.skip("k not whole blocks")
    w = synth.weights(qt, rows, k, seed=rows * 7 + k + qt)
    x = synth.activation(rows + qt, k)
    want = oracle.matvec(qt, w, k, rows, x, lanes=lanes)
    np.testing.assert_array_equal(_bits(oracle.fast_matvec(qt, w, k, rows, x, lanes=lanes)), _bits(want))
    # a row range leaves the other rows alone
    part = oracle.fast_matvec(qt, w, k, rows, x, lanes=lanes, begin=rows // 3, end=rows - 1)
    np.testing.assert_array_equal(_bits(part[rows // 3:rows - 1]), _bits(want[rows // 3:rows - 1]))
    assert not part[:rows // 3].any() and part[rows - 1] == 0


@pytest.mark.skipif(not FAST_LANES, reason="host has neither AVX2 nor AVX-512")
@pytest.mark.parametrize("lanes", FAST_LANES)
def test_fast_sweep_special_values(lanes):
    """Zero, signed-zero, extreme and subnormal scales and activations: the
    paths where a reordered or contracted operation would show."""
    rows, k = 16, 512
    for qt in TYPES:
        w = synth.weights(qt, rows, k, seed=3).copy()
        x = synth.activation(4, k).copy()
        x[::7] = 0.0
        x[1::11] = -0.0
        x[2::13] = 3.0e38 if qt in (synth.F32,) else 6.0e4
        x[3::17] = 1e-40
        if qt in (synth.Q4_0, synth.Q8_0, synth.Q4_1):
            bb = synth.BLOCK_BYTES[qt]
            w[0::bb * 3] = 0x00  # some scales -> zero / subnormal f16
            w[1::bb * 3] = 0x80  # negative zero
        want = oracle.matvec(qt, w, k, rows, x, lanes=lanes)
        got = oracle.fast_matvec(qt, w, k, rows, x, lanes=lanes)
        np.testing.assert_array_equal(_bits(got), _bits(want), err_msg=str(qt))


@pytest.mark.skipif(not FAST_LANES, reason="host has neither AVX2 nor AVX-512")
@pytest.mark.parametrize("lanes", FAST_LANES)
@pytest.mark.parametrize("qt", [synth.Q4_0, synth.Q8_0])
def test_fast_int_sweep_is_the_oracle_bit_for_bit(qt, lanes):
    rows, k = 71, 4096
    w = synth.weights(qt, rows, k, seed=11 + qt)
    x = synth.activation(12 + qt, k)
    np.testing.assert_array_equal(_bits(oracle.fast_matvec_int(qt, w, k, rows, x, lanes=lanes)),
                                  _bits(oracle.matvec_int(qt, w, k, rows, x, lanes=lanes)))


@pytest.mark.skipif(not FAST_LANES, reason="host has neither AVX2 nor AVX-512")
def test_pool_splits_rows_like_the_single_thread_sweep():
    """The pinned pool (rangeOf parts, caller runs part 0) writes every row once,
    with the single-thread result; the int path over several tokens too."""
    rows, k = 1001, 1024
    for qt in (synth.Q8_0, synth.Q4_K, synth.BF16):
        w = synth.weights(qt, rows, k, seed=21)
        x = synth.activation(22, k)
        out = np.full(rows, np.nan, np.float32)
        assert oracle.fast_time_matvec(qt, w, k, rows, x, threads=3, reps=2, out=out) > 0
        np.testing.assert_array_equal(_bits(out), _bits(oracle.matvec(qt, w, k, rows, x,
                                                                      lanes=oracle.fast_native_lanes())))
    assert oracle.pool_threads() == min(3, max(1, len(oracle.physical_cores())))
    m = 3
    w = synth.weights(synth.Q4_0, rows, k, seed=23)
    x = synth.activation(24, m * k)
    out = np.full(m * rows, np.nan, np.float32)
    assert oracle.fast_time_matmul_int(synth.Q4_0, w, k, rows, m, x, threads=2, reps=1, out=out) > 0
    np.testing.assert_array_equal(_bits(out), _bits(oracle.matmul_int(synth.Q4_0, w, k, rows, m, x,
                                                                       lanes=oracle.fast_native_lanes())))


def test_physical_cores_are_distinct_and_allowed():
    cores = oracle.physical_cores()
    assert cores and len(set(cores)) == len(cores)
    assert set(cores) <= os.sched_getaffinity(0)


@pytest.mark.skipif(not FAST_LANES, reason="host has neither AVX2 nor AVX-512")
def test_pooled_matvec_is_the_oracle():
    """The pooled GEMV the model-sized decode check uses: the oracle's result
    bit for bit at the oracle's default lanes."""
    for qt in (synth.Q4_0, synth.Q8_0):
        w = synth.weights(qt, 777, 2048, seed=51)
        x = synth.activation(52, 2048)
        np.testing.assert_array_equal(_bits(oracle.pooled_matvec(qt, w, 2048, 777, x, threads=4)),
                                      _bits(oracle.matvec(qt, w, 2048, 777, x)))
