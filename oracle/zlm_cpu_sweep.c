/*
 * zlm_cpu_sweep.c -- zlm's production CPU sweep, written to run at zlm's speed.
 *
 * TEST INFRASTRUCTURE ONLY: the CPU baseline bench.py times beside the GPU
 * (and the tests that pin it).  Nothing in zlm_amd/ links or calls this file.
 *
 * zlm_oracle.c restates zlm's kernels with a runtime lane count and the quant
 * type switched per block: the right arithmetic at a fraction of the speed.
 * This file computes exactly the same operations in the same order -- its
 * outputs are bit-identical to orc_matvec / orc_matvec_int at the same lane
 * count, which tests/test_oracle.py checks for every type -- but the way zlm's
 * ReleaseFast build runs them:
 *   - the lane width is a compile-time constant: the file is compiled twice,
 *     SW_LANES=8 with AVX2+FMA+F16C and SW_LANES=16 with AVX-512, the two
 *     widths `simd.native` picks on AVX2 and AVX-512 hosts
 *     (kernels/simd.zig:30-41); zlm_cpu_pool.c picks the build for the host;
 *   - every quant type has its own row loop, so the type is resolved once per
 *     call, as the comptime-specialised sweep is (form/single.zig:29-140);
 *   - blocks are expanded and multiplied with integer and float vector
 *     instructions (layout.zig:27-51 q4_0Expand/q4_0BlockVec, :99-111
 *     q8_0BlockVec, :164-180, :215-342, :392-452), f16 scales through F16C;
 *   - `simd.fma` is a vector FMA, every other `a*b + c` two rounded vector
 *     operations (-ffp-contract=off), `@reduce(.Add)` an in-order lane sum.
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "zlm_oracle.h"

#if SW_LANES == 8
typedef __m256 V;
#define VZERO() _mm256_setzero_ps()
#define VLOAD(p) _mm256_loadu_ps(p)
#define VSTORE(p, v) _mm256_storeu_ps(p, v)
#define VSET1(s) _mm256_set1_ps(s)
#define VFMA(a, b, c) _mm256_fmadd_ps(a, b, c)
#define VMUL(a, b) _mm256_mul_ps(a, b)
#define VADD(a, b) _mm256_add_ps(a, b)
#define SW(name) name##_l8
#elif SW_LANES == 16
typedef __m512 V;
#define VZERO() _mm512_setzero_ps()
#define VLOAD(p) _mm512_loadu_ps(p)
#define VSTORE(p, v) _mm512_storeu_ps(p, v)
#define VSET1(s) _mm512_set1_ps(s)
#define VFMA(a, b, c) _mm512_fmadd_ps(a, b, c)
#define VMUL(a, b) _mm512_mul_ps(a, b)
#define VADD(a, b) _mm512_add_ps(a, b)
#define SW(name) name##_l16
#else
#error "SW_LANES must be 8 or 16"
#endif

#define INL static inline __attribute__((always_inline))

INL float f16(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return _cvtsh_ss(h); /* exact widening, as @floatCast(f16 -> f32) */
}

/* `@reduce(.Add, v)`: the in-order lane sum. */
INL float vsum(V v) {
    float t[SW_LANES];
    VSTORE(t, v);
    float r = t[0];
    for (int j = 1; j < SW_LANES; j++) r += t[j];
    return r;
}

/* int8 / uint8 lanes of a 128-bit register to f32 lanes: 8 (the low half) or 16. */
#if SW_LANES == 8
INL V cvt_i8(__m128i b) { return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b)); }
INL V cvt_u8(__m128i b) { return _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(b)); }
#else
INL V cvt_i8(__m128i b) { return _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(b)); }
INL V cvt_u8(__m128i b) { return _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(b)); }
#endif

/* sum_j q[j]*x[j] over a block's 32 elements, `lanes` at a time from a zero
 * accumulator with fma (q4_0BlockVec / q8_0BlockVec / q4_1BlockVecLanes);
 * lo holds elements 0..15, hi 16..31 as int8 (sgn) or uint8 lanes. */
INL V block_vec(__m128i lo, __m128i hi, const float *xb, int sgn) {
    V bv = VZERO();
#if SW_LANES == 8
    const __m128i parts[4] = {lo, _mm_srli_si128(lo, 8), hi, _mm_srli_si128(hi, 8)};
    for (int s = 0; s < 4; s++) bv = VFMA(sgn ? cvt_i8(parts[s]) : cvt_u8(parts[s]), VLOAD(xb + 8 * s), bv);
#else
    bv = VFMA(sgn ? cvt_i8(lo) : cvt_u8(lo), VLOAD(xb), bv);
    bv = VFMA(sgn ? cvt_i8(hi) : cvt_u8(hi), VLOAD(xb + 16), bv);
#endif
    return bv;
}

/* Q4_0.fpBlock (kernels/quantized.zig:42-47): acc = fma(d, blockvec(nib-8), acc). */
static void rows_q4_0(const uint8_t *w, size_t nb, const float *x, float *out, size_t begin, size_t end) {
    const __m128i m4 = _mm_set1_epi8(0x0F), b8 = _mm_set1_epi8(8);
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * nb * 18;
        V acc = VZERO();
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * 18;
            const __m128i bytes = _mm_loadu_si128((const __m128i *)(b + 2));
            const __m128i lo = _mm_sub_epi8(_mm_and_si128(bytes, m4), b8);
            const __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(bytes, 4), m4), b8);
            acc = VFMA(VSET1(f16(b)), block_vec(lo, hi, x + rb * 32, 1), acc);
        }
        out[i] = vsum(acc) + 0.0f;
    }
}

/* Q8_0.fpBlock (quantized.zig:142-147). */
static void rows_q8_0(const uint8_t *w, size_t nb, const float *x, float *out, size_t begin, size_t end) {
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * nb * 34;
        V acc = VZERO();
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * 34;
            const __m128i lo = _mm_loadu_si128((const __m128i *)(b + 2));
            const __m128i hi = _mm_loadu_si128((const __m128i *)(b + 18));
            acc = VFMA(VSET1(f16(b)), block_vec(lo, hi, x + rb * 32, 1), acc);
        }
        out[i] = vsum(acc) + 0.0f;
    }
}

/* Q4_1.fpBlock (quantized.zig:71-77): acc = fma(d, blockvec(nib), acc); corr += m * xsum. */
static void rows_q4_1(const uint8_t *w, size_t nb, const float *x, const float *xsum, float *out, size_t begin,
                      size_t end) {
    const __m128i m4 = _mm_set1_epi8(0x0F);
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * nb * 20;
        V acc = VZERO();
        float corr = 0.0f;
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * 20;
            const __m128i bytes = _mm_loadu_si128((const __m128i *)(b + 4));
            const __m128i lo = _mm_and_si128(bytes, m4);
            const __m128i hi = _mm_and_si128(_mm_srli_epi16(bytes, 4), m4);
            acc = VFMA(VSET1(f16(b)), block_vec(lo, hi, x + rb * 32, 0), acc);
            corr += f16(b + 2) * xsum[rb];
        }
        out[i] = vsum(acc) + corr;
    }
}

/* q4KNibVec (layout.zig:215-261): the lanes-wide partial of 32 nibbles (bytes
 * of `q`, already masked) times x: products rounded, then summed pairwise. */
INL V q4k_nibvec(__m256i q, const float *xb) {
    const __m128i q0 = _mm256_castsi256_si128(q), q1 = _mm256_extracti128_si256(q, 1);
#if SW_LANES == 8
    const V p0 = VMUL(cvt_u8(q0), VLOAD(xb)), p1 = VMUL(cvt_u8(_mm_srli_si128(q0, 8)), VLOAD(xb + 8));
    const V p2 = VMUL(cvt_u8(q1), VLOAD(xb + 16)), p3 = VMUL(cvt_u8(_mm_srli_si128(q1, 8)), VLOAD(xb + 24));
    return VADD(VADD(p0, p1), VADD(p2, p3));
#else
    return VADD(VMUL(cvt_u8(q0), VLOAD(xb)), VMUL(cvt_u8(q1), VLOAD(xb + 16)));
#endif
}

/* Q4_K.fpBlock (quantized.zig:105-109) over q4KBlockAccumGen (layout.zig:309-342). */
static void rows_q4_k(const uint8_t *w, size_t nb, const float *x, const float *xsum, float *out, size_t begin,
                      size_t end) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * nb * 144;
        V acc = VZERO();
        float corr = 0.0f;
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * 144;
            const float d = f16(b), dmin = f16(b + 2);
            const uint8_t *sc = b + 4;
            const float *xb = x + rb * 256, *xs = xsum + rb * 8;
            float msum = 0.0f;
            for (int g = 0; g < 4; g++) {
                uint8_t s1, m1, s2, m2;
                orc_get_scale_min_k4(2 * g, sc, &s1, &m1);
                orc_get_scale_min_k4(2 * g + 1, sc, &s2, &m2);
                const __m256i qs = _mm256_loadu_si256((const __m256i *)(b + 16 + 32 * g));
                const V v1 = q4k_nibvec(_mm256_and_si256(qs, m4), xb + 64 * g);
                acc = VFMA(VSET1(d * (float)s1), v1, acc);
                const V v2 = q4k_nibvec(_mm256_and_si256(_mm256_srli_epi16(qs, 4), m4), xb + 64 * g + 32);
                acc = VFMA(VSET1(d * (float)s2), v2, acc);
                msum += (dmin * (float)m1) * xs[2 * g] + (dmin * (float)m2) * xs[2 * g + 1];
            }
            corr -= msum;
        }
        out[i] = vsum(acc) + corr;
    }
}

/* Sixteen f32 lanes: one zmm, or two ymm on the AVX2 build (q6KBlockDot is
 * 16 lanes wide whatever the native width, layout.zig:414-452). */
#if SW_LANES == 16
typedef __m512 V16;
INL V16 v16_zero(void) { return _mm512_setzero_ps(); }
INL V16 v16_q6(__m128i q, const float *xb) {
    return _mm512_mul_ps(_mm512_sub_ps(_mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(q)), _mm512_set1_ps(32.0f)),
                         _mm512_loadu_ps(xb));
}
INL V16 v16_fma(float s, V16 v, V16 acc) { return _mm512_fmadd_ps(_mm512_set1_ps(s), v, acc); }
INL void v16_store(float *t, V16 v) { _mm512_storeu_ps(t, v); }
#else
typedef struct {
    __m256 a, b;
} V16;
INL V16 v16_zero(void) { return (V16){_mm256_setzero_ps(), _mm256_setzero_ps()}; }
INL V16 v16_q6(__m128i q, const float *xb) {
    const __m256 c = _mm256_set1_ps(32.0f);
    const __m256 a = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(q));
    const __m256 b = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(q, 8)));
    return (V16){_mm256_mul_ps(_mm256_sub_ps(a, c), _mm256_loadu_ps(xb)),
                 _mm256_mul_ps(_mm256_sub_ps(b, c), _mm256_loadu_ps(xb + 8))};
}
INL V16 v16_fma(float s, V16 v, V16 acc) {
    const __m256 sv = _mm256_set1_ps(s);
    return (V16){_mm256_fmadd_ps(sv, v.a, acc.a), _mm256_fmadd_ps(sv, v.b, acc.b)};
}
INL void v16_store(float *t, V16 v) {
    _mm256_storeu_ps(t, v.a);
    _mm256_storeu_ps(t + 8, v.b);
}
#endif

/* q6KChunkVec16 (layout.zig:392-412): 16 six-bit quants, low or high nibble
 * of ql with two bits of qh from `shift`, as uint8 lanes. */
INL __m128i q6_quants(const uint8_t *ql, const uint8_t *qh, int hi, int shift) {
    const __m128i m4 = _mm_set1_epi8(0x0F), m2 = _mm_set1_epi8(3);
    __m128i l = _mm_loadu_si128((const __m128i *)ql);
    l = hi ? _mm_and_si128(_mm_srli_epi16(l, 4), m4) : _mm_and_si128(l, m4);
    const __m128i h = _mm_and_si128(_mm_srl_epi16(_mm_loadu_si128((const __m128i *)qh), _mm_cvtsi32_si128(shift)), m2);
    return _mm_or_si128(l, _mm_slli_epi16(h, 4));
}

/* q6KBlockDot (layout.zig:414-452): 16-wide fma accumulation, one reduce per
 * block, added to the row's correction (the production sweep's Q6_K body). */
static void rows_q6_k(const uint8_t *w, size_t nb, const float *x, float *out, size_t begin, size_t end) {
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * nb * 210;
        float corr = 0.0f;
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * 210;
            const float d = f16(b + 208);
            const uint8_t *ql = b, *qh = b + 128;
            const int8_t *sc = (const int8_t *)(b + 192);
            const float *xb = x + rb * 256;
            V16 acc = v16_zero();
            for (int n = 0; n < 2; n++) {
                const int y = 128 * n, qlo = 64 * n, qho = 32 * n, sco = 8 * n;
                for (int lb = 0; lb < 32; lb += 16) {
                    const int is = lb / 16;
                    acc = v16_fma(d * (float)sc[sco + is + 0],
                                  v16_q6(q6_quants(ql + qlo + lb, qh + qho + lb, 0, 0), xb + y + lb), acc);
                    acc = v16_fma(d * (float)sc[sco + is + 2],
                                  v16_q6(q6_quants(ql + qlo + lb + 32, qh + qho + lb, 0, 2), xb + y + lb + 32), acc);
                    acc = v16_fma(d * (float)sc[sco + is + 4],
                                  v16_q6(q6_quants(ql + qlo + lb, qh + qho + lb, 1, 4), xb + y + lb + 64), acc);
                    acc = v16_fma(d * (float)sc[sco + is + 6],
                                  v16_q6(q6_quants(ql + qlo + lb + 32, qh + qho + lb, 1, 6), xb + y + lb + 96), acc);
                }
            }
            float t[16];
            v16_store(t, acc);
            float s = t[0];
            for (int j = 1; j < 16; j++) s += t[j];
            corr += s;
        }
        out[i] = 0.0f + corr;
    }
}

/* matVecF32 / matVecF16 (matvec/kernels/float.zig:67-95): one f32 accumulator
 * per row in element order (a product and a sum, two roundings): a sequential
 * dependency chain in zlm too, so it stays scalar. */
static void rows_f32(const uint8_t *w, size_t k, const float *x, float *out, size_t begin, size_t end) {
    for (size_t i = begin; i < end; i++) {
        const float *row = (const float *)(w + i * k * 4);
        float acc = 0.0f;
        for (size_t j = 0; j < k; j++) {
            float v;
            memcpy(&v, row + j, 4);
            acc += v * x[j];
        }
        out[i] = acc;
    }
}

static void rows_f16(const uint8_t *w, size_t k, const float *x, float *out, size_t begin, size_t end) {
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * k * 2;
        float acc = 0.0f;
        for (size_t j = 0; j < k; j++) acc += f16(row + 2 * j) * x[j];
        out[i] = acc;
    }
}

/* matVecBF16 (matvec/kernels/bfloat.zig:44-67): two 8-lane accumulators of
 * rounded products and sums, reduced in lane order, then the tail. */
static void rows_bf16(const uint8_t *w, size_t k, const float *x, float *out, size_t begin, size_t end) {
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * k * 2;
        __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
        size_t j = 0;
        for (; j + 16 <= k; j += 16) {
            const __m256i r0 = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(row + 2 * j)));
            const __m256i r1 = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(row + 2 * j + 16)));
            a0 = _mm256_add_ps(a0, _mm256_mul_ps(_mm256_castsi256_ps(_mm256_slli_epi32(r0, 16)), _mm256_loadu_ps(x + j)));
            a1 = _mm256_add_ps(a1,
                               _mm256_mul_ps(_mm256_castsi256_ps(_mm256_slli_epi32(r1, 16)), _mm256_loadu_ps(x + j + 8)));
        }
        float t0[8], t1[8];
        _mm256_storeu_ps(t0, a0);
        _mm256_storeu_ps(t1, a1);
        float s0 = t0[0], s1 = t1[0];
        for (int l = 1; l < 8; l++) {
            s0 += t0[l];
            s1 += t1[l];
        }
        float acc = s0 + s1;
        for (; j < k; j++) {
            const uint32_t bits = (uint32_t)(row[2 * j] | (row[2 * j + 1] << 8)) << 16;
            float v;
            memcpy(&v, &bits, 4);
            acc += v * x[j];
        }
        out[i] = acc;
    }
}

/* q4KNibXSum32 / q4KXSum (layout.zig:294-301, :499-504), the per-32 sums the
 * min-term types read (xBlockSum for q4_1 is the same sum). */
static float xsum32(const float *xb) {
    float v[8];
    for (int j = 0; j < 8; j++) v[j] = (xb[j] + xb[8 + j]) + (xb[16 + j] + xb[24 + j]);
    float r = v[0];
    for (int j = 1; j < 8; j++) r += v[j];
    return r;
}

/* The production fp sweep over rows [begin, end) (matVecRowsWithPlan(.production),
 * single.zig:168-205), shape checks as orc_matvec's. */
int SW(orc_sweep_matvec)(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows, const float *x,
                         float *out, size_t begin, size_t end) {
    const size_t be = orc_block_elems(t), bb = orc_block_bytes(t);
    if (be == 0) return ORC_E_UNSUPPORTED;
    if (k % be != 0) return ORC_E_SHAPE;
    if (w_len < rows * (k / be) * bb) return ORC_E_TRUNCATED;
    if (begin > end || end > rows) return ORC_E_RANGE;
    const size_t nb = k / be;
    switch (t) {
    case ORC_Q4_0: rows_q4_0(w, nb, x, out, begin, end); return ORC_OK;
    case ORC_Q8_0: rows_q8_0(w, nb, x, out, begin, end); return ORC_OK;
    case ORC_Q6_K: rows_q6_k(w, nb, x, out, begin, end); return ORC_OK;
    case ORC_F32: rows_f32(w, k, x, out, begin, end); return ORC_OK;
    case ORC_F16: rows_f16(w, k, x, out, begin, end); return ORC_OK;
    case ORC_BF16: rows_bf16(w, k, x, out, begin, end); return ORC_OK;
    case ORC_Q4_1:
    case ORC_Q4_K: {
        if (k / 32 > 2048) return ORC_E_SHAPE; /* the bounded activation cache (types.zig:8) */
        float xs[2048];
        for (size_t c = 0; c < k / 32; c++) xs[c] = xsum32(x + 32 * c);
        if (t == ORC_Q4_1) rows_q4_1(w, nb, x, xs, out, begin, end);
        else rows_q4_k(w, nb, x, xs, out, begin, end);
        return ORC_OK;
    }
    default: return ORC_E_UNSUPPORTED;
    }
}

/* ---- the int path (q8 activations), Q4_0 and Q8_0 --------------------- */

/* The i32 products of a block folded into `lanes` groups of consecutive terms
 * (q4_0IntBlockVec / q8_0IntBlockVec, layout.zig:63-94, :119-138), as f32. */
#if SW_LANES == 8
INL V fold16(__m256i p_lo, __m256i p_hi) { return _mm256_cvtepi32_ps(_mm256_add_epi32(p_lo, p_hi)); }
#endif

/* Q4_0.intBlock (quantized.zig:49-55): unsigned nibble x q8 activation;
 * acc = fma(dw*dx, f32(iv), acc); corr -= dw*(8*dx*sums). */
static void rows_q4_0_int(const uint8_t *w, size_t nb, const int8_t *qx, const float *dx, const int32_t *sums,
                          float *out, size_t begin, size_t end) {
    const __m128i m4 = _mm_set1_epi8(0x0F);
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * nb * 18;
        V acc = VZERO();
        float corr = 0.0f;
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * 18;
            const __m128i bytes = _mm_loadu_si128((const __m128i *)(b + 2));
            const __m256i lo = _mm256_cvtepu8_epi16(_mm_and_si128(bytes, m4));
            const __m256i hi = _mm256_cvtepu8_epi16(_mm_and_si128(_mm_srli_epi16(bytes, 4), m4));
            const __m256i x0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(qx + rb * 32)));
            const __m256i x1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(qx + rb * 32 + 16)));
            /* p[j] = lo[j]*qx[j] + hi[j]*qx[16+j] (|products| < 2^15) */
            const __m256i p16 = _mm256_add_epi16(_mm256_mullo_epi16(lo, x0), _mm256_mullo_epi16(hi, x1));
#if SW_LANES == 8
            const V iv = fold16(_mm256_cvtepi16_epi32(_mm256_castsi256_si128(p16)),
                                _mm256_cvtepi16_epi32(_mm256_extracti128_si256(p16, 1)));
#else
            const V iv = _mm512_cvtepi32_ps(_mm512_cvtepi16_epi32(p16));
#endif
            const float dw = f16(b);
            acc = VFMA(VSET1(dw * dx[rb]), iv, acc);
            corr -= dw * (8.0f * dx[rb] * (float)sums[rb]);
        }
        out[i] = vsum(acc) + corr;
    }
}

/* Q8_0.intBlock (quantized.zig:149-156). */
static void rows_q8_0_int(const uint8_t *w, size_t nb, const int8_t *qx, const float *dx, float *out, size_t begin,
                          size_t end) {
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * nb * 34;
        V acc = VZERO();
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * 34;
            __m256i p[2];
            for (int h = 0; h < 2; h++) {
                const __m256i wq = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + 2 + 16 * h)));
                const __m256i xq = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(qx + rb * 32 + 16 * h)));
                p[h] = _mm256_mullo_epi16(wq, xq); /* |q*qx| <= 127*127 < 2^15 */
            }
            /* 32 products into `lanes` groups of consecutive terms: lane j sums p[j + m*lanes] */
#if SW_LANES == 8
            const __m256i s = _mm256_add_epi32(
                _mm256_add_epi32(_mm256_cvtepi16_epi32(_mm256_castsi256_si128(p[0])),
                                 _mm256_cvtepi16_epi32(_mm256_extracti128_si256(p[0], 1))),
                _mm256_add_epi32(_mm256_cvtepi16_epi32(_mm256_castsi256_si128(p[1])),
                                 _mm256_cvtepi16_epi32(_mm256_extracti128_si256(p[1], 1))));
            const V iv = _mm256_cvtepi32_ps(s);
#else
            const V iv = _mm512_cvtepi32_ps(_mm512_add_epi32(_mm512_cvtepi16_epi32(p[0]), _mm512_cvtepi16_epi32(p[1])));
#endif
            acc = VFMA(VSET1(f16(b) * dx[rb]), iv, acc);
        }
        out[i] = vsum(acc) + 0.0f;
    }
}

/* The `.int` sweep (single.zig:65-73, :82-140) of one token over rows
 * [begin, end), from an activation already quantized by orc_quantize_act_q8. */
int SW(orc_sweep_matvec_int_q8)(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                                const int8_t *qx, const float *dx, const int32_t *sums, float *out, size_t begin,
                                size_t end) {
    if (t != ORC_Q4_0 && t != ORC_Q8_0) return ORC_E_UNSUPPORTED;
    const size_t bb = orc_block_bytes(t);
    if (k % 32 != 0) return ORC_E_SHAPE;
    if (w_len < rows * (k / 32) * bb) return ORC_E_TRUNCATED;
    if (begin > end || end > rows) return ORC_E_RANGE;
    if (t == ORC_Q4_0) rows_q4_0_int(w, k / 32, qx, dx, sums, out, begin, end);
    else rows_q8_0_int(w, k / 32, qx, dx, out, begin, end);
    return ORC_OK;
}
