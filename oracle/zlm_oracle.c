/*
 * zlm_oracle.c -- CPU restatement of zlm's quantized matvec/matmul kernels.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker of the HIP backend and the CPU
 * baseline of bench.py.  Nothing in zlm_amd/ links or calls this file.
 *
 * zlm is Zig 0.16 and no Zig toolchain exists in this environment, so the
 * reference kernels cannot be built; this file restates them.  It keeps the
 * reference's operation order and its fused multiply-add points:
 *   - `simd.fma` (kernels/simd.zig:51-68) is `@mulAdd` on FMA hosts, so every
 *     such call is `fmaf` here;
 *   - every other `a*b + c` in the Zig source is two rounded operations, so the
 *     file is compiled with -ffp-contract=off;
 *   - `@reduce(.Add, v)` over f32 lanes is restated as an in-order lane sum.
 * The reference's exact output bits also depend on LLVM's lowering of
 * `@reduce`; the GPU parity bar is therefore a relative-L2 tolerance, while
 * dequantized blocks are compared bit-exactly.
 *
 * `lanes` is the `simd.native` width the Zig build would pick: 16 on AVX-512
 * hosts, 8 on AVX2 hosts, 4 elsewhere (kernels/simd.zig:30-41).
 */
#define _GNU_SOURCE
#include "zlm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define ALWAYS_INLINE static inline __attribute__((always_inline))

/* ---- f16 <-> f32 ------------------------------------------------------- */

/* Exact widening, as Zig's @floatCast(f16 -> f32) (quant/types.zig:21-23). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            float v = (float)man * 0x1p-24f; /* subnormal: man * 2^-24, exact */
            return sign ? -v : v;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round-to-nearest-even narrowing (used only to build synthetic scales). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float v;
        memcpy(&v, &ax, 4);
        float s = v * 0x1p24f;
        uint32_t r = (uint32_t)rintf(s);
        return (uint16_t)(sign | r);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t half = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
    return (uint16_t)(sign | half);
}

ALWAYS_INLINE float rd_f16(const uint8_t *p) {
    return orc_f16_to_f32((uint16_t)(p[0] | ((uint16_t)p[1] << 8)));
}

/* ---- block formats (gpu/backend/root.zig:198-220, gguf/format.zig:135-159) */

size_t orc_block_elems(uint32_t t) {
    switch (t) {
    case ORC_Q4_0: case ORC_Q4_1: case ORC_Q8_0: return 32;
    case ORC_Q4_K: case ORC_Q6_K: return 256;
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    default: return 0;
    }
}

size_t orc_block_bytes(uint32_t t) {
    switch (t) {
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q8_0: return 34;
    case ORC_Q4_K: return 144;
    case ORC_Q6_K: return 210;
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    default: return 0;
    }
}

/* gguf/format.zig:170-174: ceil(n / block_elems) * block_bytes. */
int64_t orc_tensor_byte_length(uint32_t t, uint64_t n) {
    size_t be = orc_block_elems(t), bb = orc_block_bytes(t);
    if (be == 0) return -1;
    return (int64_t)(((n + be - 1) / be) * bb);
}

/* quant/k_quants.zig:24-32. */
void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ---- dequant codecs (bit-exact targets) -------------------------------- */

/* quant/standard.zig:44-93: element j = d*f32(lo(q[j])-8), j+16 = d*f32(hi-8). */
static void dq_q4_0_block(const uint8_t *b, float *out /*32*/) {
    float d = rd_f16(b);
    for (int j = 0; j < 16; j++) {
        out[j] = (float)((int)(b[2 + j] & 0x0F) - 8) * d;
        out[16 + j] = (float)((int)(b[2 + j] >> 4) - 8) * d;
    }
}

/* quant/standard.zig:10-42: d*f32(q). */
static void dq_q8_0_block(const uint8_t *b, float *out) {
    float d = rd_f16(b);
    for (int j = 0; j < 32; j++) out[j] = (float)(int8_t)b[2 + j] * d;
}

/* quant/standard.zig:95-160 (q4_1): f32(q)*d + m, two roundings. */
static void dq_q4_1_block(const uint8_t *b, float *out) {
    float d = rd_f16(b), m = rd_f16(b + 2);
    for (int j = 0; j < 16; j++) {
        out[j] = (float)(b[4 + j] & 0x0F) * d + m;
        out[16 + j] = (float)(b[4 + j] >> 4) * d + m;
    }
}

/* quant/k_quants.zig:34-72: per 64-element group, fma(f32(nib), d*sc, -(dmin*mn)). */
static void dq_q4_k_block(const uint8_t *b, float *out) {
    float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *sc = b + 4, *q = b + 16;
    for (int g = 0; g < 4; g++) {
        uint8_t s1, m1, s2, m2;
        orc_get_scale_min_k4(2 * g, sc, &s1, &m1);
        orc_get_scale_min_k4(2 * g + 1, sc, &s2, &m2);
        float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        float d2 = d * (float)s2, mm2 = dmin * (float)m2;
        const uint8_t *qq = q + 32 * g;
        for (int l = 0; l < 32; l++) {
            out[64 * g + l] = fmaf((float)(qq[l] & 0x0F), d1, -mm1);
            out[64 * g + 32 + l] = fmaf((float)(qq[l] >> 4), d2, -mm2);
        }
    }
}

/* quant/k_quants.zig:128-175: f32(q-32) * (d*sc). */
static void dq_q6_k_block(const uint8_t *b, float *out) {
    float d = rd_f16(b + 208);
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    for (int n = 0; n < 2; n++) {
        const uint8_t *l0 = ql + 64 * n, *h0 = qh + 32 * n;
        const int8_t *s = sc + 8 * n;
        float *o = out + 128 * n;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (l0[l] & 0xF) | (((h0[l] >> 0) & 3) << 4);
            int q2 = (l0[l + 32] & 0xF) | (((h0[l] >> 2) & 3) << 4);
            int q3 = (l0[l] >> 4) | (((h0[l] >> 4) & 3) << 4);
            int q4 = (l0[l + 32] >> 4) | (((h0[l] >> 6) & 3) << 4);
            o[l] = (float)(q1 - 32) * (d * (float)s[is + 0]);
            o[l + 32] = (float)(q2 - 32) * (d * (float)s[is + 2]);
            o[l + 64] = (float)(q3 - 32) * (d * (float)s[is + 4]);
            o[l + 96] = (float)(q4 - 32) * (d * (float)s[is + 6]);
        }
    }
}

/*
 * quant/root.zig:44-57 (`dequantTo`) over quant/root.zig:21-40 (`dequant`):
 * whole blocks, then a partial tail decoded from one more full block.  The
 * K-quant codecs reject a non-multiple length (k_quants.zig:35, :129).
 */
int orc_dequant(uint32_t t, const uint8_t *data, size_t data_len, float *out, size_t n) {
    size_t be = orc_block_elems(t), bb = orc_block_bytes(t);
    if (be == 0) return ORC_E_UNSUPPORTED;
    if ((t == ORC_Q4_K || t == ORC_Q6_K) && n % be != 0) return ORC_E_SHAPE;
    size_t full = n / be, rem = n % be;
    size_t need = full * bb + (rem ? bb : 0);
    if (data_len < need) return ORC_E_TRUNCATED;
    float tmp[256];
    for (size_t i = 0; i < full + (rem ? 1 : 0); i++) {
        const uint8_t *b = data + i * bb;
        float *dst = (i < full) ? out + i * be : tmp;
        switch (t) {
        case ORC_Q4_0: dq_q4_0_block(b, dst); break;
        case ORC_Q4_1: dq_q4_1_block(b, dst); break;
        case ORC_Q8_0: dq_q8_0_block(b, dst); break;
        case ORC_Q4_K: dq_q4_k_block(b, dst); break;
        case ORC_Q6_K: dq_q6_k_block(b, dst); break;
        case ORC_F32: memcpy(dst, b, 4); break;
        case ORC_F16: dst[0] = rd_f16(b); break;
        case ORC_BF16: {
            uint32_t bits = ((uint32_t)b[0] | ((uint32_t)b[1] << 8)) << 16;
            memcpy(dst, &bits, 4);
            break;
        }
        default: return ORC_E_UNSUPPORTED;
        }
        if (i == full) memcpy(out + full * be, tmp, rem * sizeof(float));
    }
    return ORC_OK;
}

/* ---- the production fp sweep ------------------------------------------- */

/* `@reduce(.Add, v)` restated as an in-order lane sum. */
ALWAYS_INLINE float lane_sum(const float *v, int L) {
    float r = v[0];
    for (int j = 1; j < L; j++) r += v[j];
    return r;
}

/*
 * Q4_0.fpBlock (matvec/kernels/quantized.zig:42-47) over q4_0BlockVec
 * (matvec/layout.zig:27-51): the signed nibbles times x, `lanes` at a time with
 * fma, then acc = fma(d, blockvec, acc).
 */
ALWAYS_INLINE void fp_q4_0(int L, const uint8_t *b, const float *xb, float *acc) {
    float q[32], bv[16];
    for (int j = 0; j < 16; j++) {
        q[j] = (float)((int)(b[2 + j] & 0x0F) - 8);
        q[16 + j] = (float)((int)(b[2 + j] >> 4) - 8);
    }
    for (int j = 0; j < L; j++) bv[j] = 0.0f;
    for (int s = 0; s < 32; s += L)
        for (int j = 0; j < L; j++) bv[j] = fmaf(q[s + j], xb[s + j], bv[j]);
    float d = rd_f16(b);
    for (int j = 0; j < L; j++) acc[j] = fmaf(d, bv[j], acc[j]);
}

/* Q8_0.fpBlock (quantized.zig:142-147) over q8_0BlockVec (layout.zig:99-111). */
ALWAYS_INLINE void fp_q8_0(int L, const uint8_t *b, const float *xb, float *acc) {
    float bv[16];
    for (int j = 0; j < L; j++) bv[j] = 0.0f;
    for (int s = 0; s < 32; s += L)
        for (int j = 0; j < L; j++) bv[j] = fmaf((float)(int8_t)b[2 + s + j], xb[s + j], bv[j]);
    float d = rd_f16(b);
    for (int j = 0; j < L; j++) acc[j] = fmaf(d, bv[j], acc[j]);
}

/* q4KNibVec (layout.zig:215-261): unscaled lanes-wide partial of 32 nibbles. */
ALWAYS_INLINE void q4k_nibvec(int L, const uint8_t *qs, const float *xb, int hi, float *out) {
    float p[32];
    for (int j = 0; j < 32; j++) p[j] = (float)(hi ? (qs[j] >> 4) : (qs[j] & 0x0F)) * xb[j];
    if (L == 8) {
        for (int j = 0; j < 8; j++) out[j] = (p[j] + p[8 + j]) + (p[16 + j] + p[24 + j]);
    } else if (L == 16) {
        for (int j = 0; j < 16; j++) out[j] = p[j] + p[16 + j];
    } else {
        for (int j = 0; j < 4; j++)
            out[j] = ((p[j] + p[4 + j]) + (p[8 + j] + p[12 + j])) +
                     ((p[16 + j] + p[20 + j]) + (p[24 + j] + p[28 + j]));
    }
}

/* q4KNibXSum32 (layout.zig:294-301) and q4KXSum (layout.zig:499-504). */
static float q4k_xsum32(const float *xb) {
    float v[8];
    for (int j = 0; j < 8; j++) v[j] = (xb[j] + xb[8 + j]) + (xb[16 + j] + xb[24 + j]);
    return lane_sum(v, 8);
}

static void q4k_xsum(const float *x, size_t n, float *xsum) {
    for (size_t c = 0; c < n / 32; c++) xsum[c] = q4k_xsum32(x + 32 * c);
}

/*
 * Q4_K.fpBlock (quantized.zig:105-109) over q4KBlockAccumGen (layout.zig:309-342):
 * acc = fma(d*sc, nibvec, acc) per 32-chunk; the min term d_min*mn*xsum summed
 * into `msum`, subtracted from `corr` once per super-block.
 */
ALWAYS_INLINE void fp_q4_k(int L, const uint8_t *b, const float *xb, const float *xs, float *acc,
                           float *corr) {
    float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *sc = b + 4, *qs = b + 16;
    float msum = 0.0f, v[16];
    for (int g = 0; g < 4; g++) {
        uint8_t s1, m1, s2, m2;
        orc_get_scale_min_k4(2 * g, sc, &s1, &m1);
        orc_get_scale_min_k4(2 * g + 1, sc, &s2, &m2);
        q4k_nibvec(L, qs + 32 * g, xb + 64 * g, 0, v);
        float ds1 = d * (float)s1;
        for (int j = 0; j < L; j++) acc[j] = fmaf(ds1, v[j], acc[j]);
        q4k_nibvec(L, qs + 32 * g, xb + 64 * g + 32, 1, v);
        float ds2 = d * (float)s2;
        for (int j = 0; j < L; j++) acc[j] = fmaf(ds2, v[j], acc[j]);
        msum += (dmin * (float)m1) * xs[2 * g] + (dmin * (float)m2) * xs[2 * g + 1];
    }
    *corr -= msum;
}

/* q6KChunkVec16 (layout.zig:392-412): (f32(q) - 32) * x over 16 elements. */
ALWAYS_INLINE void q6k_chunk(const uint8_t *ql, const uint8_t *qh, const float *xb, int hi,
                             int shift, float *out) {
    for (int j = 0; j < 16; j++) {
        int nib = hi ? (ql[j] >> 4) : (ql[j] & 0x0F);
        int hb = (qh[j] >> shift) & 3;
        float qf = (float)(int8_t)(uint8_t)(nib | (hb << 4)) - 32.0f;
        out[j] = qf * xb[j];
    }
}

/* q6KBlockDot (layout.zig:414-452): 16-wide fma accumulation, one reduce. */
static float q6k_block_dot(const uint8_t *b, const float *xb) {
    float d = rd_f16(b + 208);
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float acc[16] = {0}, v[16];
    for (int n = 0; n < 2; n++) {
        int y = 128 * n, qlo = 64 * n, qho = 32 * n, sco = 8 * n;
        for (int lb = 0; lb < 32; lb += 16) {
            int is = lb / 16;
            float a0 = (float)sc[sco + is + 0], a2 = (float)sc[sco + is + 2];
            float a4 = (float)sc[sco + is + 4], a6 = (float)sc[sco + is + 6];
            float s;
            q6k_chunk(ql + qlo + lb, qh + qho + lb, xb + y + lb, 0, 0, v);
            s = d * a0;
            for (int j = 0; j < 16; j++) acc[j] = fmaf(s, v[j], acc[j]);
            q6k_chunk(ql + qlo + lb + 32, qh + qho + lb, xb + y + lb + 32, 0, 2, v);
            s = d * a2;
            for (int j = 0; j < 16; j++) acc[j] = fmaf(s, v[j], acc[j]);
            q6k_chunk(ql + qlo + lb, qh + qho + lb, xb + y + lb + 64, 1, 4, v);
            s = d * a4;
            for (int j = 0; j < 16; j++) acc[j] = fmaf(s, v[j], acc[j]);
            q6k_chunk(ql + qlo + lb + 32, qh + qho + lb, xb + y + lb + 96, 1, 6, v);
            s = d * a6;
            for (int j = 0; j < 16; j++) acc[j] = fmaf(s, v[j], acc[j]);
        }
    }
    return lane_sum(acc, 16);
}

/* Q4_1.fpBlock (quantized.zig:71-77) over q4_1BlockVecLanes (layout.zig:164-180). */
ALWAYS_INLINE void fp_q4_1(int L, const uint8_t *b, const float *xb, float xsum, float *acc,
                           float *corr) {
    float q[32], bv[16];
    for (int j = 0; j < 16; j++) {
        q[j] = (float)(b[4 + j] & 0x0F);
        q[16 + j] = (float)(b[4 + j] >> 4);
    }
    for (int j = 0; j < L; j++) bv[j] = 0.0f;
    for (int s = 0; s < 32; s += L)
        for (int j = 0; j < L; j++) bv[j] = fmaf(q[s + j], xb[s + j], bv[j]);
    float d = rd_f16(b), mn = rd_f16(b + 2);
    for (int j = 0; j < L; j++) acc[j] = fmaf(d, bv[j], acc[j]);
    *corr += mn * xsum;
}

/* xBlockSum (layout.zig:489-495) as the q4_1 min-term activation sum. */
static float q4_1_xsum(const float *xb) { return q4k_xsum32(xb); }

/*
 * The L3 sweep at tile=1, unroll=1 (matvec/form/single.zig:29-140), i.e. the
 * `production_fp` body every type uses (quantized.zig:205-241).  Per row:
 * acc = 0 (lanes), corr = 0; fpBlock over the row's blocks; out = reduce + corr.
 */
ALWAYS_INLINE void sweep_fp(int L, uint32_t t, const uint8_t *w, size_t k, const float *x,
                            const float *xsum, float *out, size_t begin, size_t end) {
    size_t be = orc_block_elems(t), bb = orc_block_bytes(t), nb = k / be, rowb = nb * bb;
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * rowb;
        float acc[16], corr = 0.0f;
        for (int j = 0; j < L; j++) acc[j] = 0.0f;
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * bb;
            switch (t) {
            case ORC_Q4_0: fp_q4_0(L, b, x + rb * 32, acc); break;
            case ORC_Q8_0: fp_q8_0(L, b, x + rb * 32, acc); break;
            case ORC_Q4_1: fp_q4_1(L, b, x + rb * 32, xsum[rb], acc, &corr); break;
            case ORC_Q4_K: fp_q4_k(L, b, x + rb * 256, xsum + rb * 8, acc, &corr); break;
            case ORC_Q6_K: corr += q6k_block_dot(b, x + rb * 256); break;
            default: break;
            }
        }
        out[i] = lane_sum(acc, L) + corr;
    }
}

static int check_shape(uint32_t t, size_t w_len, size_t k, size_t rows, size_t begin, size_t end) {
    size_t be = orc_block_elems(t), bb = orc_block_bytes(t);
    if (be == 0) return ORC_E_UNSUPPORTED;
    if (k % be != 0) return ORC_E_SHAPE;
    if (w_len < rows * (k / be) * bb) return ORC_E_TRUNCATED;
    if (begin > end || end > rows) return ORC_E_RANGE;
    return ORC_OK;
}

/* One weight element of a float row (F32 / F16 / BF16) widened to f32. */
ALWAYS_INLINE float float_elem(uint32_t t, const uint8_t *row, size_t j) {
    if (t == ORC_F32) {
        float v;
        memcpy(&v, row + 4 * j, 4);
        return v;
    }
    uint16_t h = (uint16_t)(row[2 * j] | ((uint16_t)row[2 * j + 1] << 8));
    if (t == ORC_F16) return orc_f16_to_f32(h);
    uint32_t bits = (uint32_t)h << 16;
    float v;
    memcpy(&v, &bits, 4);
    return v;
}

/*
 * matVecF32 / matVecF16 (matvec/kernels/float.zig:67-95), the float types'
 * production_fp: per row one f32 accumulator, acc += w * x[j] (a product and a
 * sum, two roundings), in element order.
 */
static void matvec_float_seq(uint32_t t, const uint8_t *w, size_t k, const float *x, float *out,
                             size_t begin, size_t end) {
    size_t rowb = k * orc_block_bytes(t);
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * rowb;
        float acc = 0.0f;
        for (size_t j = 0; j < k; j++) acc += float_elem(t, row, j) * x[j];
        out[i] = acc;
    }
}

/*
 * matVecBF16 (matvec/kernels/bfloat.zig:44-67): two 8-lane accumulators over
 * 16-element steps (acc0 += w[j..j+8]*x, acc1 += w[j+8..j+16]*x, products and
 * sums rounded separately), acc = reduce(acc0) + reduce(acc1), then the tail
 * elements one by one.
 */
static void matvec_bf16(const uint8_t *w, size_t k, const float *x, float *out, size_t begin,
                        size_t end) {
    size_t rowb = k * 2;
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * rowb;
        float a0[8] = {0}, a1[8] = {0};
        size_t j = 0;
        for (; j + 16 <= k; j += 16) {
            for (int l = 0; l < 8; l++) {
                a0[l] += float_elem(ORC_BF16, row, j + l) * x[j + l];
                a1[l] += float_elem(ORC_BF16, row, j + 8 + l) * x[j + 8 + l];
            }
        }
        float acc = lane_sum(a0, 8) + lane_sum(a1, 8);
        for (; j < k; j++) acc += float_elem(ORC_BF16, row, j) * x[j];
        out[i] = acc;
    }
}

/* matVecRowsWithPlan(.production) (single.zig:168-205): each type's production_fp. */
int orc_matvec(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows, const float *x,
               float *out, size_t begin, size_t end, int lanes) {
    int rc = check_shape(t, w_len, k, rows, begin, end);
    if (rc) return rc;
    if (t == ORC_F32 || t == ORC_F16) {
        matvec_float_seq(t, w, k, x, out, begin, end);
        return ORC_OK;
    }
    if (t == ORC_BF16) {
        matvec_bf16(w, k, x, out, begin, end);
        return ORC_OK;
    }
    float *xsum = NULL;
    if (t == ORC_Q4_K || t == ORC_Q4_1) {
        /* The bounded activation cache (types.zig:8, single.zig:76-80). */
        if (k / 32 > 2048) return ORC_E_SHAPE;
        xsum = (float *)malloc((k / 32) * sizeof(float));
        if (t == ORC_Q4_K) {
            q4k_xsum(x, k, xsum);
        } else {
            for (size_t c = 0; c < k / 32; c++) xsum[c] = q4_1_xsum(x + 32 * c);
        }
    }
    switch (lanes) {
    case 4: sweep_fp(4, t, w, k, x, xsum, out, begin, end); break;
    case 16: sweep_fp(16, t, w, k, x, xsum, out, begin, end); break;
    default: sweep_fp(8, t, w, k, x, xsum, out, begin, end); break;
    }
    free(xsum);
    return ORC_OK;
}

/*
 * lmHeadRows (single.zig:294-360): q8_0/q6_k/q4_k rows through row_dot.dot
 * (form/dot.zig:21-51), which is the tile-1 sweep at native lanes: one fpBlock
 * per block, one reduce per row.  That is the same arithmetic as orc_matvec.
 */
int orc_lm_head_rows(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                     const float *x, float *out, size_t begin, size_t end, int lanes) {
    return orc_matvec(t, w, w_len, k, rows, x, out, begin, end, lanes);
}

/* ---- the int path (q8 activations) ------------------------------------- */

/*
 * quantizeActivationQ8Sum (layout.zig:458-476): per 32-block amax, d = amax/127
 * (f32), inv = d != 0 ? 1/d : 0, q = round-half-away(v*inv) clamped to +-127,
 * sums = integer sum of q.
 */
void orc_quantize_act_q8(const float *x, size_t blocks, int8_t *qx, float *dx, int32_t *sums) {
    for (size_t rb = 0; rb < blocks; rb++) {
        const float *xb = x + rb * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        float d = amax / 127.0f;
        float inv = (d != 0.0f) ? 1.0f / d : 0.0f;
        int32_t s = 0;
        for (int j = 0; j < 32; j++) {
            float r = roundf(xb[j] * inv);
            int32_t q = (int32_t)r;
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            qx[rb * 32 + j] = (int8_t)q;
            s += q;
        }
        dx[rb] = d;
        sums[rb] = s;
    }
}

/* Fold `n` integer products into L lanes of consecutive groups (layout.zig:80-93). */
ALWAYS_INLINE void fold_lanes(int L, const int32_t *p, int n, float *ivf) {
    for (int j = 0; j < L; j++) {
        int32_t a = 0;
        for (int m = 0; m < n / L; m++) a += p[j + m * L];
        ivf[j] = (float)a;
    }
}

/*
 * Q4_0.intBlock (quantized.zig:49-55) over q4_0IntBlockVec (layout.zig:63-94):
 * unsigned nibble times q8 activation; acc = fma(dw*dx, f32(iv), acc);
 * corr -= dw*(8*dx*sums).
 */
ALWAYS_INLINE void int_q4_0(int L, const uint8_t *b, const int8_t *qx, float dx, int32_t sum,
                            float *acc, float *corr) {
    int32_t p[16];
    float ivf[16];
    for (int j = 0; j < 16; j++) p[j] = (int32_t)(b[2 + j] & 0x0F) * qx[j] + (int32_t)(b[2 + j] >> 4) * qx[16 + j];
    fold_lanes(L, p, 16, ivf);
    float dw = rd_f16(b);
    float s = dw * dx;
    for (int j = 0; j < L; j++) acc[j] = fmaf(s, ivf[j], acc[j]);
    *corr -= dw * (8.0f * dx * (float)sum);
}

/* Q8_0.intBlock (quantized.zig:149-156) over q8_0IntBlockVec (layout.zig:119-138). */
ALWAYS_INLINE void int_q8_0(int L, const uint8_t *b, const int8_t *qx, float dx, float *acc) {
    int32_t p[32];
    float ivf[16];
    for (int j = 0; j < 32; j++) p[j] = (int32_t)(int8_t)b[2 + j] * qx[j];
    fold_lanes(L, p, 32, ivf);
    float s = rd_f16(b) * dx;
    for (int j = 0; j < L; j++) acc[j] = fmaf(s, ivf[j], acc[j]);
}

/*
 * Q4_1.intBlock (quantized.zig:79-87) over q4_1IntBlockVec (layout.zig:185-210):
 * unsigned nibble times q8 activation folded into lanes;
 * acc = fma(d*dx, f32(iv), acc); corr += (mn*dx) * f32(sums).
 */
ALWAYS_INLINE void int_q4_1(int L, const uint8_t *b, const int8_t *qx, float dx, int32_t sum,
                            float *acc, float *corr) {
    int32_t p[16];
    float ivf[16];
    for (int j = 0; j < 16; j++) p[j] = (int32_t)(b[4 + j] & 0x0F) * qx[j] + (int32_t)(b[4 + j] >> 4) * qx[16 + j];
    fold_lanes(L, p, 16, ivf);
    float d = rd_f16(b), mn = rd_f16(b + 2);
    float s = d * dx;
    for (int j = 0; j < L; j++) acc[j] = fmaf(s, ivf[j], acc[j]);
    *corr += mn * dx * (float)sum;
}

/* q4KBlockIntAccum (layout.zig:349-387) as Q4_K.intBlock (quantized.zig:111-123). */
ALWAYS_INLINE void int_q4_k(int L, const uint8_t *b, const int8_t *qx, const float *dx,
                            const int32_t *sums, float *acc, float *corr) {
    float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *sc = b + 4, *qs = b + 16;
    float c = 0.0f, ivf[16];
    int32_t p[32];
    for (int g = 0; g < 4; g++) {
        uint8_t s1, m1, s2, m2;
        orc_get_scale_min_k4(2 * g, sc, &s1, &m1);
        orc_get_scale_min_k4(2 * g + 1, sc, &s2, &m2);
        int cc = 2 * g;
        for (int j = 0; j < 32; j++) p[j] = (int32_t)(qs[32 * g + j] & 0x0F) * qx[cc * 32 + j];
        fold_lanes(L, p, 32, ivf);
        float f1 = d * (float)s1 * dx[cc];
        for (int j = 0; j < L; j++) acc[j] = fmaf(f1, ivf[j], acc[j]);
        for (int j = 0; j < 32; j++) p[j] = (int32_t)(qs[32 * g + j] >> 4) * qx[(cc + 1) * 32 + j];
        fold_lanes(L, p, 32, ivf);
        float f2 = d * (float)s2 * dx[cc + 1];
        for (int j = 0; j < L; j++) acc[j] = fmaf(f2, ivf[j], acc[j]);
        c += (dmin * (float)m1 * dx[cc]) * (float)sums[cc] +
             (dmin * (float)m2 * dx[cc + 1]) * (float)sums[cc + 1];
    }
    *corr -= c;
}

/* The sweep's `.int` instantiation (single.zig:65-73, :82-140), tile 1, unroll 1. */
ALWAYS_INLINE void sweep_int(int L, uint32_t t, const uint8_t *w, size_t k, const int8_t *qx,
                             const float *dx, const int32_t *sums, float *out, size_t begin,
                             size_t end) {
    size_t be = orc_block_elems(t), bb = orc_block_bytes(t), nb = k / be, rowb = nb * bb;
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * rowb;
        float acc[16], corr = 0.0f;
        for (int j = 0; j < L; j++) acc[j] = 0.0f;
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * bb;
            switch (t) {
            case ORC_Q4_0: int_q4_0(L, b, qx + rb * 32, dx[rb], sums[rb], acc, &corr); break;
            case ORC_Q8_0: int_q8_0(L, b, qx + rb * 32, dx[rb], acc); break;
            case ORC_Q4_1: int_q4_1(L, b, qx + rb * 32, dx[rb], sums[rb], acc, &corr); break;
            case ORC_Q4_K: int_q4_k(L, b, qx + rb * 256, dx + rb * 8, sums + rb * 8, acc, &corr); break;
            default: break;
            }
        }
        out[i] = lane_sum(acc, L) + corr;
    }
}

int orc_matvec_int(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                   const float *x, float *out, size_t begin, size_t end, int lanes) {
    if (t != ORC_Q4_0 && t != ORC_Q8_0 && t != ORC_Q4_1 && t != ORC_Q4_K) return ORC_E_UNSUPPORTED;
    int rc = check_shape(t, w_len, k, rows, begin, end);
    if (rc) return rc;
    size_t chunks = k / 32;
    /* single.zig:62-67: a too-large activation falls back to the fp body. */
    if (chunks > 2048) return orc_matvec(t, w, w_len, k, rows, x, out, begin, end, lanes);
    int8_t *qx = (int8_t *)malloc(k);
    float *dx = (float *)malloc(chunks * sizeof(float));
    int32_t *sums = (int32_t *)malloc(chunks * sizeof(int32_t));
    orc_quantize_act_q8(x, chunks, qx, dx, sums);
    switch (lanes) {
    case 4: sweep_int(4, t, w, k, qx, dx, sums, out, begin, end); break;
    case 16: sweep_int(16, t, w, k, qx, dx, sums, out, begin, end); break;
    default: sweep_int(8, t, w, k, qx, dx, sums, out, begin, end); break;
    }
    free(qx);
    free(dx);
    free(sums);
    return ORC_OK;
}

/* ---- prefill GEMM forms ------------------------------------------------ */

/*
 * batched.matVecQ4_0BatchedRows (form/batched.zig:31-82), the body both the
 * M<4 and the register-tiled M>=4 q4_0 forms run: per block, four 8-wide nibble
 * vectors, s = q0*x0, then fma(q1,x2), fma(q2,x1), fma(q3,x3); vacc = fma(d,s,vacc).
 */
static void batched_q4_0(const uint8_t *w, size_t k, size_t rows, size_t M, const float *x,
                         float *out, size_t begin, size_t end) {
    size_t nb = k / 32, rowb = nb * 18;
    for (size_t i = begin; i < end; i++) {
        float vacc[32][8];
        for (size_t t = 0; t < M; t++)
            for (int j = 0; j < 8; j++) vacc[t][j] = 0.0f;
        const uint8_t *row = w + i * rowb;
        for (size_t rb = 0; rb < nb; rb++) {
            const uint8_t *b = row + rb * 18;
            float d = rd_f16(b);
            float q0[8], q1[8], q2[8], q3[8];
            for (int j = 0; j < 8; j++) {
                q0[j] = (float)((int)(b[2 + j] & 0x0F) - 8);
                q1[j] = (float)((int)(b[2 + j] >> 4) - 8);
                q2[j] = (float)((int)(b[10 + j] & 0x0F) - 8);
                q3[j] = (float)((int)(b[10 + j] >> 4) - 8);
            }
            for (size_t t = 0; t < M; t++) {
                const float *xb = x + t * k + rb * 32;
                for (int j = 0; j < 8; j++) {
                    float s = q0[j] * xb[j];
                    s = fmaf(q1[j], xb[16 + j], s);
                    s = fmaf(q2[j], xb[8 + j], s);
                    s = fmaf(q3[j], xb[24 + j], s);
                    vacc[t][j] = fmaf(d, s, vacc[t][j]);
                }
            }
        }
        for (size_t t = 0; t < M; t++) out[t * rows + i] = lane_sum(vacc[t], 8);
    }
}

/*
 * The q8_0 batched forms (form/batched.zig:365-468): per block the 16-wide
 * r = (q0*x0 + q1*x1) * d; M>=4 tiles tokens by 4 with one accumulator each,
 * M<4 rotates four accumulators by block index and reduces (a0+a1)+(a2+a3).
 */
static void batched_q8_0(const uint8_t *w, size_t k, size_t rows, size_t M, const float *x,
                         float *out, size_t begin, size_t end) {
    size_t nb = k / 32, rowb = nb * 34;
    for (size_t i = begin; i < end; i++) {
        const uint8_t *row = w + i * rowb;
        for (size_t t = 0; t < M; t++) {
            float acc[4][16];
            for (int a = 0; a < 4; a++)
                for (int j = 0; j < 16; j++) acc[a][j] = 0.0f;
            for (size_t rb = 0; rb < nb; rb++) {
                const uint8_t *b = row + rb * 34;
                float d = rd_f16(b);
                const float *xb = x + t * k + rb * 32;
                int slot = (M >= 4) ? 0 : (int)(rb % 4);
                for (int j = 0; j < 16; j++) {
                    float r = ((float)(int8_t)b[2 + j] * xb[j] + (float)(int8_t)b[18 + j] * xb[16 + j]) * d;
                    acc[slot][j] += r;
                }
            }
            float v[16];
            if (M >= 4) {
                out[t * rows + i] = lane_sum(acc[0], 16);
            } else {
                for (int j = 0; j < 16; j++) v[j] = (acc[0][j] + acc[1][j]) + (acc[2][j] + acc[3][j]);
                out[t * rows + i] = lane_sum(v, 16);
            }
        }
    }
}

/*
 * matMulRows (single.zig:213-233): M == 1 is the GEMV; otherwise 32-token
 * sub-batches through matMulSubBatch (single.zig:258-292): q4_0 and q8_0 have
 * batched forms, q6_k is the per-token row dot, the rest per-token matVecRows.
 */
int orc_matmul_rows(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows, size_t m,
                    const float *x, float *out, size_t begin, size_t end, int lanes) {
    int rc = check_shape(t, w_len, k, rows, begin, end);
    if (rc) return rc;
    if (m == 0) return ORC_OK;
    if (m == 1) return orc_matvec(t, w, w_len, k, rows, x, out, begin, end, lanes);
    for (size_t tok = 0; tok < m; tok += 32) {
        size_t sub = (m - tok < 32) ? m - tok : 32;
        const float *xs = x + tok * k;
        float *os = out + tok * rows;
        if (t == ORC_Q4_0) {
            batched_q4_0(w, k, rows, sub, xs, os, begin, end);
        } else if (t == ORC_Q8_0) {
            batched_q8_0(w, k, rows, sub, xs, os, begin, end);
        } else {
            for (size_t s = 0; s < sub; s++) {
                rc = orc_matvec(t, w, w_len, k, rows, xs + s * k, os + s * rows, begin, end, lanes);
                if (rc) return rc;
            }
        }
    }
    return ORC_OK;
}

/*
 * The int prefill oracle: each token's activation quantized to q8 blocks and
 * run through the `.int` sweep (layout.zig:458-476, quantized.zig:49-55), the
 * arithmetic of fixtures.q4_0IntOracle (matvec/fixtures.zig:19-48) per token.
 */
int orc_matmul_int(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows, size_t m,
                   const float *x, float *out, size_t begin, size_t end, int lanes) {
    for (size_t tok = 0; tok < m; tok++) {
        int rc = orc_matvec_int(t, w, w_len, k, rows, x + tok * k, out + tok * rows, begin, end, lanes);
        if (rc) return rc;
    }
    return ORC_OK;
}

/* ---- fused gate_up ----------------------------------------------------- */

/* ActivationKind.apply (kernels/transformer/activation.zig:4-14). */
float orc_act_apply(int act, float g, float u) {
    if (act == ORC_ACT_GELU) {
        /* geluTanh (activation.zig:46-48) in f32: 0.5*x*(1+tanh(c*(x+0.044715*x^3))). */
        float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
        return (0.5f * g * (1.0f + tanhf(inner))) * u;
    }
    return (g / (1.0f + expf(-g))) * u;
}

/*
 * fusedGateUpRows (matvec/form/fused.zig:27-86), generic path: the gate and up
 * production GEMVs, then act.apply(gate, up) per row.
 */
int orc_gate_up(uint32_t t, const uint8_t *wg, const uint8_t *wu, size_t w_len, size_t k,
                size_t rows, const float *x, int act, float *out, size_t begin, size_t end,
                int lanes) {
    float *g = (float *)malloc(rows * sizeof(float));
    float *u = (float *)malloc(rows * sizeof(float));
    int rc = orc_matvec(t, wg, w_len, k, rows, x, g, begin, end, lanes);
    if (!rc) rc = orc_matvec(t, wu, w_len, k, rows, x, u, begin, end, lanes);
    if (!rc)
        for (size_t i = begin; i < end; i++) out[i] = orc_act_apply(act, g[i], u[i]);
    free(g);
    free(u);
    return rc;
}

/* ---- the CPU baseline timer -------------------------------------------- */

/* Pool.rangeOf (runtime/pool.zig:52-66): ceil-first split of `total` rows. */
void orc_range_of(size_t total, size_t parts, size_t idx, size_t *begin, size_t *end) {
    if (idx >= parts) {
        *begin = total;
        *end = total;
        return;
    }
    size_t b = 0;
    for (size_t i = 0; i < idx; i++) {
        size_t rp = parts - i, rem = total - b;
        b += (rem + rp - 1) / rp;
    }
    size_t rp = parts - idx, rem = total - b;
    *begin = b;
    *end = b + (rem + rp - 1) / rp;
}

typedef struct {
    uint32_t t;
    const uint8_t *w;
    size_t w_len, k, rows, m;
    const float *x;
    float *out;
    size_t begin, end;
    int lanes, mode; /* 0 = fp GEMV, 1 = int GEMM over m tokens */
} job_t;

static void *run_job(void *arg) {
    job_t *j = (job_t *)arg;
    if (j->mode == 0)
        orc_matvec(j->t, j->w, j->w_len, j->k, j->rows, j->x, j->out, j->begin, j->end, j->lanes);
    else
        orc_matmul_int(j->t, j->w, j->w_len, j->k, j->rows, j->m, j->x, j->out, j->begin, j->end, j->lanes);
    return NULL;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static double time_jobs(job_t base, int threads, int reps) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    job_t jobs[256];
    double best = 1e30;
    for (int r = 0; r < reps; r++) {
        double t0 = now_s();
        for (int i = 0; i < threads; i++) {
            jobs[i] = base;
            orc_range_of(base.rows, (size_t)threads, (size_t)i, &jobs[i].begin, &jobs[i].end);
            if (i > 0) pthread_create(&tid[i], NULL, run_job, &jobs[i]);
        }
        run_job(&jobs[0]);
        for (int i = 1; i < threads; i++) pthread_join(tid[i], NULL);
        double dt = now_s() - t0;
        if (dt < best) best = dt;
    }
    return best;
}

/* Min-of-`reps` wall seconds of the production sweep split over `threads`. */
double orc_time_matvec(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                       const float *x, float *out, int threads, int reps, int lanes) {
    job_t b = {t, w, w_len, k, rows, 1, x, out, 0, rows, lanes, 0};
    return time_jobs(b, threads, reps);
}

double orc_time_matmul_int(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                           size_t m, const float *x, float *out, int threads, int reps, int lanes) {
    job_t b = {t, w, w_len, k, rows, m, x, out, 0, rows, lanes, 1};
    return time_jobs(b, threads, reps);
}
