// zlm_kernels.hip -- CDNA4 (gfx950) kernels for zlm's quantized GEMV/GEMM path.
//
// Built as a device-only code object (hipcc --genco) and loaded by the host
// library with hipModuleLoad; every entry point is extern "C" so the host can
// look it up by name.
//
// Weight layouts in HBM (produced once by the repack kernels from the raw GGUF
// blocks of reference src/kernels/linear/quant/types.zig:6-53):
//   q4_0  payload [rows][nb][16 B nibbles]        + scales [rows][nb] f16
//   q8_0  payload [rows][nb][32 B int8]           + scales [rows][nb] f16
//   q6_k  payload [rows][nb][208 B ql|qh|sc]      + scales [rows][nb] f16
//   q4_k  raw     [rows][nb][144 B]  (already a multiple of 16 B per block)
// Every payload block is a whole number of 16-byte chunks, so the GEMV
// streams it with 128-bit loads; a wavefront's 64 lanes read 1 KiB of
// consecutive payload per load instruction.
//
// GEMV scheme (one kernel per quant, templated on the row tile RT, the x
// capacity KCAP and the waves per workgroup):
//   * the workgroup stages x (fp32) once into LDS, padded by one float4 per 32
//     floats so 128-bit LDS reads of neighbouring lanes fall in distinct banks,
//     plus the fp32 sum of every 16-element run of x;
//   * each wave owns a tile of RT rows (grid-stride over tiles); lane l walks
//     the row's 16-byte chunks l, l+64, ...; the x values a chunk needs are read
//     from LDS once and applied to all RT rows;
//   * the nibble/byte bias (-8 for q4_0, -32 for q6_k) is folded through the
//     run sums, so the inner loop is extract -> cvt -> fma on fp32;
//   * the RT per-lane partials are reduced with a transposing butterfly (each
//     shuffle stage halves the live values), one lane per row writes y.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kWave = 64;

enum QType : int { Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q6_K = 14 };

__device__ __forceinline__ float h2f(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits & 0xffffu)));
}

__device__ __forceinline__ float ub(uint32_t w, int i) { return static_cast<float>((w >> (8 * i)) & 0xffu); }
__device__ __forceinline__ float sb(uint32_t w, int i) {
    return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * i)) >> 24);
}

// LDS position of x element e: one float4 of padding after every 32 floats.
__device__ __forceinline__ int xpad(int e) { return e + ((e >> 5) << 2); }

template <int KCAP>
struct XTile {
    static constexpr int kFloats = KCAP + KCAP / 8;
    static constexpr int kRuns = KCAP / 16;
};

// Stage x[0..k) into LDS (padded) and the sums of its 16-element runs.
template <int KCAP>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int k, float* xl, float* xs) {
    const int n4 = k >> 2;
    for (int i = threadIdx.x; i < n4; i += blockDim.x) {
        float4 v = reinterpret_cast<const float4*>(x)[i];
        *reinterpret_cast<float4*>(xl + xpad(i << 2)) = v;
    }
    const int nrun = k >> 4;
    for (int r = threadIdx.x; r < nrun; r += blockDim.x) {
        const float4* p = reinterpret_cast<const float4*>(x + (r << 4));
        float4 a = p[0], b = p[1], c = p[2], d = p[3];
        xs[r] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) +
                (((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w)));
    }
    __syncthreads();
}

__device__ __forceinline__ float4 lds4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// ---- per-quant chunk steps ------------------------------------------------

// q4_0: chunk c = block c (16 nibble bytes). Byte j holds element j (low) and
// j+16 (high); value (nib-8)*d.  Sum_j (nib-8)*x = Sum nib*x - 8*Sum x.
template <int RT>
__device__ __forceinline__ void step_q4_0(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc,
                                          const float* xl, const float* xs, const uint32_t* rr, uint32_t nb,
                                          int c, float* acc) {
    uint4 q[RT];
    float d[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const size_t bi = static_cast<size_t>(rr[r]) * nb + c;
        q[r] = reinterpret_cast<const uint4*>(w)[bi];
        d[r] = h2f(dsc[bi]);
    }
    const float* xb = xl + xpad(c << 5);
    const float xsum = xs[2 * c] + xs[2 * c + 1];
    float s[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) s[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = lds4(xb + 4 * i);
        const float4 xh = lds4(xb + 16 + 4 * i);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint32_t wv = (&q[r].x)[i];
            const uint32_t lo = wv & 0x0F0F0F0Fu, hi = (wv >> 4) & 0x0F0F0F0Fu;
            s[r] = fmaf(ub(lo, 0), xa.x, s[r]);
            s[r] = fmaf(ub(lo, 1), xa.y, s[r]);
            s[r] = fmaf(ub(lo, 2), xa.z, s[r]);
            s[r] = fmaf(ub(lo, 3), xa.w, s[r]);
            s[r] = fmaf(ub(hi, 0), xh.x, s[r]);
            s[r] = fmaf(ub(hi, 1), xh.y, s[r]);
            s[r] = fmaf(ub(hi, 2), xh.z, s[r]);
            s[r] = fmaf(ub(hi, 3), xh.w, s[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++) acc[r] = fmaf(d[r], fmaf(-8.0f, xsum, s[r]), acc[r]);
}

// q8_0: chunk c = half block (16 int8); block c/2 carries the scale.
template <int RT>
__device__ __forceinline__ void step_q8_0(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc,
                                          const float* xl, const float* xs, const uint32_t* rr, uint32_t nb,
                                          int c, float* acc) {
    uint4 q[RT];
    float d[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const size_t row = rr[r];
        q[r] = reinterpret_cast<const uint4*>(w)[row * (2 * nb) + c];
        d[r] = h2f(dsc[row * nb + (c >> 1)]);
    }
    const float* xb = xl + xpad(c << 4);
    float s[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) s[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = lds4(xb + 4 * i);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint32_t wv = (&q[r].x)[i];
            s[r] = fmaf(sb(wv, 0), xa.x, s[r]);
            s[r] = fmaf(sb(wv, 1), xa.y, s[r]);
            s[r] = fmaf(sb(wv, 2), xa.z, s[r]);
            s[r] = fmaf(sb(wv, 3), xa.w, s[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++) acc[r] = fmaf(d[r], s[r], acc[r]);
}

// getScaleMinK4 (reference quant/k_quants.zig:24-32) on the 12 packed bytes
// held as three dwords; j in 0..7, any lane-varying j.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, float& sc, float& mn) {
    const int t = (j & 3) * 8;
    const uint32_t b0 = (s0 >> t) & 0xffu, b1 = (s1 >> t) & 0xffu, b2 = (s2 >> t) & 0xffu;
    uint32_t d, m;
    if (j < 4) {
        d = b0 & 63u;
        m = b1 & 63u;
    } else {
        d = (b2 & 15u) | ((b0 >> 6) << 4);
        m = (b2 >> 4) | ((b1 >> 6) << 4);
    }
    sc = static_cast<float>(d);
    mn = static_cast<float>(m);
}

// q4_k: 8 lanes per 256-element super-block. Piece p (16 qs bytes) of group
// g = p/2: low nibbles are elements 64g + 16(p%2) + j (scale 2g), high nibbles
// elements +32 (scale 2g+1).  value = d*sc*nib - dmin*mn.
template <int RT>
__device__ __forceinline__ void step_q4_k(const uint8_t* __restrict__ w, const uint16_t* __restrict__,
                                          const float* xl, const float* xs, const uint32_t* rr, uint32_t nb,
                                          int c, float* acc) {
    const int sbk = c >> 3, p = c & 7, g = p >> 1, h = p & 1;
    uint4 hd[RT], q[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const uint8_t* blk = w + (static_cast<size_t>(rr[r]) * nb + sbk) * 144;
        hd[r] = *reinterpret_cast<const uint4*>(blk);
        q[r] = *reinterpret_cast<const uint4*>(blk + 16 + 16 * p);
    }
    const int elo = 256 * sbk + 64 * g + 16 * h, ehi = elo + 32;
    const float* xa_p = xl + xpad(elo);
    const float* xb_p = xl + xpad(ehi);
    const float xs_lo = xs[elo >> 4], xs_hi = xs[ehi >> 4];
    float slo[RT], shi[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) slo[r] = shi[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = lds4(xa_p + 4 * i);
        const float4 xb = lds4(xb_p + 4 * i);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint32_t wv = (&q[r].x)[i];
            const uint32_t lo = wv & 0x0F0F0F0Fu, hi = (wv >> 4) & 0x0F0F0F0Fu;
            slo[r] = fmaf(ub(lo, 0), xa.x, slo[r]);
            slo[r] = fmaf(ub(lo, 1), xa.y, slo[r]);
            slo[r] = fmaf(ub(lo, 2), xa.z, slo[r]);
            slo[r] = fmaf(ub(lo, 3), xa.w, slo[r]);
            shi[r] = fmaf(ub(hi, 0), xb.x, shi[r]);
            shi[r] = fmaf(ub(hi, 1), xb.y, shi[r]);
            shi[r] = fmaf(ub(hi, 2), xb.z, shi[r]);
            shi[r] = fmaf(ub(hi, 3), xb.w, shi[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const float d = h2f(hd[r].x), dmin = h2f(hd[r].x >> 16);
        float sc1, mn1, sc2, mn2;
        scale_min_k4(2 * g, hd[r].y, hd[r].z, hd[r].w, sc1, mn1);
        scale_min_k4(2 * g + 1, hd[r].y, hd[r].z, hd[r].w, sc2, mn2);
        float t = (d * sc1) * slo[r];
        t = fmaf(d * sc2, shi[r], t);
        t = fmaf(-(dmin * mn1), xs_lo, t);
        t = fmaf(-(dmin * mn2), xs_hi, t);
        acc[r] += t;
    }
}

// q6_k: 8 lanes per super-block. Lane part p: half n = p/4, 16-run h, and
// which ql half (ws): low nibbles + qh bits (2ws) -> elements
// 128n + 32ws + 16h + j, high nibbles + qh bits (4+2ws) -> +64.
// value = d*sc*(q-32); Sum (q-32)*x = Sum q*x - 32*Sum x.
template <int RT>
__device__ __forceinline__ void step_q6_k(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc,
                                          const float* xl, const float* xs, const uint32_t* rr, uint32_t nb,
                                          int c, float* acc) {
    const int sbk = c >> 3, p = c & 7, n = p >> 2, h = (p >> 1) & 1, ws = p & 1;
    uint4 ql[RT], qh[RT];
    uint2 scp[RT];
    float d[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const size_t bi = static_cast<size_t>(rr[r]) * nb + sbk;
        const uint8_t* blk = w + bi * 208;
        ql[r] = *reinterpret_cast<const uint4*>(blk + 64 * n + 32 * ws + 16 * h);
        qh[r] = *reinterpret_cast<const uint4*>(blk + 128 + 32 * n + 16 * h);
        scp[r] = *reinterpret_cast<const uint2*>(blk + 192 + 8 * n);
        d[r] = h2f(dsc[bi]);
    }
    const int ea = 256 * sbk + 128 * n + 32 * ws + 16 * h, eb = ea + 64;
    const float* xa_p = xl + xpad(ea);
    const float* xb_p = xl + xpad(eb);
    const float xs_a = xs[ea >> 4], xs_b = xs[eb >> 4];
    const int sh_lo = 2 * ws, sh_hi = 4 + 2 * ws, sci = 8 * (h + 2 * ws);
    float sa[RT], sbv[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) sa[r] = sbv[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = lds4(xa_p + 4 * i);
        const float4 xb = lds4(xb_p + 4 * i);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint32_t lw = (&ql[r].x)[i], hw = (&qh[r].x)[i];
            const uint32_t lo = (lw & 0x0F0F0F0Fu) | (((hw >> sh_lo) & 0x03030303u) << 4);
            const uint32_t hi = ((lw >> 4) & 0x0F0F0F0Fu) | (((hw >> sh_hi) & 0x03030303u) << 4);
            sa[r] = fmaf(ub(lo, 0), xa.x, sa[r]);
            sa[r] = fmaf(ub(lo, 1), xa.y, sa[r]);
            sa[r] = fmaf(ub(lo, 2), xa.z, sa[r]);
            sa[r] = fmaf(ub(lo, 3), xa.w, sa[r]);
            sbv[r] = fmaf(ub(hi, 0), xb.x, sbv[r]);
            sbv[r] = fmaf(ub(hi, 1), xb.y, sbv[r]);
            sbv[r] = fmaf(ub(hi, 2), xb.z, sbv[r]);
            sbv[r] = fmaf(ub(hi, 3), xb.w, sbv[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const float sc_a = static_cast<float>(static_cast<int32_t>(scp[r].x << (24 - sci)) >> 24);
        const float sc_b = static_cast<float>(static_cast<int32_t>(scp[r].y << (24 - sci)) >> 24);
        float t = (d[r] * sc_a) * fmaf(-32.0f, xs_a, sa[r]);
        t = fmaf(d[r] * sc_b, fmaf(-32.0f, xs_b, sbv[r]), t);
        acc[r] += t;
    }
}

// Reduce RT per-lane partials over the wavefront and write y[r0 .. r0+RT).
// Stage s exchanges across lane bit (5-s) and keeps half of the live values,
// so RT values cost RT-1 + (6-log2 RT) shuffles instead of 6*RT.
template <int RT>
__device__ __forceinline__ void reduce_write(float* v, float* __restrict__ y, uint32_t r0, uint32_t rows,
                                             int lane) {
    constexpr int LOG = (RT >= 8) ? 3 : (RT >= 4) ? 2 : (RT >= 2) ? 1 : 0;
#pragma unroll
    for (int st = 0; st < LOG; st++) {
        const int half = (RT >> st) >> 1;
        const int bit = 32 >> st;
        const bool upper = (lane & bit) != 0;
#pragma unroll
        for (int i = 0; i < half; i++) {
            const float keep = upper ? v[half + i] : v[i];
            const float send = upper ? v[i] : v[half + i];
            v[i] = keep + __shfl_xor(send, bit, kWave);
        }
    }
    float s = v[0];
#pragma unroll
    for (int off = 32 >> LOG; off >= 1; off >>= 1) s += __shfl_xor(s, off, kWave);
    if ((lane & ((64 >> LOG) - 1)) == 0) {
        const uint32_t row = r0 + (lane >> (6 - LOG));
        if (row < rows) y[row] = s;
    }
}

template <int QT>
__device__ __forceinline__ int chunks_per_row(uint32_t nb) {
    return (QT == Q4_0) ? static_cast<int>(nb) : (QT == Q8_0) ? static_cast<int>(2 * nb) : static_cast<int>(8 * nb);
}

template <int QT>
__device__ __forceinline__ int elems_per_block() {
    return (QT == Q4_0 || QT == Q8_0) ? 32 : 256;
}

template <int QT, int RT>
__device__ __forceinline__ void step(const uint8_t* w, const uint16_t* dsc, const float* xl, const float* xs,
                                     const uint32_t* rr, uint32_t nb, int c, float* acc) {
    if constexpr (QT == Q4_0) step_q4_0<RT>(w, dsc, xl, xs, rr, nb, c, acc);
    if constexpr (QT == Q8_0) step_q8_0<RT>(w, dsc, xl, xs, rr, nb, c, acc);
    if constexpr (QT == Q4_K) step_q4_k<RT>(w, dsc, xl, xs, rr, nb, c, acc);
    if constexpr (QT == Q6_K) step_q6_k<RT>(w, dsc, xl, xs, rr, nb, c, acc);
}

// One GEMV: y[r] = sum_k w[r,k] * x[k] for r < rows, k = nb * block_elems.
template <int QT, int KCAP, int WAVES, int RT>
__device__ __forceinline__ void gemv(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc,
                                     const float* __restrict__ x, float* __restrict__ y, uint32_t rows,
                                     uint32_t nb) {
    __shared__ __attribute__((aligned(16))) float xl[XTile<KCAP>::kFloats];
    __shared__ float xs[XTile<KCAP>::kRuns];
    const int k = static_cast<int>(nb) * elems_per_block<QT>();
    stage_x<KCAP>(x, k, xl, xs);
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wid = threadIdx.x / kWave;
    const uint32_t ntiles = (rows + RT - 1) / RT;
    const int C = chunks_per_row<QT>(nb);
    for (uint32_t tile = blockIdx.x * WAVES + wid; tile < ntiles; tile += gridDim.x * WAVES) {
        const uint32_t r0 = tile * RT;
        uint32_t rr[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) rr[r] = min(r0 + r, rows - 1);
        float acc[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) acc[r] = 0.0f;
#pragma unroll 2
        for (int c = lane; c < C; c += kWave) step<QT, RT>(w, dsc, xl, xs, rr, nb, c, acc);
        reduce_write<RT>(acc, y, r0, rows, lane);
    }
}

}  // namespace

// ---- GEMV entry points: zlm_gemv_<quant>_k<KCAP>_w<WAVES>_r<RT> ----------

#define ZLM_GEMV(QN, QT, KCAP, WAVES, RT)                                                                 \
    extern "C" __global__ void __launch_bounds__(WAVES * 64)                                             \
        zlm_gemv_##QN##_k##KCAP##_w##WAVES##_r##RT(const uint8_t* __restrict__ w,                         \
                                                    const uint16_t* __restrict__ dsc,                     \
                                                    const float* __restrict__ x, float* __restrict__ y,   \
                                                    uint32_t rows, uint32_t nb) {                         \
        gemv<QT, KCAP, WAVES, RT>(w, dsc, x, y, rows, nb);                                               \
    }

#define ZLM_GEMV_ALL_K(QN, QT, RT) \
    ZLM_GEMV(QN, QT, 4096, 4, RT)  \
    ZLM_GEMV(QN, QT, 8192, 4, RT)  \
    ZLM_GEMV(QN, QT, 16384, 8, RT) \
    ZLM_GEMV(QN, QT, 32768, 8, RT)

#define ZLM_GEMV_QUANT(QN, QT) \
    ZLM_GEMV_ALL_K(QN, QT, 2)  \
    ZLM_GEMV_ALL_K(QN, QT, 4)  \
    ZLM_GEMV_ALL_K(QN, QT, 8)

ZLM_GEMV_QUANT(q4_0, Q4_0)
ZLM_GEMV_QUANT(q8_0, Q8_0)
ZLM_GEMV_QUANT(q4_k, Q4_K)
ZLM_GEMV_QUANT(q6_k, Q6_K)

// ---- repack: raw GGUF blocks -> aligned payload + separate f16 scales -----
// One thread per block; `bb` raw block bytes, the scale at `soff` within the
// raw block, the payload is the remaining bytes in order.

extern "C" __global__ void __launch_bounds__(256)
    zlm_repack_split(const uint8_t* __restrict__ raw, uint8_t* __restrict__ payload, uint16_t* __restrict__ dsc,
                     uint64_t nblocks, uint32_t bb, uint32_t soff) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* src = raw + b * bb;
    const uint32_t pb = bb - 2;
    uint8_t* dst = payload + b * pb;
    dsc[b] = static_cast<uint16_t>(src[soff] | (static_cast<uint16_t>(src[soff + 1]) << 8));
    uint32_t o = 0;
    for (uint32_t i = 0; i < bb; i++) {
        if (i == soff || i == soff + 1) continue;
        dst[o++] = src[i];
    }
}

// ---- dequant from the device layout (bit-exact vs the CPU codecs) ---------
// One thread per block; `out` receives block_elems floats per block.

#pragma clang fp contract(off)

extern "C" __global__ void __launch_bounds__(256)
    zlm_dequant_q4_0(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc, float* __restrict__ out,
                     uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* q = w + b * 16;
    const float d = h2f(dsc[b]);
    float* o = out + b * 32;
    for (int j = 0; j < 16; j++) {
        o[j] = static_cast<float>(static_cast<int>(q[j] & 15) - 8) * d;
        o[16 + j] = static_cast<float>(static_cast<int>(q[j] >> 4) - 8) * d;
    }
}

extern "C" __global__ void __launch_bounds__(256)
    zlm_dequant_q8_0(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc, float* __restrict__ out,
                     uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const int8_t* q = reinterpret_cast<const int8_t*>(w + b * 32);
    const float d = h2f(dsc[b]);
    float* o = out + b * 32;
    for (int j = 0; j < 32; j++) o[j] = static_cast<float>(q[j]) * d;
}

extern "C" __global__ void __launch_bounds__(256)
    zlm_dequant_q4_k(const uint8_t* __restrict__ w, const uint16_t* __restrict__, float* __restrict__ out,
                     uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* blk = w + b * 144;
    const uint32_t* hd = reinterpret_cast<const uint32_t*>(blk);
    const float d = h2f(hd[0]), dmin = h2f(hd[0] >> 16);
    float* o = out + b * 256;
    for (int g = 0; g < 4; g++) {
        float sc1, mn1, sc2, mn2;
        scale_min_k4(2 * g, hd[1], hd[2], hd[3], sc1, mn1);
        scale_min_k4(2 * g + 1, hd[1], hd[2], hd[3], sc2, mn2);
        const float d1 = d * sc1, m1 = dmin * mn1, d2 = d * sc2, m2 = dmin * mn2;
        const uint8_t* q = blk + 16 + 32 * g;
        for (int l = 0; l < 32; l++) {
            o[64 * g + l] = __builtin_fmaf(static_cast<float>(q[l] & 15), d1, -m1);
            o[64 * g + 32 + l] = __builtin_fmaf(static_cast<float>(q[l] >> 4), d2, -m2);
        }
    }
}

extern "C" __global__ void __launch_bounds__(256)
    zlm_dequant_q6_k(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc, float* __restrict__ out,
                     uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* blk = w + b * 208;
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192);
    const float d = h2f(dsc[b]);
    float* o = out + b * 256;
    for (int n = 0; n < 2; n++) {
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const uint8_t a = ql[64 * n + l], a2 = ql[64 * n + l + 32], hb = qh[32 * n + l];
            const int q1 = (a & 15) | (((hb >> 0) & 3) << 4);
            const int q2 = (a2 & 15) | (((hb >> 2) & 3) << 4);
            const int q3 = (a >> 4) | (((hb >> 4) & 3) << 4);
            const int q4 = (a2 >> 4) | (((hb >> 6) & 3) << 4);
            o[128 * n + l] = static_cast<float>(q1 - 32) * (d * static_cast<float>(sc[8 * n + is + 0]));
            o[128 * n + l + 32] = static_cast<float>(q2 - 32) * (d * static_cast<float>(sc[8 * n + is + 2]));
            o[128 * n + l + 64] = static_cast<float>(q3 - 32) * (d * static_cast<float>(sc[8 * n + is + 4]));
            o[128 * n + l + 96] = static_cast<float>(q4 - 32) * (d * static_cast<float>(sc[8 * n + is + 6]));
        }
    }
}

// ---- activation quantizer (reference matvec/layout.zig:458-476) -----------
// One thread per 32-element block: d = amax/127 (f32, correctly rounded),
// inv = d != 0 ? 1/d : 0, q = round-half-away(v*inv) clamped to +-127.

extern "C" __global__ void __launch_bounds__(256)
    zlm_quantize_q8(const float* __restrict__ x, int8_t* __restrict__ qx, float* __restrict__ dx,
                    int32_t* __restrict__ sums, uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float4* xb = reinterpret_cast<const float4*>(x + b * 32);
    float v[32];
    for (int i = 0; i < 8; i++) {
        const float4 t = xb[i];
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = __fdiv_rn(amax, 127.0f);
    const float inv = (d != 0.0f) ? __fdiv_rn(1.0f, d) : 0.0f;
    int32_t s = 0;
    uint32_t packed[8];
    for (int i = 0; i < 8; i++) {
        uint32_t wv = 0;
        for (int j = 0; j < 4; j++) {
            int32_t q = static_cast<int32_t>(roundf(v[4 * i + j] * inv));
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            s += q;
            wv |= (static_cast<uint32_t>(q) & 0xffu) << (8 * j);
        }
        packed[i] = wv;
    }
    uint4* dst = reinterpret_cast<uint4*>(qx + b * 32);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    dx[b] = d;
    sums[b] = s;
}
