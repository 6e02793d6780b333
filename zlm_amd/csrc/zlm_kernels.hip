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
// GEMV scheme (one kernel per quant, templated on the row tile RT, the chunk
// steps per row STEPS and the x capacity KCAP):
//   * each wave owns tiles of RT rows (grid-stride over tiles); lane l covers
//     the row's 16-byte chunks l, l+64, ... (STEPS of them), and the wave
//     issues all of a tile's loads before computing any, so a tile is one
//     memory round trip;
//   * the workgroup stages x (fp32) once into LDS, padded by one float4 per 32
//     floats so 128-bit LDS reads of neighbouring lanes fall in distinct banks,
//     plus the fp32 sum of every 16-element run of x.  x's global loads are
//     issued before the first tile's weight loads and the prologue has no
//     branches, so the staging barrier waits for x alone;
//   * the x values a chunk needs are read from LDS once and applied to all RT
//     rows; the nibble/byte bias (-8 for q4_0, -32 for q6_k) is folded
//     through the run sums, so the inner loop is extract -> cvt -> fma in fp32;
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

// LDS footprint of a staged x of capacity KCAP: the padded values plus one
// dummy float4 (kDummy) and the run sums plus one dummy slot (index kRuns),
// the targets of out-of-range threads' stores.
template <int KCAP>
struct XTile {
    static constexpr int kDummy = KCAP + KCAP / 8;
    static constexpr int kFloats = kDummy + 4;
    static constexpr int kRuns = KCAP / 16;
};

// Stage x[0..k) into LDS (padded) and the sums of its 16-element runs.  x is
// read from global memory once: thread i holds float4 i, and the four
// consecutive lanes that hold one run add their partials with two shuffles.
// k is a multiple of 32 and blockDim a multiple of 64, so every loop trip is
// wave-uniform and a run never straddles two waves.
template <int KCAP>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int k, float* xl, float* xs) {
    const int n4 = k >> 2;
    for (int base = 0; base < n4; base += blockDim.x) {
        const int i = base + threadIdx.x;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < n4) {
            v = reinterpret_cast<const float4*>(x)[i];
            *reinterpret_cast<float4*>(xl + xpad(i << 2)) = v;
        }
        float s = (v.x + v.y) + (v.z + v.w);
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        if (i < n4 && (i & 3) == 0) xs[i >> 2] = s;
    }
    __syncthreads();
}

// The same staging split in two phases, so a kernel can issue x's global loads
// first, then its weight loads, and only then wait for x: loads complete in
// issue order, so x must be requested before the weights or the LDS store
// would wait for the whole weight tile.  NX = float4s of x per thread.
template <int NX>
struct XRegs {
    float4 v[NX];
};

// Both phases are branch-free (clamped loads, selects, a dummy LDS slot for
// out-of-range threads): a branch here would make the compiler wait for every
// outstanding load, weights included, before the barrier.
template <int NX>
__device__ __forceinline__ void xload(const float* __restrict__ x, int k, XRegs<NX>& r) {
    const int n4 = k >> 2;
#pragma unroll
    for (int j = 0; j < NX; j++) {
        const int i = j * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
        r.v[j] = reinterpret_cast<const float4*>(x)[min(i, n4 - 1)];
    }
}

template <int KCAP, int NX>
__device__ __forceinline__ void xstore(const XRegs<NX>& r, int k, float* xl, float* xs) {
    const int n4 = k >> 2;
#pragma unroll
    for (int j = 0; j < NX; j++) {
        const int i = j * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
        const bool valid = i < n4;
        float4 v = r.v[j];
        v.x = valid ? v.x : 0.0f;
        v.y = valid ? v.y : 0.0f;
        v.z = valid ? v.z : 0.0f;
        v.w = valid ? v.w : 0.0f;
        *reinterpret_cast<float4*>(xl + (valid ? xpad(i << 2) : XTile<KCAP>::kDummy)) = v;
        float s = (v.x + v.y) + (v.z + v.w);
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        xs[(valid && (i & 3) == 0) ? (i >> 2) : XTile<KCAP>::kRuns] = s;
    }
    __syncthreads();
}

__device__ __forceinline__ float4 lds4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// ---- per-quant fragments --------------------------------------------------
// A fragment is what one lane loads for one 16-byte chunk position `c` of RT
// rows; `load_frag` only issues global loads, `compute_frag` only touches
// registers and LDS, so the main loop can keep the next fragment's loads in
// flight while it computes the current one.

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

template <bool NT>
__device__ __forceinline__ uint4 ld16(const uint8_t* p) {
    if constexpr (NT) {
        const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
        return make_uint4(t.x, t.y, t.z, t.w);
    } else {
        return *reinterpret_cast<const uint4*>(p);
    }
}

template <bool NT>
__device__ __forceinline__ uint2 ld8(const uint8_t* p) {
    if constexpr (NT) {
        const v2u t = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(p));
        return make_uint2(t.x, t.y);
    } else {
        return *reinterpret_cast<const uint2*>(p);
    }
}

template <bool NT>
__device__ __forceinline__ uint32_t ld2(const uint16_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

template <int QT, int RT>
struct Frag;

template <int RT>
struct Frag<Q4_0, RT> {
    uint4 q[RT];
    uint32_t d[RT];
};
template <int RT>
struct Frag<Q8_0, RT> {
    uint4 q[RT];
    uint32_t d[RT];
};
template <int RT>
struct Frag<Q4_K, RT> {
    uint4 hd[RT];
    uint4 q[RT];
};
template <int RT>
struct Frag<Q6_K, RT> {
    uint4 ql[RT];
    uint4 qh[RT];
    uint2 sc[RT];
    uint32_t d[RT];
};

// q4_0: chunk c = block c (16 nibble bytes).  q8_0: chunk c = half block c
// (16 int8; block c/2 holds the scale).  q4_k / q6_k: 8 chunks per 256-element
// super-block (c>>3), see the compute steps.
template <int QT, int RT, bool NT>
__device__ __forceinline__ void load_frag(Frag<QT, RT>& f, const uint8_t* __restrict__ w,
                                          const uint16_t* __restrict__ dsc, const uint32_t* rr, uint32_t nb, int c) {
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const size_t row = rr[r];
        if constexpr (QT == Q4_0) {
            const size_t bi = row * nb + c;
            f.q[r] = ld16<NT>(w + bi * 16);
            f.d[r] = ld2<NT>(dsc + bi);
        } else if constexpr (QT == Q8_0) {
            f.q[r] = ld16<NT>(w + (row * (2 * nb) + c) * 16);
            f.d[r] = ld2<NT>(dsc + row * nb + (c >> 1));
        } else if constexpr (QT == Q4_K) {
            const uint8_t* blk = w + (row * nb + (c >> 3)) * 144;
            f.hd[r] = ld16<false>(blk);
            f.q[r] = ld16<NT>(blk + 16 + 16 * (c & 7));
        } else {
            const int p = c & 7, n = p >> 2, h = (p >> 1) & 1, ws = p & 1;
            const size_t bi = row * nb + (c >> 3);
            const uint8_t* blk = w + bi * 208;
            f.ql[r] = ld16<NT>(blk + 64 * n + 32 * ws + 16 * h);
            f.qh[r] = ld16<false>(blk + 128 + 32 * n + 16 * h);
            f.sc[r] = ld8<false>(blk + 192 + 8 * n);
            f.d[r] = ld2<false>(dsc + bi);
        }
    }
}

// Byte j of a q4_0 block holds element j (low nibble) and j+16 (high);
// value (nib-8)*d, and Sum (nib-8)*x = Sum nib*x - 8*Sum x.
template <int RT>
__device__ __forceinline__ void compute_q4_0(const Frag<Q4_0, RT>& f, const float* xl, const float* xs, int c,
                                             bool valid, float* acc) {
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
            const uint32_t wv = (&f.q[r].x)[i];
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
    for (int r = 0; r < RT; r++) acc[r] = fmaf(valid ? h2f(f.d[r]) : 0.0f, fmaf(-8.0f, xsum, s[r]), acc[r]);
}

template <int RT>
__device__ __forceinline__ void compute_q8_0(const Frag<Q8_0, RT>& f, const float* xl, const float*, int c,
                                             bool valid, float* acc) {
    const float* xb = xl + xpad(c << 4);
    float s[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) s[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = lds4(xb + 4 * i);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint32_t wv = (&f.q[r].x)[i];
            s[r] = fmaf(sb(wv, 0), xa.x, s[r]);
            s[r] = fmaf(sb(wv, 1), xa.y, s[r]);
            s[r] = fmaf(sb(wv, 2), xa.z, s[r]);
            s[r] = fmaf(sb(wv, 3), xa.w, s[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++) acc[r] = fmaf(valid ? h2f(f.d[r]) : 0.0f, s[r], acc[r]);
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

// q4_k piece p = c&7 of super-block c>>3 (16 qs bytes of group g = p/2): low
// nibbles are elements 64g + 16(p%2) + j (scale 2g), high nibbles +32 (scale
// 2g+1); value d*sc*nib - dmin*mn.
template <int RT>
__device__ __forceinline__ void compute_q4_k(const Frag<Q4_K, RT>& f, const float* xl, const float* xs, int c,
                                             bool valid, float* acc) {
    const int sbk = c >> 3, p = c & 7, g = p >> 1, h = p & 1;
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
            const uint32_t wv = (&f.q[r].x)[i];
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
        const uint32_t dd = valid ? f.hd[r].x : 0u;
        const float d = h2f(dd), dmin = h2f(dd >> 16);
        float sc1, mn1, sc2, mn2;
        scale_min_k4(2 * g, f.hd[r].y, f.hd[r].z, f.hd[r].w, sc1, mn1);
        scale_min_k4(2 * g + 1, f.hd[r].y, f.hd[r].z, f.hd[r].w, sc2, mn2);
        float t = (d * sc1) * slo[r];
        t = fmaf(d * sc2, shi[r], t);
        t = fmaf(-(dmin * mn1), xs_lo, t);
        t = fmaf(-(dmin * mn2), xs_hi, t);
        acc[r] += t;
    }
}

// q6_k part p = c&7 of super-block c>>3: half n = p/4, 16-run h, ql half ws;
// low nibbles + qh bits 2ws are elements 128n + 32ws + 16h + j, high nibbles +
// qh bits 4+2ws are those +64.  value d*sc*(q-32); Sum (q-32)*x = Sum q*x - 32*Sum x.
template <int RT>
__device__ __forceinline__ void compute_q6_k(const Frag<Q6_K, RT>& f, const float* xl, const float* xs, int c,
                                             bool valid, float* acc) {
    const int sbk = c >> 3, p = c & 7, n = p >> 2, h = (p >> 1) & 1, ws = p & 1;
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
            const uint32_t lw = (&f.ql[r].x)[i], hw = (&f.qh[r].x)[i];
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
        const float d = valid ? h2f(f.d[r]) : 0.0f;
        const float sc_a = static_cast<float>(static_cast<int32_t>(f.sc[r].x << (24 - sci)) >> 24);
        const float sc_b = static_cast<float>(static_cast<int32_t>(f.sc[r].y << (24 - sci)) >> 24);
        float t = (d * sc_a) * fmaf(-32.0f, xs_a, sa[r]);
        t = fmaf(d * sc_b, fmaf(-32.0f, xs_b, sbv[r]), t);
        acc[r] += t;
    }
}

template <int QT, int RT>
__device__ __forceinline__ void compute_frag(const Frag<QT, RT>& f, const float* xl, const float* xs, int c,
                                             bool valid, float* acc) {
    if constexpr (QT == Q4_0) compute_q4_0<RT>(f, xl, xs, c, valid, acc);
    if constexpr (QT == Q8_0) compute_q8_0<RT>(f, xl, xs, c, valid, acc);
    if constexpr (QT == Q4_K) compute_q4_k<RT>(f, xl, xs, c, valid, acc);
    if constexpr (QT == Q6_K) compute_q6_k<RT>(f, xl, xs, c, valid, acc);
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

// Issue the loads of every chunk step of row tile `t`.  Rows past the end are
// clamped to the last row and chunk positions past the row's end to its last
// chunk, so the loads are branch-free; compute_tile gives those a zero scale.
// With EXACT the caller guarantees STEPS == ceil(C/64); otherwise steps that
// start past the row's end are skipped by a wave-uniform test.
template <int QT, int RT, int STEPS, bool EXACT, bool NT>
__device__ __forceinline__ void load_tile(Frag<QT, RT> (&f)[STEPS], const uint8_t* __restrict__ w,
                                          const uint16_t* __restrict__ dsc, uint32_t t, uint32_t rows, uint32_t nb,
                                          int C, int lane) {
    uint32_t rr[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) rr[r] = min(t * RT + r, rows - 1);
#pragma unroll
    for (int s = 0; s < STEPS; s++)
        if (EXACT || s * kWave < C) load_frag<QT, RT, NT>(f[s], w, dsc, rr, nb, min(lane + s * kWave, C - 1));
}

template <int QT, int RT, int STEPS, bool EXACT>
__device__ __forceinline__ void compute_tile(const Frag<QT, RT> (&f)[STEPS], const float* xl, const float* xs,
                                             int C, int lane, float* acc) {
#pragma unroll
    for (int r = 0; r < RT; r++) acc[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
        const int c = lane + s * kWave;
        if (EXACT || s * kWave < C) compute_frag<QT, RT>(f[s], xl, xs, min(c, C - 1), c < C, acc);
    }
}

// One GEMV: y[r] = sum_k w[r,k] * x[k] for r < rows, k = nb * block_elems.
// A wave owns row tiles blockIdx*WAVES + wid + j*gridDim*WAVES.  For each tile
// it issues the loads of every chunk step (64 consecutive 16-byte chunks per
// row per step) before it computes any of them, so a tile costs one memory
// round trip.  The first tile is peeled and kept branch-free: x's loads, then
// the tile's loads, then x's LDS store and the barrier, so the barrier waits
// for x only and step s computes as soon as its own loads land.  Occupancy
// (several waves per SIMD) overlaps one wave's compute with others' loads.
template <int QT, int KCAP, int WAVES, int RT, int STEPS, bool EXACT, bool NT>
__device__ __forceinline__ void gemv(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc,
                                     const float* __restrict__ x, float* __restrict__ y, uint32_t rows,
                                     uint32_t nb) {
    __shared__ __attribute__((aligned(16))) float xl[XTile<KCAP>::kFloats];
    __shared__ float xs[XTile<KCAP>::kRuns + 1];
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wid = threadIdx.x / kWave;
    const int C = chunks_per_row<QT>(nb);
    const uint32_t ntiles = (rows + RT - 1) / RT;
    const uint32_t tstride = gridDim.x * WAVES;
    uint32_t tile = blockIdx.x * WAVES + wid;

    const int k = static_cast<int>(nb) * elems_per_block<QT>();
    XRegs<(KCAP / 4 + WAVES * kWave - 1) / (WAVES * kWave)> xr;
    xload(x, k, xr);
    Frag<QT, RT> f[STEPS];
    load_tile<QT, RT, STEPS, EXACT, NT>(f, w, dsc, min(tile, ntiles - 1), rows, nb, C, lane);
    xstore<KCAP>(xr, k, xl, xs);

    float acc[RT];
    compute_tile<QT, RT, STEPS, EXACT>(f, xl, xs, C, lane, acc);
    if (tile < ntiles) reduce_write<RT>(acc, y, tile * RT, rows, lane);
    for (tile += tstride; tile < ntiles; tile += tstride) {
        load_tile<QT, RT, STEPS, EXACT, NT>(f, w, dsc, tile, rows, nb, C, lane);
        compute_tile<QT, RT, STEPS, EXACT>(f, xl, xs, C, lane, acc);
        reduce_write<RT>(acc, y, tile * RT, rows, lane);
    }
}

// The software-pipelined form: each wave walks a flat sequence of (row tile,
// chunk step) items and issues every item's loads one item ahead of its
// compute.  Kept for launch-shape comparisons.
template <int QT, int KCAP, int WAVES, int RT, bool NT>
__device__ __forceinline__ void gemv_pipe(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc,
                                          const float* __restrict__ x, float* __restrict__ y, uint32_t rows,
                                          uint32_t nb) {
    __shared__ __attribute__((aligned(16))) float xl[XTile<KCAP>::kFloats];
    __shared__ float xs[XTile<KCAP>::kRuns + 1];
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wid = threadIdx.x / kWave;
    const int C = chunks_per_row<QT>(nb);
    const int steps = (C + kWave - 1) / kWave;
    const uint32_t ntiles = (rows + RT - 1) / RT;
    const uint32_t tstride = gridDim.x * WAVES;
    uint32_t tile = blockIdx.x * WAVES + wid;
    const uint32_t my_tiles = tile < ntiles ? (ntiles - 1 - tile) / tstride + 1 : 0;
    const uint32_t items = my_tiles * static_cast<uint32_t>(steps);

    uint32_t rr[RT];
    auto set_rows = [&](uint32_t t) {
#pragma unroll
        for (int r = 0; r < RT; r++) rr[r] = min(t * RT + r, rows - 1);
    };
    Frag<QT, RT> cur;
    if (items > 0) {
        set_rows(tile);
        load_frag<QT, RT, NT>(cur, w, dsc, rr, nb, min(lane, C - 1));
    }
    stage_x<KCAP>(x, static_cast<int>(nb) * elems_per_block<QT>(), xl, xs);

    float acc[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) acc[r] = 0.0f;
    int step = 0;
    for (uint32_t it = 0; it < items; it++) {
        // next item: same tile, next step; or the wave's next tile, step 0
        const bool last_step = (step == steps - 1);
        const uint32_t ntile = last_step ? tile + tstride : tile;
        const int nstep = last_step ? 0 : step + 1;
        Frag<QT, RT> nxt;
        if (it + 1 < items) {
            uint32_t nrr[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) nrr[r] = min(ntile * RT + r, rows - 1);
            load_frag<QT, RT, NT>(nxt, w, dsc, nrr, nb, min(lane + nstep * kWave, C - 1));
        }
        const int c = lane + step * kWave;
        compute_frag<QT, RT>(cur, xl, xs, min(c, C - 1), c < C, acc);
        if (last_step) {
            reduce_write<RT>(acc, y, tile * RT, rows, lane);
#pragma unroll
            for (int r = 0; r < RT; r++) acc[r] = 0.0f;
        }
        tile = ntile;
        step = nstep;
        cur = nxt;
    }
}

}  // namespace

// ---- GEMV entry points ---------------------------------------------------
// zlm_gemv_<quant>_r<RT>_s<STEPS>: STEPS == ceil(chunks per row / 64) exactly
// (q4_0 and the K-quants have k/32 chunks per row, q8_0 k/16), x capacity the
// smallest of 4096/8192/16384/32768 that holds STEPS steps.
// zlm_gemv_<quant>_r1_g<STEPS>: the generic form for any other k up to 32768.
// Every instance runs 4 waves (256 threads) per workgroup.

#define ZLM_GEMV(NAME, QT, KCAP, RT, STEPS, EXACT)                                                        \
    extern "C" __global__ void __launch_bounds__(256)                                                    \
        NAME(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc, const float* __restrict__ x, \
             float* __restrict__ y, uint32_t rows, uint32_t nb) {                                        \
        gemv<QT, KCAP, 4, RT, STEPS, EXACT, true>(w, dsc, x, y, rows, nb);                               \
    }

// q4_0 / q4_k / q6_k: KCAP = 2048 * STEPS rounded up to a tier.
#define ZLM_GEMV_Q4(QN, QT)                                         \
    ZLM_GEMV_Q4_COMMON(QN, QT)                                      \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s6, QT, 16384, 2, 6, true)          \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s8, QT, 16384, 2, 8, true)

// The K-quants keep RT 1 from 6 steps up (their fragments are larger).
#define ZLM_GEMV_Q4_COMMON(QN, QT)                                  \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s1, QT, 4096, 1, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s1, QT, 4096, 2, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s1, QT, 4096, 4, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s2, QT, 4096, 1, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s2, QT, 4096, 2, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s2, QT, 4096, 4, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s3, QT, 8192, 1, 3, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s3, QT, 8192, 2, 3, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s3, QT, 8192, 4, 3, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s4, QT, 8192, 1, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s4, QT, 8192, 2, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s4, QT, 8192, 4, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s6, QT, 16384, 1, 6, true)          \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s8, QT, 16384, 1, 8, true)          \
    ZLM_GEMV(zlm_gemv_##QN##_r1_g16, QT, 32768, 1, 16, false)

// q8_0: KCAP = 1024 * STEPS rounded up to a tier.
#define ZLM_GEMV_Q8(QN, QT)                                         \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s1, QT, 4096, 1, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s1, QT, 4096, 2, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s1, QT, 4096, 4, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s2, QT, 4096, 1, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s2, QT, 4096, 2, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s2, QT, 4096, 4, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s3, QT, 4096, 1, 3, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s3, QT, 4096, 2, 3, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s3, QT, 4096, 4, 3, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s4, QT, 4096, 1, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s4, QT, 4096, 2, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s4, QT, 4096, 4, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s6, QT, 8192, 1, 6, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s6, QT, 8192, 2, 6, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s8, QT, 8192, 1, 8, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s8, QT, 8192, 2, 8, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s12, QT, 16384, 1, 12, true)        \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s12, QT, 16384, 2, 12, true)        \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s15, QT, 16384, 1, 15, true)        \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s16, QT, 16384, 1, 16, true)        \
    ZLM_GEMV(zlm_gemv_##QN##_r1_g32, QT, 32768, 1, 32, false)

#ifndef ZLM_NO_ENTRY_POINTS
ZLM_GEMV_Q4(q4_0, Q4_0)
ZLM_GEMV_Q4_COMMON(q4_k, Q4_K)
ZLM_GEMV_Q4_COMMON(q6_k, Q6_K)
ZLM_GEMV_Q8(q8_0, Q8_0)
#endif

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

// Quantize one 32-element block; `x` may be null (a padding token: zeros).
__device__ __forceinline__ void quantize_block(const float* __restrict__ x, uint4* dst, float* d_out,
                                               int32_t* s_out) {
    float v[32];
    for (int i = 0; i < 8; i++) {
        const float4 t = x ? reinterpret_cast<const float4*>(x)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
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
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    *d_out = d;
    if (s_out) *s_out = s;
}

// Row-major output: qx [nblocks][32], dx and sums [nblocks].
extern "C" __global__ void __launch_bounds__(256)
    zlm_quantize_q8(const float* __restrict__ x, int8_t* __restrict__ qx, float* __restrict__ dx,
                    int32_t* __restrict__ sums, uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    quantize_block(x + b * 32, reinterpret_cast<uint4*>(qx + b * 32), dx + b, sums + b);
}

// The prefill GEMM's tiled output for m tokens of nb blocks, tokens padded to
// mt*32: qx [mt][nb][32 tokens][32 B], dx [mt][nb][32 tokens]; padding tokens
// are zeros.  One thread per (token, block).
extern "C" __global__ void __launch_bounds__(256)
    zlm_quantize_q8_tiled(const float* __restrict__ x, int8_t* __restrict__ qx, float* __restrict__ dx,
                          uint32_t m, uint32_t nb, uint32_t mt) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<uint64_t>(mt) * 32 * nb) return;
    const uint32_t t = static_cast<uint32_t>(i / nb), b = static_cast<uint32_t>(i % nb);
    const uint64_t slot = (static_cast<uint64_t>(t / 32) * nb + b) * 32 + (t % 32);
    quantize_block(t < m ? x + (static_cast<uint64_t>(t) * nb + b) * 32 : nullptr,
                   reinterpret_cast<uint4*>(qx + slot * 32), dx + slot, nullptr);
}

// The prefill GEMM's tiled Q4_0 weight layout, rows padded to rt*32:
// payload [rt][nb][32 rows][16 B], scales [rt][nb][32 rows]; padding rows have
// zero scales.  One thread per (row, block) of the padded matrix.
extern "C" __global__ void __launch_bounds__(256)
    zlm_tile_q4_0(const uint8_t* __restrict__ payload, const uint16_t* __restrict__ scales,
                  uint8_t* __restrict__ tpayload, uint16_t* __restrict__ tscales, uint32_t rows, uint32_t nb,
                  uint32_t rt) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<uint64_t>(rt) * 32 * nb) return;
    const uint32_t r = static_cast<uint32_t>(i / nb), b = static_cast<uint32_t>(i % nb);
    const uint64_t slot = (static_cast<uint64_t>(r / 32) * nb + b) * 32 + (r % 32);
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    uint16_t d = 0;
    if (r < rows) {
        q = reinterpret_cast<const uint4*>(payload)[static_cast<uint64_t>(r) * nb + b];
        d = scales[static_cast<uint64_t>(r) * nb + b];
    }
    reinterpret_cast<uint4*>(tpayload)[slot] = q;
    tscales[slot] = d;
}

// ---- device copy (16-byte granules; the traffic-counter calibration kernel) --

extern "C" __global__ void __launch_bounds__(256)
    zlm_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, uint64_t n16) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

// ---- prefill GEMM: Q4_0 weights x Q8_0-quantized activations, int8 MFMA ----
//
// out[t*rows + r] = sum_b dw[r,b] * dx[t,b] * sum_j (nib[r,b,j] - 8) * qx[t,b,j]
// (the int path of reference kernels/quantized.zig:49-55 over the activation
// quantizer of matvec/layout.zig:458-476, i.e. zlm_quantize_q8's output).
//
// v_mfma_i32_32x32x32_i8 computes one 32-element block for a 32-token x
// 32-row tile: A = activations (lane l: token l%32, block elements
// 16*(l/32)..+15 of qx), B = weights (lane l: row l%32, the same elements: the
// low nibbles of the row's 16 block bytes for lanes 0-31, the high nibbles for
// 32-63), D[t = 8*(i/4) + 4*(l/32) + i%4][r = l%32].  A nibble n enters as the
// int8 16*(n-8) (n^8 in the high nibble), so each block dot is exact in int32.
// The block's scale matrix dx[t]*dw[r]/16 is the outer product of two vectors;
// v_mfma_f32_32x32x2f32 with the vectors in k = 0 and zeros in k = 1 produces
// it in the same D layout on the matrix pipe, leaving one convert and one fma
// per output on the VALU.  A wave owns 64 tokens x 32 rows (two MFMA tiles
// share the unpacked weights) and keeps the next four blocks' loads in flight
// while it computes the current four.  A workgroup of 4 waves owns 128 tokens
// x 64 rows; padding tokens and rows of the tiled layouts are zeros and their
// outputs are not stored, blocks past the end get a zero scale.
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct GemmBlk {
    uint4 a0, a1, w;
    uint32_t d;
    float x0, x1;
};

// Depth 1 keeps the kernel at 129 VGPRs, so the 3 waves per SIMD that the
// 12288 x 512 launch places are all resident at once (depths 2-4 measured no
// faster and need 193-250 VGPRs).
#ifndef ZLM_GEMM_DEPTH
#define ZLM_GEMM_DEPTH 1
#endif
#ifndef ZLM_GEMM_WAVES_PER_EU
#define ZLM_GEMM_WAVES_PER_EU 3
#endif
constexpr int kGemmDepth = ZLM_GEMM_DEPTH;  // blocks per register set

__device__ __forceinline__ void gemm_load(GemmBlk& g, const int8_t* a0, const int8_t* a1, const uint8_t* wr,
                                          const uint16_t* dr, const float* x0, const float* x1, uint32_t b) {
    g.a0 = *reinterpret_cast<const uint4*>(a0 + static_cast<size_t>(b) * 1024);
    g.a1 = *reinterpret_cast<const uint4*>(a1 + static_cast<size_t>(b) * 1024);
    g.w = *reinterpret_cast<const uint4*>(wr + static_cast<size_t>(b) * 512);
    g.d = dr[static_cast<size_t>(b) * 32];
    g.x0 = x0[static_cast<size_t>(b) * 32];
    g.x1 = x1[static_cast<size_t>(b) * 32];
}

__device__ __forceinline__ void gemm_block(const GemmBlk& g, bool valid, bool lo_half, int sh, v16f& acc0,
                                           v16f& acc1) {
    v4i bv;
    bv.x = static_cast<int>(((g.w.x << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
    bv.y = static_cast<int>(((g.w.y << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
    bv.z = static_cast<int>(((g.w.z << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
    bv.w = static_cast<int>(((g.w.w << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
    const v4i a0 = {static_cast<int>(g.a0.x), static_cast<int>(g.a0.y), static_cast<int>(g.a0.z),
                    static_cast<int>(g.a0.w)};
    const v4i a1 = {static_cast<int>(g.a1.x), static_cast<int>(g.a1.y), static_cast<int>(g.a1.z),
                    static_cast<int>(g.a1.w)};
    const v16i zi = {};
    const v16i i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bv, zi, 0, 0, 0);
    const v16i i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bv, zi, 0, 0, 0);
    const bool use = valid && lo_half;
    const float bw = use ? h2f(g.d) : 0.0f;
    const float s0 = use ? g.x0 : 0.0f;  // the 16 of the nibble encoding is divided out at the store
    const float s1 = use ? g.x1 : 0.0f;
    const v16f zf = {};
    const v16f c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(s0, bw, zf, 0, 0, 0);
    const v16f c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(s1, bw, zf, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        acc0[i] = fmaf(c0[i], static_cast<float>(i0[i]), acc0[i]);
        acc1[i] = fmaf(c1[i], static_cast<float>(i1[i]), acc1[i]);
    }
}

// Operands come from the tiled layouts (zlm_quantize_q8_tiled, zlm_tile_q4_0),
// so each per-block load of a wave is one contiguous run: 1 KiB of qx per
// 32-token tile, 512 B of weights and 64 B of scales per 32-row tile.
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q4_0_q8(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ qx,
                     const float* __restrict__ dx, float* __restrict__ out, uint32_t rows, uint32_t m, uint32_t nb,
                     uint32_t mt) {
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    const uint32_t tok0 = blockIdx.y * 128 + 64 * (wid & 1);  // multiple of 32
    const uint32_t row0 = blockIdx.x * 64 + 32 * (wid >> 1);  // multiple of 32
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const uint32_t tt0 = min(tok0 / 32, mt - 1), tt1 = min(tok0 / 32 + 1, mt - 1);
    const uint32_t rt = min(row0 / 32, (rows + 31) / 32 - 1);  // a wave past the last tile re-reads it, stores nothing
    const int8_t* a0 = qx + static_cast<size_t>(tt0) * nb * 1024 + l32 * 32 + 16 * half;
    const int8_t* a1 = qx + static_cast<size_t>(tt1) * nb * 1024 + l32 * 32 + 16 * half;
    const uint8_t* wr = wq + static_cast<size_t>(rt) * nb * 512 + l32 * 16;
    const uint16_t* dr = wd + static_cast<size_t>(rt) * nb * 32 + l32;
    const float* x0 = dx + static_cast<size_t>(tt0) * nb * 32 + l32;
    const float* x1 = dx + static_cast<size_t>(tt1) * nb * 32 + l32;
    const int sh = half ? 0 : 4;  // lanes 0-31 take the low nibbles, 32-63 the high
    const bool lo_half = half == 0;

    v16f acc0 = {}, acc1 = {};
    // Two register sets, A and B, alternate: one set's loads are in flight
    // while the other's blocks are computed.  The scheduling barriers keep each
    // set's loads ahead of the compute (the scheduler would otherwise sink them
    // next to their uses), and the ping-pong needs no register copies.
    GemmBlk A[kGemmDepth], B[kGemmDepth];
#pragma unroll
    for (int p = 0; p < kGemmDepth; p++) gemm_load(A[p], a0, a1, wr, dr, x0, x1, min(static_cast<uint32_t>(p), nb - 1));
    for (uint32_t b = 0; b < nb; b += 2 * kGemmDepth) {
#pragma unroll
        for (int p = 0; p < kGemmDepth; p++)
            gemm_load(B[p], a0, a1, wr, dr, x0, x1, min(b + kGemmDepth + p, nb - 1));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < kGemmDepth; p++) gemm_block(A[p], b + p < nb, lo_half, sh, acc0, acc1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < kGemmDepth; p++)
            gemm_load(A[p], a0, a1, wr, dr, x0, x1, min(b + 2 * kGemmDepth + p, nb - 1));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < kGemmDepth; p++) gemm_block(B[p], b + kGemmDepth + p < nb, lo_half, sh, acc0, acc1);
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t r = row0 + l32;
    if (r < rows) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t t = tok0 + 8 * (i / 4) + 4 * half + (i % 4);
            if (t < m) out[static_cast<size_t>(t) * rows + r] = acc0[i] * 0.0625f;
            if (t + 32 < m) out[static_cast<size_t>(t + 32) * rows + r] = acc1[i] * 0.0625f;
        }
    }
}

