// gemv_impl.h -- shared device code of the gfx950 GEMV kernels (included by
// each zlm_gemv_<quant>.hip instance file and by zlm_kernels.hip).
//
// Weight layouts in HBM (produced once by the repack kernels from the raw GGUF
// blocks of reference src/kernels/linear/quant/types.zig:6-53):
//   q4_0  payload [rows][nb][16 B nibbles]        + scales [rows][nb] f16
//   q4_1  payload [rows][nb][16 B nibbles]        + scales [rows][nb] (f16 d, f16 m)
//   q8_0  payload [rows][nb][32 B int8]           + scales [rows][nb] f16
//   q6_k  payload [rows][nb][128 B ql]            + records [rows][nb][84 B]:
//         bytes 8p..8p+7 = the qh bits of chunk p (see q6_k_rows), 64..65 =
//         f16 d, 68+2p / 69+2p = the chunk's two int8 scales; see
//         zlm_repack_q6_k
//   q4_k  payload [rows][nb][128 B qs]            + records [rows][nb][20 B]:
//         dword 0 = f16 d | f16 dmin << 16, dword 1+g (g = 0..3) = the 6-bit
//         scales and mins of sub-blocks 2g, 2g+1 decoded to bytes
//         (sc[2g], sc[2g+1], mn[2g], mn[2g+1]); see zlm_repack_q4_k
//   f32 / f16 / bf16  raw [rows][k] (k a multiple of 32, so rows stay 16-byte
//         aligned; the kernels count nb = k/32 "blocks" of 32 elements)
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
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kWave = 64;

// GGML type codes (reference gguf/format.zig:41-77).
enum QType : int { F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q8_0 = 8, Q4_K = 12, Q6_K = 14, BF16 = 30 };

constexpr bool is_float_type(int qt) { return qt == F32 || qt == F16 || qt == BF16; }

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

// Staging of x[0..k) into LDS (padded) plus the sums of its 16-element runs,
// in two phases, so a kernel can issue x's global loads first, then its weight
// loads, and only then wait for x: loads complete in issue order, so x must be
// requested before the weights or the LDS store would wait for the whole
// weight tile.  Thread i holds float4 i (+ j*blockDim); the four consecutive
// lanes that hold one run add their partials with two shuffles.  k is a
// multiple of 32 and blockDim a multiple of 64, so a run never straddles two
// waves.  NX = float4s of x per thread.
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

// With XQ the LDS tile holds x in three int8 planes instead of fp32: per
// 32-element block a power-of-two scale s = 2^(5-e) (e = exponent of the
// block's amax, so |x*s| < 64), q0 = rint(x*s), q1 = rint(128*(x*s - q0)),
// q2 = rint(128*(128*(x*s - q0) - q1)); x = (q0 + q1/128 + q2/16384) / s to
// within amax * 2^-20.  Plane p is KCAP bytes at byte offset p*KCAP of the
// tile, then the per-block 1/s (KCAP/32 floats); the dummy slot takes
// out-of-range threads' stores.  The 8 lanes that hold one block's float4s
// share its amax with three shuffles.
template <int KCAP>
struct XQTile {
    static constexpr int kScales = 3 * KCAP / 4;         // float index of 1/s
    static constexpr int kDummy = kScales + KCAP / 32;   // float index of the dummy slot
    static_assert(kDummy + 4 <= XTile<KCAP>::kFloats, "the int8 planes fit the fp32 tile");
};

// The block exponent e of a block whose largest magnitude is am.
__device__ __forceinline__ int xq_exp(float am) {
    const int eb = static_cast<int>((__builtin_bit_cast(uint32_t, am) >> 23) & 0xffu);
    return min(max(eb - 127, -122), 127);
}

// The three int8 planes of four x values at block scale s, one byte each.
__device__ __forceinline__ void xq_planes(float4 v, float s, uint32_t& p0, uint32_t& p1, uint32_t& p2) {
    const float t[4] = {v.x * s, v.y * s, v.z * s, v.w * s};
    p0 = p1 = p2 = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float q0 = rintf(t[j]);
        const float u = (t[j] - q0) * 128.0f;
        const float q1 = rintf(u);
        const float q2 = rintf((u - q1) * 128.0f);
        p0 |= (static_cast<uint32_t>(static_cast<int>(q0)) & 0xffu) << (8 * j);
        p1 |= (static_cast<uint32_t>(static_cast<int>(q1)) & 0xffu) << (8 * j);
        p2 |= (static_cast<uint32_t>(static_cast<int>(q2)) & 0xffu) << (8 * j);
    }
}

// The q8 activation quantizer (reference matvec/layout.zig:458-476) over a
// 32-element block held as one float4 by each of 8 consecutive lanes: amax of
// the block, d = amax/127, 1/d correctly rounded, q = round-half-away(v/d)
// clamped to +-127.  Returns the lane's four q bytes (element order), the
// block's d and the sum of the lane's four q.  Every lane of the 8 must call
// it (the amax is shared with shuffles).
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, __shfl_xor(v, 1, kWave));
    v = fmaxf(v, __shfl_xor(v, 2, kWave));
    return fmaxf(v, __shfl_xor(v, 4, kWave));
}
__device__ __forceinline__ int32_t sum8(int32_t v) {
    v += __shfl_xor(v, 1, kWave);
    v += __shfl_xor(v, 2, kWave);
    return v + __shfl_xor(v, 4, kWave);
}
__device__ __forceinline__ uint32_t q8_quant4(float4 v, float& d, int32_t& s) {
    const float amax = max8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    d = __fdiv_rn(amax, 127.0f);
    const float inv = (d != 0.0f) ? __fdiv_rn(1.0f, d) : 0.0f;
    const float e[4] = {v.x, v.y, v.z, v.w};
    s = 0;
    uint32_t wv = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int32_t q = static_cast<int32_t>(roundf(e[j] * inv));
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        s += q;
        wv |= (static_cast<uint32_t>(q) & 0xffu) << (8 * j);
    }
    return wv;
}

template <int KCAP, bool XQ>
__device__ __forceinline__ void xput(float4 v, int i, bool valid, float* xl) {
    if constexpr (!XQ) {
        *reinterpret_cast<float4*>(xl + (valid ? xpad(i << 2) : XTile<KCAP>::kDummy)) = v;
    } else {
        float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        am = fmaxf(am, __shfl_xor(am, 1, kWave));
        am = fmaxf(am, __shfl_xor(am, 2, kWave));
        am = fmaxf(am, __shfl_xor(am, 4, kWave));
        const int e = xq_exp(am);
        uint32_t p0, p1, p2;
        xq_planes(v, ldexpf(1.0f, 5 - e), p0, p1, p2);
        uint32_t* w = reinterpret_cast<uint32_t*>(xl);
        const int slot = valid ? i : XQTile<KCAP>::kDummy;
        w[slot] = p0;
        w[valid ? KCAP / 4 + i : XQTile<KCAP>::kDummy + 1] = p1;
        w[valid ? KCAP / 2 + i : XQTile<KCAP>::kDummy + 2] = p2;
        xl[(valid && (i & 7) == 0) ? XQTile<KCAP>::kScales + (i >> 3) : XQTile<KCAP>::kDummy + 3] =
            ldexpf(1.0f, e - 5);
    }
}

template <int KCAP, int NX, bool XQ = false, bool SYNC = true>
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
        xput<KCAP, XQ>(v, i, valid, xl);
        float s = (v.x + v.y) + (v.z + v.w);
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        xs[(valid && (i & 3) == 0) ? (i >> 2) : XTile<KCAP>::kRuns] = s;
    }
    if constexpr (SYNC) __syncthreads();
}

// xstore with RMSNorm folded in (reference kernels/transformer/norm.zig:26-37:
// out = x * (1/sqrt(mean(x^2) + eps)) * w).  LDS receives x*w; the scalar
// 1/sqrt(mean(x^2)+eps) is returned and applied to the row sums, so the norm
// costs no pass of its own.  Every workgroup reduces the same per-wave partials
// in the same order, so all of them use the same scale.  `red` holds one float
// per wave.
template <int KCAP, int NX, int WAVES, bool XQ = false>
__device__ __forceinline__ float xstore_norm(const XRegs<NX>& r, const XRegs<NX>& g, int k, float eps, float* xl,
                                             float* xs, float* red) {
    const int n4 = k >> 2;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NX; j++) {
        const int i = j * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
        const bool valid = i < n4;
        float4 v = r.v[j];
        v.x = valid ? v.x : 0.0f;
        v.y = valid ? v.y : 0.0f;
        v.z = valid ? v.z : 0.0f;
        v.w = valid ? v.w : 0.0f;
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
        v.x *= g.v[j].x;
        v.y *= g.v[j].y;
        v.z *= g.v[j].z;
        v.w *= g.v[j].w;
        xput<KCAP, XQ>(v, i, valid, xl);
        float s = (v.x + v.y) + (v.z + v.w);
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        xs[(valid && (i & 3) == 0) ? (i >> 2) : XTile<KCAP>::kRuns] = s;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; w++) tot += red[w];
    return 1.0f / sqrtf(tot / static_cast<float>(k) + eps);
}

__device__ __forceinline__ float4 lds4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ __forceinline__ float wave_sum_all(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// ---- per-quant fragments --------------------------------------------------
// A fragment is what one lane loads for one 16-byte chunk position `c` of RT
// rows; `load_frag` only issues global loads, `compute_frag` only touches
// registers and LDS, so the main loop can keep the next fragment's loads in
// flight while it computes the current one.

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef unsigned int v2u_a4 __attribute__((ext_vector_type(2), aligned(4)));  // 8 bytes at a 4-byte boundary

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

// 8 bytes from a 4-byte aligned address (the q6_k records have an 84-byte stride).
template <bool NT>
__device__ __forceinline__ uint2 ld8_a4(const uint8_t* p) {
    const v2u_a4 t = NT ? __builtin_nontemporal_load(reinterpret_cast<const v2u_a4*>(p))
                        : *reinterpret_cast<const v2u_a4*>(p);
    return make_uint2(t.x, t.y);
}

template <bool NT>
__device__ __forceinline__ uint32_t ld4(const uint32_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
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
struct Frag<Q4_1, RT> {
    uint4 q[RT];
    uint32_t dm[RT];  // f16 d (low half), f16 m (high half)
};
template <int RT>
struct Frag<F32, RT> {
    uint4 q[RT];
};
template <int RT>
struct Frag<F16, RT> {
    uint4 q[RT];
};
template <int RT>
struct Frag<BF16, RT> {
    uint4 q[RT];
};
template <int RT>
struct Frag<Q4_K, RT> {
    uint32_t dm[RT];  // f16 d | f16 dmin << 16
    uint32_t sm[RT];  // bytes sc[2g], sc[2g+1], mn[2g], mn[2g+1] of the chunk's group g
    uint4 q[RT];
};
template <int RT>
struct Frag<Q6_K, RT> {
    uint4 ql[RT];
    uint2 qh[RT];     // the chunk's 32 2-bit high parts, two per byte pair (see q6_k_rows)
    uint32_t sc[RT];  // bytes 2(p&1), 2(p&1)+1: the chunk's two int8 scales
    uint32_t d[RT];   // f16 d in the low half
};

// q4_0 / q4_1: chunk c = block c (16 nibble bytes).  q8_0: chunk c = half
// block c (16 int8; block c/2 holds the scale).  q4_k / q6_k: 8 chunks per
// 256-element super-block (c>>3), see the compute steps.  f32: chunk c =
// elements 4c..4c+3; f16 / bf16: elements 8c..8c+7.
// The rows a wave tile covers: for each of its RT fragment rows, the matrix
// (payload and scales) and the row index.  A plain tile is RT consecutive rows
// of one matrix; a pair tile (fused gate_up) is RT/2 rows of the gate matrix
// followed by the same RT/2 rows of the up matrix.
template <int RT>
struct TileRows {
    const uint8_t* w[RT];
    const uint16_t* d[RT];
    uint32_t r[RT];
};

template <int QT, int RT, bool NT>
__device__ __forceinline__ void load_frag(Frag<QT, RT>& f, const TileRows<RT>& tr, uint32_t nb, int c) {
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const uint8_t* __restrict__ w = tr.w[r];
        const uint16_t* __restrict__ dsc = tr.d[r];
        const size_t row = tr.r[r];
        if constexpr (QT == Q4_0) {
            const size_t bi = row * nb + c;
            f.q[r] = ld16<NT>(w + bi * 16);
            f.d[r] = ld2<NT>(dsc + bi);
        } else if constexpr (QT == Q4_1) {
            const size_t bi = row * nb + c;
            f.q[r] = ld16<NT>(w + bi * 16);
            f.dm[r] = ld4<NT>(reinterpret_cast<const uint32_t*>(dsc) + bi);
        } else if constexpr (QT == F32) {
            f.q[r] = ld16<NT>(w + (row * (8 * static_cast<size_t>(nb)) + c) * 16);
        } else if constexpr (QT == F16 || QT == BF16) {
            f.q[r] = ld16<NT>(w + (row * (4 * static_cast<size_t>(nb)) + c) * 16);
        } else if constexpr (QT == Q8_0) {
            f.q[r] = ld16<NT>(w + (row * (2 * nb) + c) * 16);
            f.d[r] = ld2<NT>(dsc + row * nb + (c >> 1));
        } else if constexpr (QT == Q4_K) {
            const size_t bi = row * nb + (c >> 3);
            const uint32_t* rec = reinterpret_cast<const uint32_t*>(dsc) + bi * 5;
            f.dm[r] = ld4<false>(rec);
            f.sm[r] = ld4<false>(rec + 1 + ((c & 7) >> 1));
            f.q[r] = ld16<NT>(w + bi * 128 + 16 * (c & 7));
        } else {
            const int p = c & 7, n = p >> 2, h = (p >> 1) & 1, ws = p & 1;
            const size_t bi = row * nb + (c >> 3);
            f.ql[r] = ld16<NT>(w + bi * 128 + (64 * n + 32 * ws + 16 * h));
            const uint8_t* rec = reinterpret_cast<const uint8_t*>(dsc) + bi * 84;
            f.qh[r] = ld8_a4<NT>(rec + 8 * p);
            f.d[r] = ld4<false>(reinterpret_cast<const uint32_t*>(rec + 64));
            f.sc[r] = ld4<false>(reinterpret_cast<const uint32_t*>(rec + 68 + 4 * (p >> 1)));
        }
    }
}

// Byte j of a q4_0 block holds element j (low nibble) and j+16 (high);
// value (nib-8)*d, and Sum (nib-8)*x = Sum nib*x - 8*Sum x.  x through
// accessors (xa(i) / xh(i): float4 i of elements 0..15 / 16..31), so the
// LDS-staged and the register-held x share the math.
template <int RT, class XA, class XH>
__device__ __forceinline__ void q4_0_rows(const Frag<Q4_0, RT>& f, XA xa_at, XH xh_at, float xsum, bool valid,
                                          float* acc) {
    float s[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) s[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = xa_at(i);
        const float4 xh = xh_at(i);
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
__device__ __forceinline__ void compute_q4_0(const Frag<Q4_0, RT>& f, const float* xl, const float* xs, int c,
                                             bool valid, float* acc) {
    const float* xb = xl + xpad(c << 5);
    q4_0_rows<RT>(
        f, [&](int i) { return lds4(xb + 4 * i); }, [&](int i) { return lds4(xb + 16 + 4 * i); },
        xs[2 * c] + xs[2 * c + 1], valid, acc);
}

// Byte j of a q4_1 block holds element j (low nibble) and j+16 (high); value
// nib*d + m, and Sum (nib*d + m)*x = d*Sum nib*x + m*Sum x (the reference's
// fpBlock splits it the same way: quantized.zig:71-77).
template <int RT>
__device__ __forceinline__ void compute_q4_1(const Frag<Q4_1, RT>& f, const float* xl, const float* xs, int c,
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
    for (int r = 0; r < RT; r++) {
        const uint32_t dm = valid ? f.dm[r] : 0u;
        acc[r] = fmaf(h2f(dm), s[r], fmaf(h2f(dm >> 16), xsum, acc[r]));
    }
}

// Raw float rows: f32 chunk = 4 elements, f16 / bf16 chunk = 8 (bf16 is the
// top half of an f32, reference bfloat.zig:24-34).
__device__ __forceinline__ float bf16lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

template <int QT, int RT>
__device__ __forceinline__ void compute_float(const Frag<QT, RT>& f, const float* xl, int c, bool valid, float* acc) {
    if constexpr (QT == F32) {
        const float4 xa = lds4(xl + xpad(c << 2));
#pragma unroll
        for (int r = 0; r < RT; r++) {
            float s = __builtin_bit_cast(float, f.q[r].x) * xa.x;
            s = fmaf(__builtin_bit_cast(float, f.q[r].y), xa.y, s);
            s = fmaf(__builtin_bit_cast(float, f.q[r].z), xa.z, s);
            s = fmaf(__builtin_bit_cast(float, f.q[r].w), xa.w, s);
            acc[r] += valid ? s : 0.0f;
        }
    } else {
        const float* xb = xl + xpad(c << 3);
        const float4 xa = lds4(xb), xc = lds4(xb + 4);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint32_t w0 = f.q[r].x, w1 = f.q[r].y, w2 = f.q[r].z, w3 = f.q[r].w;
            float s;
            if constexpr (QT == F16) {
                s = h2f(w0) * xa.x;
                s = fmaf(h2f(w0 >> 16), xa.y, s);
                s = fmaf(h2f(w1), xa.z, s);
                s = fmaf(h2f(w1 >> 16), xa.w, s);
                s = fmaf(h2f(w2), xc.x, s);
                s = fmaf(h2f(w2 >> 16), xc.y, s);
                s = fmaf(h2f(w3), xc.z, s);
                s = fmaf(h2f(w3 >> 16), xc.w, s);
            } else {
                s = bf16lo(w0) * xa.x;
                s = fmaf(bf16hi(w0), xa.y, s);
                s = fmaf(bf16lo(w1), xa.z, s);
                s = fmaf(bf16hi(w1), xa.w, s);
                s = fmaf(bf16lo(w2), xc.x, s);
                s = fmaf(bf16hi(w2), xc.y, s);
                s = fmaf(bf16lo(w3), xc.z, s);
                s = fmaf(bf16hi(w3), xc.w, s);
            }
            acc[r] += valid ? s : 0.0f;
        }
    }
}

// q4_0 against the int8 planes (XQ) of one block position for RT rows: per
// plane the 32 nibble-times-q products by v_dot4_i32_i8 (nibbles 0..15 are
// valid int8), the planes combined in fp32, the nibble bias -8 through the
// block's fp32 x sum.  pl / ph: planes of elements 0..15 / 16..31; d1 = 1/s.
template <int RT>
__device__ __forceinline__ void q4_0_xq_rows(const Frag<Q4_0, RT>& f, const uint4 (&pl)[3], const uint4 (&ph)[3],
                                             float d1, float xsum, bool valid, float* acc) {
#pragma unroll
    for (int r = 0; r < RT; r++) {
        int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t wv = (&f.q[r].x)[i];
            const int lo = static_cast<int>(wv & 0x0F0F0F0Fu), hi = static_cast<int>((wv >> 4) & 0x0F0F0F0Fu);
            s0 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&pl[0].x)[i]), s0, false);
            s0 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&ph[0].x)[i]), s0, false);
            s1 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&pl[1].x)[i]), s1, false);
            s1 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&ph[1].x)[i]), s1, false);
            s2 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&pl[2].x)[i]), s2, false);
            s2 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&ph[2].x)[i]), s2, false);
        }
        const float v =
            fmaf(static_cast<float>(s2), 1.0f / 16384.0f, fmaf(static_cast<float>(s1), 1.0f / 128.0f, static_cast<float>(s0)));
        acc[r] = fmaf(valid ? h2f(f.d[r]) : 0.0f, fmaf(v, d1, -8.0f * xsum), acc[r]);
    }
}

// q4_0 against the XQ planes of the LDS tile (block c).
template <int RT, int KCAP>
__device__ __forceinline__ void compute_q4_0_xq(const Frag<Q4_0, RT>& f, const float* xl, const float* xs, int c,
                                                bool valid, float* acc) {
    const int8_t* xq = reinterpret_cast<const int8_t*>(xl);
    const float d1 = xl[XQTile<KCAP>::kScales + c];
    const float xsum = xs[2 * c] + xs[2 * c + 1];
    uint4 pl[3], ph[3];
#pragma unroll
    for (int p = 0; p < 3; p++) {
        pl[p] = *reinterpret_cast<const uint4*>(xq + p * KCAP + 32 * c);
        ph[p] = *reinterpret_cast<const uint4*>(xq + p * KCAP + 32 * c + 16);
    }
    q4_0_xq_rows<RT>(f, pl, ph, d1, xsum, valid, acc);
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

// q4_k piece p = c&7 of super-block c>>3 (16 qs bytes of group g = p/2): low
// nibbles are elements 64g + 16(p%2) + j (scale 2g), high nibbles +32 (scale
// 2g+1); value d*sc*nib - dmin*mn, the four 6-bit factors bytes of the
// fragment's sm dword.  The math takes x through accessors
// (xa(i) / xb(i): float4 i of the low / high run, xs_lo / xs_hi: the runs'
// sums), so the LDS-staged and the register-held x share it.
template <int QT>
__device__ __forceinline__ void kquant_runs(int c, int& e_lo, int& e_hi) {
    const int sbk = c >> 3, p = c & 7;
    if constexpr (QT == Q4_K) {
        e_lo = 256 * sbk + 64 * (p >> 1) + 16 * (p & 1);
        e_hi = e_lo + 32;
    } else {
        e_lo = 256 * sbk + 128 * (p >> 2) + 32 * (p & 1) + 16 * ((p >> 1) & 1);
        e_hi = e_lo + 64;
    }
}

template <int RT, class XA, class XB>
__device__ __forceinline__ void q4_k_rows(const Frag<Q4_K, RT>& f, int c, XA xa_at, XB xb_at, float xs_lo,
                                          float xs_hi, bool valid, float* acc) {
    float slo[RT], shi[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) slo[r] = shi[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = xa_at(i);
        const float4 xb = xb_at(i);
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
        const uint32_t dd = valid ? f.dm[r] : 0u;
        const float d = h2f(dd), dmin = h2f(dd >> 16);
        const float sc1 = ub(f.sm[r], 0), sc2 = ub(f.sm[r], 1), mn1 = ub(f.sm[r], 2), mn2 = ub(f.sm[r], 3);
        float t = (d * sc1) * slo[r];
        t = fmaf(d * sc2, shi[r], t);
        t = fmaf(-(dmin * mn1), xs_lo, t);
        t = fmaf(-(dmin * mn2), xs_hi, t);
        acc[r] += t;
    }
}

template <int RT>
__device__ __forceinline__ void compute_q4_k(const Frag<Q4_K, RT>& f, const float* xl, const float* xs, int c,
                                             bool valid, float* acc) {
    int elo, ehi;
    kquant_runs<Q4_K>(c, elo, ehi);
    const float* xa_p = xl + xpad(elo);
    const float* xb_p = xl + xpad(ehi);
    q4_k_rows<RT>(
        f, c, [&](int i) { return lds4(xa_p + 4 * i); }, [&](int i) { return lds4(xb_p + 4 * i); }, xs[elo >> 4],
        xs[ehi >> 4], valid, acc);
}

// q6_k part p = c&7 of super-block c>>3: half n = p/4, 16-run h, ql half ws;
// low nibbles of the 16 ql bytes are elements 128n + 32ws + 16h + j (scale
// byte 0 of the pair), high nibbles are those +64 (scale byte 1).  The high
// two bits of ql dword i sit in qh dword i/2 (zlm_repack_q6_k): byte b holds
// the low-nibble element's bits at 0-1 and the high-nibble element's at 2-3
// for even i, at 4-5 and 6-7 for odd i, so one shift and one mask put them at
// bits 4-5 of each byte (bits shifted in from neighbouring bytes fall outside
// the mask).  value d*sc*(q-32); Sum (q-32)*x = Sum q*x - 32*Sum x.  x through
// accessors as for q4_k.
template <int RT, class XA, class XB>
__device__ __forceinline__ void q6_k_rows(const Frag<Q6_K, RT>& f, int c, XA xa_at, XB xb_at, float xs_a,
                                          float xs_b, bool valid, float* acc) {
    const int sh = 16 * (c & 1);  // the scale pair's bit offset in f.sc
    float sa[RT], sbv[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) sa[r] = sbv[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = xa_at(i);
        const float4 xb = xb_at(i);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint32_t lw = (&f.ql[r].x)[i], hw = (&f.qh[r].x)[i >> 1];
            const uint32_t lo = (lw & 0x0F0F0F0Fu) | (((i & 1) ? hw : (hw << 4)) & 0x30303030u);
            const uint32_t hi = ((lw >> 4) & 0x0F0F0F0Fu) | (((i & 1) ? (hw >> 2) : (hw << 2)) & 0x30303030u);
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
        const float sc_a = static_cast<float>(static_cast<int32_t>(f.sc[r] << (24 - sh)) >> 24);
        const float sc_b = static_cast<float>(static_cast<int32_t>(f.sc[r] << (16 - sh)) >> 24);
        float t = (d * sc_a) * fmaf(-32.0f, xs_a, sa[r]);
        t = fmaf(d * sc_b, fmaf(-32.0f, xs_b, sbv[r]), t);
        acc[r] += t;
    }
}

template <int RT>
__device__ __forceinline__ void compute_q6_k(const Frag<Q6_K, RT>& f, const float* xl, const float* xs, int c,
                                             bool valid, float* acc) {
    int ea, eb;
    kquant_runs<Q6_K>(c, ea, eb);
    const float* xa_p = xl + xpad(ea);
    const float* xb_p = xl + xpad(eb);
    q6_k_rows<RT>(
        f, c, [&](int i) { return lds4(xa_p + 4 * i); }, [&](int i) { return lds4(xb_p + 4 * i); }, xs[ea >> 4],
        xs[eb >> 4], valid, acc);
}

// The K-quants against the int8 planes (XQ): a piece's two 16-element runs
// each take three 16-byte plane slices and their block's 1/s; the 6-bit
// (q6_k, 0..63) or 4-bit (q4_k) quants are valid int8, so each run's
// sum q*x is three v_dot4_i32_i8 chains combined in fp32, the biases and
// mins through the fp32 run sums as in the fp32 path.
struct XqRuns {
    uint4 pa[3];  // planes of the low run
    uint4 pb[3];  // planes of the high run
    float d1a;    // 1/s of the low run's block
    float d1b;
    float sa;     // fp32 sums of the runs
    float sb;
};

__device__ __forceinline__ float xq_combine(int s0, int s1, int s2, float d1) {
    return fmaf(static_cast<float>(s2), 1.0f / 16384.0f, fmaf(static_cast<float>(s1), 1.0f / 128.0f, static_cast<float>(s0))) *
           d1;
}

template <int RT>
__device__ __forceinline__ void q4_k_xq_rows(const Frag<Q4_K, RT>& f, int c, const XqRuns& x, bool valid, float* acc) {
#pragma unroll
    for (int r = 0; r < RT; r++) {
        int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t wv = (&f.q[r].x)[i];
            const int lo = static_cast<int>(wv & 0x0F0F0F0Fu), hi = static_cast<int>((wv >> 4) & 0x0F0F0F0Fu);
            a0 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&x.pa[0].x)[i]), a0, false);
            a1 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&x.pa[1].x)[i]), a1, false);
            a2 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&x.pa[2].x)[i]), a2, false);
            b0 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&x.pb[0].x)[i]), b0, false);
            b1 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&x.pb[1].x)[i]), b1, false);
            b2 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&x.pb[2].x)[i]), b2, false);
        }
        const uint32_t dd = valid ? f.dm[r] : 0u;
        const float d = h2f(dd), dmin = h2f(dd >> 16);
        const float sc1 = ub(f.sm[r], 0), sc2 = ub(f.sm[r], 1), mn1 = ub(f.sm[r], 2), mn2 = ub(f.sm[r], 3);
        float t = (d * sc1) * xq_combine(a0, a1, a2, x.d1a);
        t = fmaf(d * sc2, xq_combine(b0, b1, b2, x.d1b), t);
        t = fmaf(-(dmin * mn1), x.sa, t);
        t = fmaf(-(dmin * mn2), x.sb, t);
        acc[r] += t;
    }
}

template <int RT>
__device__ __forceinline__ void q6_k_xq_rows(const Frag<Q6_K, RT>& f, int c, const XqRuns& x, bool valid, float* acc) {
    const int sh = 16 * (c & 1);
#pragma unroll
    for (int r = 0; r < RT; r++) {
        int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lw = (&f.ql[r].x)[i], hw = (&f.qh[r].x)[i >> 1];
            const int lo = static_cast<int>((lw & 0x0F0F0F0Fu) | (((i & 1) ? hw : (hw << 4)) & 0x30303030u));
            const int hi = static_cast<int>(((lw >> 4) & 0x0F0F0F0Fu) | (((i & 1) ? (hw >> 2) : (hw << 2)) & 0x30303030u));
            a0 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&x.pa[0].x)[i]), a0, false);
            a1 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&x.pa[1].x)[i]), a1, false);
            a2 = __builtin_amdgcn_sdot4(lo, static_cast<int>((&x.pa[2].x)[i]), a2, false);
            b0 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&x.pb[0].x)[i]), b0, false);
            b1 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&x.pb[1].x)[i]), b1, false);
            b2 = __builtin_amdgcn_sdot4(hi, static_cast<int>((&x.pb[2].x)[i]), b2, false);
        }
        const float d = valid ? h2f(f.d[r]) : 0.0f;
        const float sc_a = static_cast<float>(static_cast<int32_t>(f.sc[r] << (24 - sh)) >> 24);
        const float sc_b = static_cast<float>(static_cast<int32_t>(f.sc[r] << (16 - sh)) >> 24);
        float t = (d * sc_a) * fmaf(-32.0f, x.sa, xq_combine(a0, a1, a2, x.d1a));
        t = fmaf(d * sc_b, fmaf(-32.0f, x.sb, xq_combine(b0, b1, b2, x.d1b)), t);
        acc[r] += t;
    }
}

// The XQ runs of K-quant piece c from the LDS tile.
template <int QT, int KCAP>
__device__ __forceinline__ XqRuns xq_runs_lds(const float* xl, const float* xs, int c) {
    int ea, eb;
    kquant_runs<QT>(c, ea, eb);
    const int8_t* xq = reinterpret_cast<const int8_t*>(xl);
    XqRuns x;
#pragma unroll
    for (int p = 0; p < 3; p++) {
        x.pa[p] = *reinterpret_cast<const uint4*>(xq + p * KCAP + ea);
        x.pb[p] = *reinterpret_cast<const uint4*>(xq + p * KCAP + eb);
    }
    x.d1a = xl[XQTile<KCAP>::kScales + (ea >> 5)];
    x.d1b = xl[XQTile<KCAP>::kScales + (eb >> 5)];
    x.sa = xs[ea >> 4];
    x.sb = xs[eb >> 4];
    return x;
}

template <int QT, int RT, int KCAP = 0, bool XQ = false>
__device__ __forceinline__ void compute_frag(const Frag<QT, RT>& f, const float* xl, const float* xs, int c,
                                             bool valid, float* acc) {
    static_assert(!XQ || QT == Q4_0 || QT == Q4_K || QT == Q6_K,
                  "the int8-plane x is implemented for q4_0, q4_k and q6_k");
    if constexpr (QT == Q4_0 && XQ) compute_q4_0_xq<RT, KCAP>(f, xl, xs, c, valid, acc);
    if constexpr (QT == Q4_0 && !XQ) compute_q4_0<RT>(f, xl, xs, c, valid, acc);
    if constexpr (QT == Q4_1) compute_q4_1<RT>(f, xl, xs, c, valid, acc);
    if constexpr (is_float_type(QT)) compute_float<QT, RT>(f, xl, c, valid, acc);
    if constexpr (QT == Q8_0) compute_q8_0<RT>(f, xl, xs, c, valid, acc);
    if constexpr (QT == Q4_K && XQ) q4_k_xq_rows<RT>(f, c, xq_runs_lds<Q4_K, KCAP>(xl, xs, c), valid, acc);
    if constexpr (QT == Q4_K && !XQ) compute_q4_k<RT>(f, xl, xs, c, valid, acc);
    if constexpr (QT == Q6_K && XQ) q6_k_xq_rows<RT>(f, c, xq_runs_lds<Q6_K, KCAP>(xl, xs, c), valid, acc);
    if constexpr (QT == Q6_K && !XQ) compute_q6_k<RT>(f, xl, xs, c, valid, acc);
}

// Prologue / epilogue forms of the GEMV (template parameters PRO and EPI).
//   PRO_PLAIN  x staged as is
//   PRO_NORM   RMSNorm(x, xw, eps) folded in (xstore_norm)
//   PRO_TOK2   two tokens: x holds two k-float rows, each staged in its own
//              LDS tile; every weight fragment is loaded once and summed
//              against both (with EPI_TOK)
//   EPI_PLAIN  y[r] = row sum
//   EPI_RESID  y[r] = res[r] + row sum (res may alias y: one lane reads and
//              writes each row)
//   EPI_PAIR   fused gate_up: y[r] = act(gate row r . x, up row r . x)
//   EPI_TOK    several tokens: y[t * rows + r] = row r . x_t for t < m
enum : int { PRO_PLAIN = 0, PRO_NORM = 1, PRO_TOK2 = 2 };
enum : int { EPI_PLAIN = 0, EPI_RESID = 1, EPI_PAIR = 2, EPI_TOK = 3 };

// Kernel arguments of every GEMV form, passed by value.
struct GemvArgs {
    const uint8_t* w0;   // payload (the gate matrix for EPI_PAIR)
    const uint16_t* d0;  // split f16 scales (q4_k: the 20-byte records)
    const uint8_t* w1;   // EPI_PAIR: the up matrix
    const uint16_t* d1;
    const float* x;
    const float* xw;     // PRO_NORM: the norm weight, k floats
    float* y;
    const float* res;    // EPI_RESID
    uint32_t rows;       // output rows
    uint32_t nb;         // blocks per row
    float eps;           // PRO_NORM
    uint32_t act;        // EPI_PAIR: 0 silu, 1 gelu_tanh (reference GateUpAct)
    uint32_t m;          // EPI_TOK: tokens (rows of x and of y)
};

// ActivationKind.apply (reference kernels/transformer/activation.zig:8-13).
__device__ __forceinline__ float gate_act(uint32_t act, float g, float u) {
    if (act == 1u) {
        const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
        return (0.5f * g * (1.0f + tanhf(inner))) * u;
    }
    return (g / (1.0f + expf(-g))) * u;
}

template <int RT, bool PAIR>
__device__ __forceinline__ TileRows<RT> tile_rows(const GemvArgs& a, uint32_t t) {
    constexpr int RP = PAIR ? RT / 2 : RT;
    TileRows<RT> tr;
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const bool second = PAIR && r >= RP;
        tr.w[r] = second ? a.w1 : a.w0;
        tr.d[r] = second ? a.d1 : a.d0;
        tr.r[r] = min(t * RP + static_cast<uint32_t>(r % RP), a.rows - 1);
    }
    return tr;
}

// `lower` in the lanes whose bit BIT (32, 16 or 8) is clear, `upper` where
// it is set: a DPP move whose row mask (BIT 32, 16) or bank mask (BIT 8)
// enables exactly those lanes.
template <int BIT>
__device__ __forceinline__ float lane_pick(float lower, float upper) {
    static_assert(BIT == 32 || BIT == 16 || BIT == 8, "row or bank granularity");
    constexpr int row = BIT == 32 ? 0xC : BIT == 16 ? 0xA : 0xF;
    constexpr int bank = BIT == 8 ? 0xC : 0xF;
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, lower),
                                                                 __builtin_bit_cast(int, upper), 0xE4, row, bank,
                                                                 false));
}

// Stage ST of reduce_store's butterfly over RT values: exchange across lane
// bit 5-ST and keep half of the live values.  From RT = 8 the lane choice is
// lane_pick: as selects between array elements the compiler turned the
// pair into one load at a lane-dependent index and kept the array in
// scratch memory.
template <int RT, int ST>
__device__ __forceinline__ void butterfly_stage(float* v, int lane) {
    constexpr int half = (RT >> ST) >> 1;
    constexpr int bit = 32 >> ST;
#pragma unroll
    for (int i = 0; i < half; i++) {
        float keep, send;
        if constexpr (RT >= 8) {
            keep = lane_pick<bit>(v[i], v[half + i]);
            send = lane_pick<bit>(v[half + i], v[i]);
        } else {
            const bool upper = (lane & bit) != 0;
            keep = upper ? v[half + i] : v[i];
            send = upper ? v[i] : v[half + i];
        }
        v[i] = keep + __shfl_xor(send, bit, kWave);
    }
}

// Reduce RT per-lane partials over the wavefront and store the tile's rows.
// Stage s exchanges across lane bit (5-s) and keeps half of the live values,
// so RT values cost RT-1 + (6-log2 RT) shuffles instead of 6*RT.  Afterwards
// fragment row i's sum sits in lanes [i*64/RT, (i+1)*64/RT); for a pair tile
// the up row of gate row i is row i + RT/2, i.e. 32 lanes up.
template <int RT, int EPI, int NTOK = 1>
__device__ __forceinline__ void reduce_store(float* v, const GemvArgs& a, uint32_t t, float scale, int lane) {
    constexpr int LOG = (RT >= 8) ? 3 : (RT >= 4) ? 2 : (RT >= 2) ? 1 : 0;
    static_assert(RT <= 8, "at most 8 values per lane");
    if constexpr (LOG >= 1) butterfly_stage<RT, 0>(v, lane);
    if constexpr (LOG >= 2) butterfly_stage<RT, 1>(v, lane);
    if constexpr (LOG >= 3) butterfly_stage<RT, 2>(v, lane);
    float s = v[0];
#pragma unroll
    for (int off = 32 >> LOG; off >= 1; off >>= 1) s += __shfl_xor(s, off, kWave);
    s *= scale;
    const uint32_t fr = static_cast<uint32_t>(lane >> (6 - LOG));  // fragment row of this lane
    const bool leader = (lane & ((64 >> LOG) - 1)) == 0;
    if constexpr (EPI == EPI_PAIR) {
        static_assert(RT >= 2, "a pair tile holds a gate and an up row");
        const float u = __shfl_xor(s, 32, kWave);
        const uint32_t row = t * (RT / 2) + fr;
        if (leader && fr < static_cast<uint32_t>(RT / 2) && row < a.rows) a.y[row] = gate_act(a.act, s, u);
    } else if constexpr (EPI == EPI_TOK) {
        // RT values per lane: token 0's RT/NTOK rows, then token 1's, ...
        static_assert(NTOK >= 2 && RT % NTOK == 0, "a token tile holds a value per token");
        constexpr uint32_t RH = RT / NTOK;
        const uint32_t row = t * RH + fr % RH, tok = fr / RH;
        if (leader && row < a.rows && tok < a.m) a.y[tok * a.rows + row] = s;
    } else {
        const uint32_t row = t * RT + fr;
        if (leader && row < a.rows) {
            if constexpr (EPI == EPI_RESID) a.y[row] = a.res[row] + s;
            else a.y[row] = s;
        }
    }
}

// The row of fragment-row group `fr` of tile t and, for EPI_RESID, the
// residual value its lanes add (loaded together with the tile's weights, so
// waiting for the weights covers it).
template <int RT, int EPI>
__device__ __forceinline__ uint32_t store_row(const GemvArgs& a, uint32_t t, int lane) {
    constexpr int LOG = (RT >= 8) ? 3 : (RT >= 4) ? 2 : (RT >= 2) ? 1 : 0;
    const uint32_t fr = static_cast<uint32_t>(lane >> (6 - LOG));
    const uint32_t row = (EPI == EPI_PAIR) ? t * (RT / 2) + (fr % (RT / 2 > 0 ? RT / 2 : 1)) : t * RT + fr;
    return min(row, a.rows - 1);
}

// reduce_store for the prefetching loop: the same butterfly, then every lane
// stores its fragment row's value to the row clamped into range, with no
// branch.  A store behind a branch makes the compiler wait for every
// outstanding load (the next tile's included) before the next tile's compute;
// an unconditional one keeps the load counter exact.  Lanes of one row store
// the same value; a fragment row past the end (clamped to the last row) is a
// duplicate of the last row in the same wave and store instruction, so it
// stores that row's value too.  For EPI_PAIR both halves of the wave form
// act(gate, up) (the up half swaps its operands) and store it.
template <int RT, int EPI>
__device__ __forceinline__ void reduce_store_all(float* v, const GemvArgs& a, uint32_t t, float scale, int lane,
                                                 float rv) {
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
    s *= scale;
    const uint32_t row = store_row<RT, EPI>(a, t, lane);
    float val;
    if constexpr (EPI == EPI_PAIR) {
        static_assert(RT >= 2, "a pair tile holds a gate and an up row");
        const float o = __shfl_xor(s, 32, kWave);
        const bool lo = lane < 32;
        val = gate_act(a.act, lo ? s : o, lo ? o : s);
    } else if constexpr (EPI == EPI_RESID) {
        val = rv + s;
    } else {
        val = s;
    }
    a.y[row] = val;
}

template <int QT>
__device__ __forceinline__ int chunks_per_row(uint32_t nb) {
    if constexpr (QT == Q4_0 || QT == Q4_1) return static_cast<int>(nb);
    if constexpr (QT == Q8_0) return static_cast<int>(2 * nb);
    if constexpr (QT == F16 || QT == BF16) return static_cast<int>(4 * nb);
    return static_cast<int>(8 * nb);  // q4_k, q6_k, f32
}

template <int QT>
__device__ __forceinline__ int elems_per_block() {
    return (QT == Q4_K || QT == Q6_K) ? 256 : 32;
}

// Issue the loads of chunk group `cb` (chunks cb + lane + 64*s, s < STEPS) of
// a row tile.  Rows past the end are clamped to the last row (tile_rows) and
// chunk positions past the row's end to its last chunk, so the loads are
// branch-free; compute_group gives those a zero scale.  With EXACT the caller
// guarantees STEPS == ceil(C/64) (one group); otherwise steps that start past
// the row's end are skipped by a wave-uniform test.
template <int QT, int RT, int STEPS, bool EXACT, bool NT>
__device__ __forceinline__ void load_group(Frag<QT, RT> (&f)[STEPS], const TileRows<RT>& tr, uint32_t nb, int C,
                                           int cb, int lane) {
#pragma unroll
    for (int s = 0; s < STEPS; s++)
        if (EXACT || cb + s * kWave < C) load_frag<QT, RT, NT>(f[s], tr, nb, min(cb + lane + s * kWave, C - 1));
}

// FENCE: a scheduling barrier after each step keeps the compiler from
// hoisting later steps' LDS reads (which costs registers, hence occupancy).
template <int QT, int RT, int STEPS, bool EXACT, bool FENCE = false, int KCAP = 0, bool XQ = false>
__device__ __forceinline__ void compute_group(const Frag<QT, RT> (&f)[STEPS], const float* xl, const float* xs,
                                              int C, int cb, int lane, float* acc) {
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
        const int c = cb + lane + s * kWave;
        if (EXACT || cb + s * kWave < C) compute_frag<QT, RT, KCAP, XQ>(f[s], xl, xs, min(c, C - 1), c < C, acc);
        if constexpr (FENCE) __builtin_amdgcn_sched_barrier(0);
    }
}

// compute_group over NTOK x tiles (XF floats and XR run sums apart), both
// tokens' sums of a step before the next step, with a scheduling barrier
// after each step (hoisting every step's LDS reads for two tokens would take
// twice the registers of the one-token form).
template <int QT, int RT, int STEPS, bool EXACT, int NTOK, int XF, int XR, int KCAP>
__device__ __forceinline__ void compute_group_tok(const Frag<QT, RT> (&f)[STEPS], const float* xl, const float* xs,
                                                  int C, int cb, int lane, float* acc) {
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
        const int c = cb + lane + s * kWave;
        if (EXACT || cb + s * kWave < C) {
#pragma unroll
            for (int u = 0; u < NTOK; u++)
                compute_frag<QT, RT, KCAP, false>(f[s], xl + u * XF, xs + u * XR, min(c, C - 1), c < C,
                                                  acc + u * RT);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The fragments' sums for every staged token (one: compute_group).
template <int QT, int RT, int STEPS, bool EXACT, bool FENCE, int KCAP, bool XQ, int NTOK, int XF, int XR>
__device__ __forceinline__ void compute_tokens(const Frag<QT, RT> (&f)[STEPS], const float* xl, const float* xs,
                                               int C, int cb, int lane, float* acc) {
    if constexpr (NTOK == 1)
        compute_group<QT, RT, STEPS, EXACT, FENCE, KCAP, XQ>(f, xl, xs, C, cb, lane, acc);
    else
        compute_group_tok<QT, RT, STEPS, EXACT, NTOK, XF, XR, KCAP>(f, xl, xs, C, cb, lane, acc);
}

// One GEMV: y[r] = sum_k w[r,k] * x[k] for r < rows, k = nb * block_elems,
// in the prologue/epilogue form PRO/EPI.  A wave owns row tiles
// blockIdx*WAVES + wid + j*gridDim*WAVES.  For each tile it issues the loads
// of every chunk step (64 consecutive 16-byte chunks per row per step) before
// it computes any of them, so a tile costs one memory round trip (the generic
// form, !EXACT, walks the row in groups of STEPS steps, one round trip per
// group).  The first tile is peeled and kept branch-free: x's loads (and the
// norm weight's), then the tile's loads, then x's LDS store and the barrier,
// so the barrier waits for x only and step s computes as soon as its own loads
// land.  Occupancy (several waves per SIMD) overlaps one wave's compute with
// others' loads.
//
// PF (exact instances only): the wave loads its next tile while it computes
// the current one (two fragment sets used in turn, the last tile's prefetch
// clamped to a valid tile and dropped), stores with reduce_store_all.
// FENCE: see compute_group.
template <int QT, int KCAP, int WAVES, int RT, int STEPS, bool EXACT, bool NT, int PRO, int EPI, bool PF = false,
          bool FENCE = false, bool XQ = false>
__device__ __forceinline__ void gemv(const GemvArgs& a) {
    static_assert((PRO == PRO_TOK2) == (EPI == EPI_TOK), "the two-token prologue and epilogue go together");
    static_assert(PRO != PRO_TOK2 || (!PF && !XQ), "two-token instances stage fp32 x and do not prefetch");
    constexpr int NTOK = PRO == PRO_TOK2 ? 2 : 1;  // x rows staged, values per fragment row
    constexpr int XF = XTile<KCAP>::kFloats, XR = XTile<KCAP>::kRuns + 1;
    __shared__ __attribute__((aligned(16))) float xl[XF * NTOK];
    __shared__ float xs[XR * NTOK];
    __shared__ float red[WAVES];
    constexpr bool PAIR = EPI == EPI_PAIR;
    constexpr int RP = PAIR ? RT / 2 : RT;  // output rows per tile
    constexpr int NX = (KCAP / 4 + WAVES * kWave - 1) / (WAVES * kWave);
    constexpr int GROUP = STEPS * kWave;    // chunks per group
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wid = threadIdx.x / kWave;
    const int C = chunks_per_row<QT>(a.nb);
    const uint32_t ntiles = (a.rows + RP - 1) / RP;
    const uint32_t tstride = gridDim.x * WAVES;
    uint32_t tile = blockIdx.x * WAVES + wid;

    const int k = static_cast<int>(a.nb) * elems_per_block<QT>();
    XRegs<NX> xr, gr;
    xload(a.x, k, xr);
    if constexpr (PRO == PRO_NORM) xload(a.xw, k, gr);
    if constexpr (PRO == PRO_TOK2) xload(a.x + k, k, gr);  // the second token's row
    Frag<QT, RT> f[STEPS];
    TileRows<RT> tr = tile_rows<RT, PAIR>(a, min(tile, ntiles - 1));
    load_group<QT, RT, STEPS, EXACT, NT>(f, tr, a.nb, C, 0, lane);
    float scale = 1.0f;
    if constexpr (PRO == PRO_NORM) {
        scale = xstore_norm<KCAP, NX, WAVES, XQ>(xr, gr, k, a.eps, xl, xs, red);
    } else if constexpr (PRO == PRO_TOK2) {
        xstore<KCAP, NX, false, false>(xr, k, xl, xs);
        xstore<KCAP, NX>(gr, k, xl + XF, xs + XR);
    } else {
        xstore<KCAP, NX, XQ>(xr, k, xl, xs);
    }

    float acc[RT * NTOK];
    if constexpr (PF) {
        static_assert(EXACT, "the prefetching loop needs one step group per tile");
        Frag<QT, RT> g[STEPS];
        float rf = 0.0f, rg = 0.0f;
        if constexpr (EPI == EPI_RESID) rf = a.res[store_row<RT, EPI>(a, min(tile, ntiles - 1), lane)];
        uint32_t t = tile;
        while (t < ntiles) {
            const uint32_t t1 = t + tstride;
            {
                const uint32_t tc = min(t1, ntiles - 1);
                load_group<QT, RT, STEPS, EXACT, NT>(g, tile_rows<RT, PAIR>(a, tc), a.nb, C, 0, lane);
                if constexpr (EPI == EPI_RESID) rg = a.res[store_row<RT, EPI>(a, tc, lane)];
            }
#pragma unroll
            for (int r = 0; r < RT; r++) acc[r] = 0.0f;
            compute_group<QT, RT, STEPS, EXACT, FENCE, KCAP, XQ>(f, xl, xs, C, 0, lane, acc);
            reduce_store_all<RT, EPI>(acc, a, t, scale, lane, rf);
            if (t1 >= ntiles) break;
            t = t1 + tstride;
            {
                const uint32_t tc = min(t, ntiles - 1);
                load_group<QT, RT, STEPS, EXACT, NT>(f, tile_rows<RT, PAIR>(a, tc), a.nb, C, 0, lane);
                if constexpr (EPI == EPI_RESID) rf = a.res[store_row<RT, EPI>(a, tc, lane)];
            }
#pragma unroll
            for (int r = 0; r < RT; r++) acc[r] = 0.0f;
            compute_group<QT, RT, STEPS, EXACT, FENCE, KCAP, XQ>(g, xl, xs, C, 0, lane, acc);
            reduce_store_all<RT, EPI>(acc, a, t1, scale, lane, rg);
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < RT * NTOK; r++) acc[r] = 0.0f;
    compute_tokens<QT, RT, STEPS, EXACT, FENCE, KCAP, XQ, NTOK, XF, XR>(f, xl, xs, C, 0, lane, acc);
    if constexpr (!EXACT) {
        for (int cb = GROUP; cb < C; cb += GROUP) {
            load_group<QT, RT, STEPS, EXACT, NT>(f, tr, a.nb, C, cb, lane);
            compute_tokens<QT, RT, STEPS, EXACT, FENCE, KCAP, XQ, NTOK, XF, XR>(f, xl, xs, C, cb, lane, acc);
        }
    }
    if (tile < ntiles) reduce_store<RT * NTOK, EPI, NTOK>(acc, a, tile, scale, lane);
    for (tile += tstride; tile < ntiles; tile += tstride) {
        tr = tile_rows<RT, PAIR>(a, tile);
#pragma unroll
        for (int r = 0; r < RT * NTOK; r++) acc[r] = 0.0f;
        for (int cb = 0; cb < (EXACT ? 1 : C); cb += GROUP) {
            load_group<QT, RT, STEPS, EXACT, NT>(f, tr, a.nb, C, cb, lane);
            compute_tokens<QT, RT, STEPS, EXACT, FENCE, KCAP, XQ, NTOK, XF, XR>(f, xl, xs, C, cb, lane, acc);
        }
        reduce_store<RT * NTOK, EPI, NTOK>(acc, a, tile, scale, lane);
    }
}
// ---- the int path for a few tokens -------------------------------------------
// zlm's int prefill arithmetic (activations quantized to q8 blocks,
// matvec/layout.zig:458-476; integer block dots scaled per block,
// kernels/quantized.zig:49-55 q4_0, :79-87 q4_1, :111-123 q4_k, :149-156 q8_0)
// for m <= NTOK tokens in one pass over the weights in the GEMV layout.  Each
// workgroup quantizes the m activation rows into LDS itself (q8_quant4, the
// quantizer kernel's arithmetic); each lane loads its weight chunk once and
// forms the chunk's integer dot with every token (v_dot4_i32_i8; nibbles
// 0..15 are valid int8), then scales it in fp32.

// One token's q8 tile in LDS, in 4-byte words: the q bytes (KCAP/4 words, in
// the order the quant's chunks read them, q8_pos), the 16-element run sums
// (int32, natural order), the 32-element block scales dx (natural order) and
// 4 dummy words that out-of-range threads store to.
template <int KCAP>
struct Q8Tile {
    static constexpr int kRuns = KCAP / 4;
    static constexpr int kDx = kRuns + KCAP / 16;
    static constexpr int kDummy = kDx + KCAP / 32;
    static constexpr int kWords = kDummy + 4;
};

// Byte offset in the q area of element e (e a multiple of 4 here): q8_0 in
// order; q4_0 / q4_1 elements 0-15 of block b at 16b in the first half of
// the area and elements 16-31 at 16b in the second; q4_k the elements of
// sub-block 2g of super-block sb (nibble lows of the group's qs bytes) at
// 128sb + 32g + r in the first half and those of sub-block 2g+1 in the
// second.  Chunk c then reads its two 16-element runs at 16c in each half:
// consecutive lanes read consecutive 16-byte words.
template <int QT, int KCAP>
__device__ __forceinline__ int q8_pos(int e) {
    if constexpr (QT == Q8_0) {
        return e;
    } else if constexpr (QT == Q4_K) {
        const int r = e & 63, base = 128 * (e >> 8) + 32 * ((e >> 6) & 3);
        return r < 32 ? base + r : KCAP / 2 + base + r - 32;
    } else {
        const int j = e & 31, base = 16 * (e >> 5);
        return j < 16 ? base + j : KCAP / 2 + base + j - 16;
    }
}

// Quantize one token's x (NX float4 per thread, k elements) into its tile.
// Thread i's float4 holds elements 4i..4i+3: lanes 8b..8b+7 of a wave share
// block b (k is a multiple of 32, so a block's lanes are all in range or all
// out), lanes 4r..4r+3 run r.
template <int QT, int KCAP, int NX>
__device__ __forceinline__ void q8_store(const XRegs<NX>& r, int k, uint32_t* t) {
    using T = Q8Tile<KCAP>;
    const int n4 = k >> 2;
#pragma unroll
    for (int j = 0; j < NX; j++) {
        const int i = j * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
        const bool valid = i < n4;
        const float4 v = valid ? r.v[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float d;
        int32_t s;
        const uint32_t wv = q8_quant4(v, d, s);
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        t[valid ? q8_pos<QT, KCAP>(4 * i) / 4 : T::kDummy] = wv;
        t[(valid && (i & 3) == 0) ? T::kRuns + (i >> 2) : T::kDummy + 1] = static_cast<uint32_t>(s);
        t[(valid && (i & 7) == 0) ? T::kDx + (i >> 3) : T::kDummy + 2] = __builtin_bit_cast(uint32_t, d);
    }
}

__device__ __forceinline__ int dot16(const uint32_t (&w)[4], uint4 q, int acc) {
    acc = __builtin_amdgcn_sdot4(static_cast<int>(w[0]), static_cast<int>(q.x), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(w[1]), static_cast<int>(q.y), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(w[2]), static_cast<int>(q.z), acc, false);
    return __builtin_amdgcn_sdot4(static_cast<int>(w[3]), static_cast<int>(q.w), acc, false);
}

// Chunk c of RT weight rows against NTOK token tiles (tile t at tq + t *
// kWords): acc[t * RT + r] += the chunk's share of row r . x_t in the int
// path's form:
//   q4_0  (dw*dx) * (sum nib*q - 8 * sum q)             (block c)
//   q4_1  (d*dx) * sum nib*q + (m*dx) * sum q          (block c)
//   q8_0  (dw*dx) * sum w*q                            (half c&1 of block c>>1)
//   q4_k  per sub-block half: (d*sc*dx) * sum nib*q - (dmin*mn*dx) * sum q
//         (the lows of the chunk's 16 qs bytes: sub-block 2g, the highs 2g+1)
// A token's LDS words are read once for all RT rows.  The integer parts are
// exact; valid = false zeroes the scales.
template <int QT, int KCAP, int NTOK, int RT>
__device__ __forceinline__ void compute_int(const Frag<QT, RT>& f, const uint32_t* tq, int c, bool valid,
                                            float* acc) {
    using T = Q8Tile<KCAP>;
    uint32_t w[RT][4];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        w[r][0] = f.q[r].x;
        w[r][1] = f.q[r].y;
        w[r][2] = f.q[r].z;
        w[r][3] = f.q[r].w;
    }
    if constexpr (QT == Q8_0) {
        float dw[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) dw[r] = valid ? h2f(f.d[r]) : 0.0f;
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
            const uint32_t* tt = tq + t * T::kWords;
            const uint4 q = *reinterpret_cast<const uint4*>(tt + 4 * c);
            const float dx = __builtin_bit_cast(float, tt[T::kDx + (c >> 1)]);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const int dot = dot16(w[r], q, 0);
                acc[t * RT + r] = fmaf(dw[r] * dx, static_cast<float>(dot), acc[t * RT + r]);
            }
        }
    } else {
        uint32_t lo[RT][4], hi[RT][4];
#pragma unroll
        for (int r = 0; r < RT; r++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[r][i] = w[r][i] & 0x0F0F0F0Fu;
                hi[r][i] = (w[r][i] >> 4) & 0x0F0F0F0Fu;
            }
        }
        if constexpr (QT == Q4_K) {
            float d[RT], dmin[RT], sc1[RT], sc2[RT], mn1[RT], mn2[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const uint32_t dd = valid ? f.dm[r] : 0u;
                d[r] = h2f(dd);
                dmin[r] = h2f(dd >> 16);
                sc1[r] = ub(f.sm[r], 0);
                sc2[r] = ub(f.sm[r], 1);
                mn1[r] = ub(f.sm[r], 2);
                mn2[r] = ub(f.sm[r], 3);
            }
            const int sb = c >> 3, p = c & 7, g = p >> 1;
            const int run_lo = 16 * sb + 4 * g + (p & 1), blk_lo = 8 * sb + 2 * g;
#pragma unroll
            for (int t = 0; t < NTOK; t++) {
                const uint32_t* tt = tq + t * T::kWords;
                const uint4 qlo = *reinterpret_cast<const uint4*>(tt + 4 * c);
                const uint4 qhi = *reinterpret_cast<const uint4*>(tt + KCAP / 8 + 4 * c);
                const float slo = static_cast<float>(static_cast<int32_t>(tt[T::kRuns + run_lo]));
                const float shi = static_cast<float>(static_cast<int32_t>(tt[T::kRuns + run_lo + 2]));
                const float xlo = __builtin_bit_cast(float, tt[T::kDx + blk_lo]);
                const float xhi = __builtin_bit_cast(float, tt[T::kDx + blk_lo + 1]);
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    const int dlo = dot16(lo[r], qlo, 0);
                    const int dhi = dot16(hi[r], qhi, 0);
                    float v = (d[r] * sc1[r] * xlo) * static_cast<float>(dlo);
                    v = fmaf(d[r] * sc2[r] * xhi, static_cast<float>(dhi), v);
                    v = fmaf(-(dmin[r] * mn1[r] * xlo), slo, v);
                    v = fmaf(-(dmin[r] * mn2[r] * xhi), shi, v);
                    acc[t * RT + r] += v;
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < NTOK; t++) {
                const uint32_t* tt = tq + t * T::kWords;
                const uint4 qlo = *reinterpret_cast<const uint4*>(tt + 4 * c);
                const uint4 qhi = *reinterpret_cast<const uint4*>(tt + KCAP / 8 + 4 * c);
                const int sq = static_cast<int32_t>(tt[T::kRuns + 2 * c]) + static_cast<int32_t>(tt[T::kRuns + 2 * c + 1]);
                const float dx = __builtin_bit_cast(float, tt[T::kDx + c]);
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    int dot = dot16(lo[r], qlo, 0);
                    dot = dot16(hi[r], qhi, dot);
                    float& a = acc[t * RT + r];
                    if constexpr (QT == Q4_0) {
                        const float dw = valid ? h2f(f.d[r]) : 0.0f;
                        a = fmaf(dw * dx, static_cast<float>(dot - 8 * sq), a);
                    } else {
                        const uint32_t dm = valid ? f.dm[r] : 0u;
                        a = fmaf(h2f(dm) * dx, static_cast<float>(dot), a);
                        a = fmaf(h2f(dm >> 16) * dx, static_cast<float>(sq), a);
                    }
                }
            }
        }
    }
}

// compute_int over a group of STEPS chunk steps, a scheduling barrier after
// each step.
template <int QT, int KCAP, int NTOK, int RT, int STEPS>
__device__ __forceinline__ void compute_group_int(const Frag<QT, RT> (&f)[STEPS], const uint32_t* tq, int C, int cb,
                                                  int lane, float* acc) {
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
        const int c = cb + lane + s * kWave;
        if (cb + s * kWave < C) compute_int<QT, KCAP, NTOK, RT>(f[s], tq, min(c, C - 1), c < C, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// y[t * rows + r] = row r . x_t (int path) for t < m <= NTOK: RT-row wave
// tiles (tile = blockIdx*WAVES + wid + j*gridDim*WAVES), each row walked in
// groups of STEPS chunk steps (one memory round trip per group).  The first
// tile's first group is loaded before the activations are quantized, so the
// staging overlaps it.  Rows of x past m repeat row m-1 and are not stored.
// Each row's sums and their reduction are the same for any RT.
template <int QT, int NTOK, int KCAP, int WAVES, int STEPS, int RT = 1>
__device__ __forceinline__ void gemv_int(const GemvArgs& a) {
    static_assert(QT == Q4_0 || QT == Q4_1 || QT == Q8_0 || QT == Q4_K, "int path quants");
    static_assert(NTOK >= 2 && NTOK * RT <= 8, "the row reduction holds at most 8 values per lane");
    using T = Q8Tile<KCAP>;
    __shared__ __attribute__((aligned(16))) uint32_t tq[T::kWords * NTOK];
    constexpr int NX = (KCAP / 4 + WAVES * kWave - 1) / (WAVES * kWave);
    constexpr int GROUP = STEPS * kWave;
    constexpr int NV = NTOK * RT;
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wid = threadIdx.x / kWave;
    const int C = chunks_per_row<QT>(a.nb);
    const uint32_t ntiles = (a.rows + RT - 1) / RT;
    const uint32_t tstride = gridDim.x * WAVES;
    uint32_t tile = blockIdx.x * WAVES + wid;
    const int k = static_cast<int>(a.nb) * elems_per_block<QT>();

    XRegs<NX> xr[NTOK];
#pragma unroll
    for (int t = 0; t < NTOK; t++) xload(a.x + static_cast<size_t>(min(static_cast<uint32_t>(t), a.m - 1)) * k, k, xr[t]);
    Frag<QT, RT> f[STEPS];
    TileRows<RT> tr = tile_rows<RT, false>(a, min(tile, ntiles - 1));
    load_group<QT, RT, STEPS, false, true>(f, tr, a.nb, C, 0, lane);
#pragma unroll
    for (int t = 0; t < NTOK; t++) q8_store<QT, KCAP, NX>(xr[t], k, tq + t * T::kWords);
    __syncthreads();

    float acc[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) acc[i] = 0.0f;
    compute_group_int<QT, KCAP, NTOK, RT, STEPS>(f, tq, C, 0, lane, acc);
    for (int cb = GROUP; cb < C; cb += GROUP) {
        load_group<QT, RT, STEPS, false, true>(f, tr, a.nb, C, cb, lane);
        compute_group_int<QT, KCAP, NTOK, RT, STEPS>(f, tq, C, cb, lane, acc);
    }
    if (tile < ntiles) reduce_store<NV, EPI_TOK, NTOK>(acc, a, tile, 1.0f, lane);
    for (tile += tstride; tile < ntiles; tile += tstride) {
        tr = tile_rows<RT, false>(a, tile);
#pragma unroll
        for (int i = 0; i < NV; i++) acc[i] = 0.0f;
        for (int cb = 0; cb < C; cb += GROUP) {
            load_group<QT, RT, STEPS, false, true>(f, tr, a.nb, C, cb, lane);
            compute_group_int<QT, KCAP, NTOK, RT, STEPS>(f, tq, C, cb, lane, acc);
        }
        reduce_store<NV, EPI_TOK, NTOK>(acc, a, tile, 1.0f, lane);
    }
}

// ---- several matrices over one x in one launch -------------------------------
// The contract's matVecResidentBatch (reference gpu/backend/root.zig:249-254,
// vulkan/pipeline.zig:1770-1802) runs up to RingSize GEMVs that share k and x.
// One launch covers all of them: the row tiles of op i are global tiles
// [first[i], first[i+1]), a wave finds its op by a wave-uniform scan, and
// everything else is the plain GEMV (1-row tiles), so the launch's fixed cost
// is paid once for the whole batch.
constexpr int kMultiMax = 8;

struct GemvMultiArgs {
    const uint8_t* w[kMultiMax];
    const uint16_t* d[kMultiMax];
    float* y[kMultiMax];
    uint32_t first[kMultiMax + 1];  // first global row of op i; first[n] = all rows
    const float* x;
    uint32_t n;
    uint32_t nb;
};

__device__ __forceinline__ TileRows<1> multi_row(const GemvMultiArgs& a, uint32_t t, uint32_t& op) {
    op = 0;
#pragma unroll
    for (int i = 1; i < kMultiMax; i++)
        if (static_cast<uint32_t>(i) < a.n && t >= a.first[i]) op = static_cast<uint32_t>(i);
    TileRows<1> tr;
    tr.w[0] = a.w[op];
    tr.d[0] = a.d[op];
    tr.r[0] = t - a.first[op];
    return tr;
}

template <int QT, int KCAP, int WAVES, int STEPS, bool EXACT>
__device__ __forceinline__ void gemv_multi(const GemvMultiArgs& a) {
    __shared__ __attribute__((aligned(16))) float xl[XTile<KCAP>::kFloats];
    __shared__ float xs[XTile<KCAP>::kRuns + 1];
    constexpr int NX = (KCAP / 4 + WAVES * kWave - 1) / (WAVES * kWave);
    constexpr int GROUP = STEPS * kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wid = threadIdx.x / kWave;
    const int C = chunks_per_row<QT>(a.nb);
    const uint32_t ntiles = a.first[a.n];
    const uint32_t tstride = gridDim.x * WAVES;
    uint32_t tile = blockIdx.x * WAVES + wid;
    const int k = static_cast<int>(a.nb) * elems_per_block<QT>();
    XRegs<NX> xr;
    xload(a.x, k, xr);
    Frag<QT, 1> f[STEPS];
    uint32_t op;
    TileRows<1> tr = multi_row(a, min(tile, ntiles - 1), op);
    load_group<QT, 1, STEPS, EXACT, true>(f, tr, a.nb, C, 0, lane);
    xstore<KCAP>(xr, k, xl, xs);
    float acc[1];
    if constexpr (EXACT) {
        // The wave's next row is loaded while the current one is computed
        // (two fragment sets). Every lane stores the row's sum, so no branch
        // guards the store (a guarded store makes the wait before the next
        // compute include the prefetched loads); a prefetch past the end is
        // clamped to the last row and never computed.
        Frag<QT, 1> g[STEPS];
        uint32_t op1;
        TileRows<1> tr1;
        uint32_t t = tile;
        while (t < ntiles) {
            const uint32_t t1 = t + tstride;
            tr1 = multi_row(a, min(t1, ntiles - 1), op1);
            load_group<QT, 1, STEPS, true, true>(g, tr1, a.nb, C, 0, lane);
            acc[0] = 0.0f;
            compute_group<QT, 1, STEPS, true, true>(f, xl, xs, C, 0, lane, acc);
            a.y[op][tr.r[0]] = wave_sum_all(acc[0]);
            if (t1 >= ntiles) break;
            t = t1 + tstride;
            tr = multi_row(a, min(t, ntiles - 1), op);
            load_group<QT, 1, STEPS, true, true>(f, tr, a.nb, C, 0, lane);
            acc[0] = 0.0f;
            compute_group<QT, 1, STEPS, true, true>(g, xl, xs, C, 0, lane, acc);
            a.y[op1][tr1.r[0]] = wave_sum_all(acc[0]);
        }
        return;
    }
    for (;;) {
        acc[0] = 0.0f;
        compute_group<QT, 1, STEPS, EXACT>(f, xl, xs, C, 0, lane, acc);
        if constexpr (!EXACT) {
            for (int cb = GROUP; cb < C; cb += GROUP) {
                load_group<QT, 1, STEPS, EXACT, true>(f, tr, a.nb, C, cb, lane);
                compute_group<QT, 1, STEPS, EXACT>(f, xl, xs, C, cb, lane, acc);
            }
        }
        const float sum = wave_sum_all(acc[0]);
        if (tile < ntiles && lane == 0) a.y[op][tr.r[0]] = sum;
        tile += tstride;
        if (tile >= ntiles) break;
        tr = multi_row(a, tile, op);
        load_group<QT, 1, STEPS, EXACT, true>(f, tr, a.nb, C, 0, lane);
    }
}

// ---- split-K GEMV (short, wide matrices) -------------------------------------
// The FFN down projection (k = 12288 over 4096 rows) leaves the one-wave-per-
// row kernel one wave per SIMD: a row's 12 chunk steps of fragments take ~300
// registers, so few rows' loads are in flight.  Here the W waves of a
// workgroup share each tile of RT rows: wave w covers chunk steps
// [w*SPL, (w+1)*SPL) of every row (lane l: chunks (w*SPL + s)*64 + l, s <
// SPL), holds x of exactly those chunks in registers for the whole launch --
// x is read once per workgroup and never staged in LDS -- and the W partial
// sums of a row meet in LDS, one barrier per tile, added in wave order.  A
// wave loads its next tile while it computes the current one.  Every wave of
// the workgroup stores the tile's rows (the same values), so the stores need
// no branch.  Chunks past the row's end (W*SPL*64 > chunks) are clamped
// loads with zero x and a zero scale.
template <int QT, bool XQ>
struct XChunk;
template <>
struct XChunk<Q8_0, false> {  // the chunk's 16 x values
    float v[16];
};
template <>
struct XChunk<Q4_0, true> {  // the block's 32 x values as int8 planes (XQTile's encoding)
    uint4 pl[3];             // plane p of elements 0..15
    uint4 ph[3];             // plane p of elements 16..31
    float d1;                // 1/s
    float sum;               // the fp32 sum of the 32 values
};
struct XRuns {  // a K-quant piece's two 16-element runs of x and their sums
    float4 a[4];
    float4 b[4];
    float sa;
    float sb;
};
template <>
struct XChunk<Q4_0, false> : XRuns {};  // the block's elements 0..15 (a) and 16..31 (b)
template <>
struct XChunk<Q4_K, false> : XRuns {};
template <>
struct XChunk<Q6_K, false> : XRuns {};
template <>
struct XChunk<Q4_K, true> : XqRuns {};  // the runs as int8 planes, one scale per run
template <>
struct XChunk<Q6_K, true> : XqRuns {};

template <int QT>
constexpr int sk_chunk_elems() {
    static_assert(QT == Q8_0 || QT == Q4_0 || QT == Q4_K || QT == Q6_K,
                  "split-K is implemented for q8_0, q4_0, q4_k and q6_k");
    return QT == Q8_0 ? 16 : 32;
}

template <int QT>
struct XRaw {
    float4 v[sk_chunk_elems<QT>() / 4];
};

// x of chunk c: its consecutive elements (q8_0, q4_0) or its two runs
// (K-quants: v[0..3] the low run, v[4..7] the high one).
template <int QT>
__device__ __forceinline__ void xraw_load(const float* __restrict__ x, int c, XRaw<QT>& r) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    if constexpr (QT == Q4_K || QT == Q6_K) {
        int e_lo, e_hi;
        kquant_runs<QT>(c, e_lo, e_hi);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            r.v[i] = x4[(e_lo >> 2) + i];
            r.v[4 + i] = x4[(e_hi >> 2) + i];
        }
    } else {
        constexpr int N = sk_chunk_elems<QT>() / 4;
        const float4* p = x4 + static_cast<size_t>(c) * N;
#pragma unroll
        for (int i = 0; i < N; i++) r.v[i] = p[i];
    }
}

__device__ __forceinline__ float4 zero_unless(float4 v, bool valid) {
    return valid ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// The runs of a chunk (K-quants: its two 16-element runs; q4_0: the block's
// two halves) and their sums in xstore's order (float4 sums, then pairs).
template <int QT>
__device__ __forceinline__ XRuns make_xruns(const XRaw<QT>& r, bool valid) {
    XRuns x;
    float q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = zero_unless(r.v[i], valid);
        if (i < 4) x.a[i & 3] = v;
        else x.b[i & 3] = v;
        q[i] = (v.x + v.y) + (v.z + v.w);
    }
    x.sa = (q[0] + q[1]) + (q[2] + q[3]);
    x.sb = (q[4] + q[5]) + (q[6] + q[7]);
    return x;
}

// The block's planes exactly as xput forms them in LDS (same amax, exponent
// and rounding), and its sum in xstore's order (float4 sums, then pairs).
__device__ __forceinline__ XChunk<Q4_0, true> make_xq_block(const XRaw<Q4_0>& r, bool valid) {
    XChunk<Q4_0, true> x;
    float4 v[8];
    float am = 0.0f, q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        v[i] = zero_unless(r.v[i], valid);
        am = fmaxf(am, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        q[i] = (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    const int e = xq_exp(am);
    const float s = ldexpf(1.0f, 5 - e);
    x.d1 = ldexpf(1.0f, e - 5);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        xq_planes(v[i], s, (&x.pl[0].x)[i], (&x.pl[1].x)[i], (&x.pl[2].x)[i]);
        xq_planes(v[4 + i], s, (&x.ph[0].x)[i], (&x.ph[1].x)[i], (&x.ph[2].x)[i]);
    }
    x.sum = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
    return x;
}

// A K-quant piece's runs as int8 planes in registers: the XQ encoding with one
// power-of-two scale per 16-element run (the lane holds half of each
// 32-element block, so it scales its runs on their own).
template <int QT>
__device__ __forceinline__ XChunk<QT, true> make_xq_runs(const XRaw<QT>& r, bool valid) {
    XChunk<QT, true> x;
    float q[8];
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        v[i] = zero_unless(r.v[i], valid);
        q[i] = (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    auto encode = [](const float4* u, uint4 (&pl)[3], float& d1) {
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++)
            am = fmaxf(am, fmaxf(fmaxf(fabsf(u[i].x), fabsf(u[i].y)), fmaxf(fabsf(u[i].z), fabsf(u[i].w))));
        const int e = xq_exp(am);
        const float sc = ldexpf(1.0f, 5 - e);
#pragma unroll
        for (int i = 0; i < 4; i++) xq_planes(u[i], sc, (&pl[0].x)[i], (&pl[1].x)[i], (&pl[2].x)[i]);
        d1 = ldexpf(1.0f, e - 5);
    };
    encode(v, x.pa, x.d1a);
    encode(v + 4, x.pb, x.d1b);
    x.sa = (q[0] + q[1]) + (q[2] + q[3]);
    x.sb = (q[4] + q[5]) + (q[6] + q[7]);
    return x;
}

// The lane's register x of one chunk from its raw float4s (zero if the chunk
// is past the row's end).
template <int QT, bool XQ>
__device__ __forceinline__ XChunk<QT, XQ> make_xchunk(const XRaw<QT>& r, bool valid) {
    XChunk<QT, XQ> x;
    if constexpr (QT == Q8_0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = zero_unless(r.v[i], valid);
            x.v[4 * i] = v.x;
            x.v[4 * i + 1] = v.y;
            x.v[4 * i + 2] = v.z;
            x.v[4 * i + 3] = v.w;
        }
    } else if constexpr (QT == Q4_0 && XQ) {
        x = make_xq_block(r, valid);
    } else if constexpr (XQ) {
        x = make_xq_runs<QT>(r, valid);
    } else {
        static_cast<XRuns&>(x) = make_xruns<QT>(r, valid);
    }
    return x;
}

template <int RT>
__device__ __forceinline__ void dot_xchunk(const Frag<Q4_0, RT>& f, const XChunk<Q4_0, false>& x, int, bool valid,
                                           float* acc) {
    q4_0_rows<RT>(
        f, [&](int i) { return x.a[i]; }, [&](int i) { return x.b[i]; }, x.sa + x.sb, valid, acc);
}

template <int RT>
__device__ __forceinline__ void dot_xchunk(const Frag<Q4_K, RT>& f, const XChunk<Q4_K, true>& x, int c, bool valid,
                                           float* acc) {
    q4_k_xq_rows<RT>(f, c, x, valid, acc);
}
template <int RT>
__device__ __forceinline__ void dot_xchunk(const Frag<Q6_K, RT>& f, const XChunk<Q6_K, true>& x, int c, bool valid,
                                           float* acc) {
    q6_k_xq_rows<RT>(f, c, x, valid, acc);
}

template <int RT>
__device__ __forceinline__ void dot_xchunk(const Frag<Q4_K, RT>& f, const XChunk<Q4_K, false>& x, int c, bool valid,
                                           float* acc) {
    q4_k_rows<RT>(
        f, c, [&](int i) { return x.a[i]; }, [&](int i) { return x.b[i]; }, x.sa, x.sb, valid, acc);
}
template <int RT>
__device__ __forceinline__ void dot_xchunk(const Frag<Q6_K, RT>& f, const XChunk<Q6_K, false>& x, int c, bool valid,
                                           float* acc) {
    q6_k_rows<RT>(
        f, c, [&](int i) { return x.a[i]; }, [&](int i) { return x.b[i]; }, x.sa, x.sb, valid, acc);
}

template <int RT>
__device__ __forceinline__ void dot_xchunk(const Frag<Q8_0, RT>& f, const XChunk<Q8_0, false>& x, int, bool valid,
                                           float* acc) {
    float s[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) s[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint32_t wv = (&f.q[r].x)[i];
            s[r] = fmaf(sb(wv, 0), x.v[4 * i], s[r]);
            s[r] = fmaf(sb(wv, 1), x.v[4 * i + 1], s[r]);
            s[r] = fmaf(sb(wv, 2), x.v[4 * i + 2], s[r]);
            s[r] = fmaf(sb(wv, 3), x.v[4 * i + 3], s[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++) acc[r] = fmaf(valid ? h2f(f.d[r]) : 0.0f, s[r], acc[r]);
}

template <int RT>
__device__ __forceinline__ void dot_xchunk(const Frag<Q4_0, RT>& f, const XChunk<Q4_0, true>& x, int, bool valid,
                                           float* acc) {
    q4_0_xq_rows<RT>(f, x.pl, x.ph, x.d1, x.sum, valid, acc);
}

// The loads of tile t (RT consecutive rows, clamped) at the lane's chunks.
template <int QT, int RT, int SPL>
__device__ __forceinline__ void sk_load(Frag<QT, RT> (&f)[SPL], const GemvArgs& a, uint32_t t, const int (&cs)[SPL]) {
    TileRows<RT> tr;
#pragma unroll
    for (int r = 0; r < RT; r++) {
        tr.w[r] = a.w0;
        tr.d[r] = a.d0;
        tr.r[r] = min(t * RT + static_cast<uint32_t>(r), a.rows - 1);
    }
#pragma unroll
    for (int s = 0; s < SPL; s++) load_frag<QT, RT, true>(f[s], tr, a.nb, cs[s]);
}

template <int RT>
constexpr int sk_log() {
    static_assert(RT == 1 || RT == 2 || RT == 4 || RT == 8 || RT == 16, "split-K row tiles: 1..16 rows, a power of two");
    return (RT >= 16) ? 4 : (RT >= 8) ? 3 : (RT >= 4) ? 2 : (RT >= 2) ? 1 : 0;
}

// The output row of this lane's fragment row after the butterfly (clamped).
template <int RT>
__device__ __forceinline__ uint32_t sk_row(const GemvArgs& a, uint32_t t, int lane) {
    return min(t * RT + static_cast<uint32_t>(lane >> (6 - sk_log<RT>())), a.rows - 1);
}

// Reduce the wave's RT partials (the transposing butterfly of reduce_store,
// selecting through bit masks so the compiler keeps v in registers), meet
// the other waves' partials in red, store the tile.  EPI_RESID: the residual
// rides in wave 0's partial, so every wave has its residual load back before
// the barrier -- y may alias res, and the tile's stores follow the barrier.
// The in-wave part of a tile's reduction: after the transposing butterfly
// lane group fr holds row fr's partial of this wave (plus the residual in
// wave 0), written to red[fr][wid].
template <int W, int RT, int EPI>
__device__ __forceinline__ void sk_park(float* v, float (*red)[W], int lane, int wid, float rv) {
    constexpr int LOG = sk_log<RT>();
#pragma unroll
    for (int st = 0; st < LOG; st++) {
        const int half = (RT >> st) >> 1;
        const int bit = 32 >> st;
        const uint32_t m = (lane & bit) != 0 ? 0xffffffffu : 0u;
#pragma unroll
        for (int i = 0; i < half; i++) {
            const uint32_t lo = __builtin_bit_cast(uint32_t, v[i]);
            const uint32_t hi = __builtin_bit_cast(uint32_t, v[half + i]);
            const float keep = __builtin_bit_cast(float, (hi & m) | (lo & ~m));
            const float send = __builtin_bit_cast(float, (lo & m) | (hi & ~m));
            v[i] = keep + __shfl_xor(send, bit, kWave);
        }
    }
    float s = v[0];
#pragma unroll
    for (int off = 32 >> LOG; off >= 1; off >>= 1) s += __shfl_xor(s, off, kWave);
    if constexpr (EPI == EPI_RESID) s += wid == 0 ? rv : 0.0f;
    red[lane >> (6 - LOG)][wid] = s;
}

__device__ __forceinline__ void sk_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum a parked tile over the waves in wave order and store its rows (every
// wave stores the same values; no branch before the store).
template <int W, int RT>
__device__ __forceinline__ void sk_store(const float (*red)[W], const GemvArgs& a, uint32_t t, int lane) {
    const int fr = lane >> (6 - sk_log<RT>());
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < W; w++) tot += red[fr][w];
    a.y[sk_row<RT>(a, t, lane)] = tot;
}

template <int W, int RT, int EPI>
__device__ __forceinline__ void sk_finish(float* v, float (*red)[W], const GemvArgs& a, uint32_t t, int lane,
                                          int wid, float rv) {
    sk_park<W, RT, EPI>(v, red, lane, wid, rv);
    sk_barrier();
    sk_store<W, RT>(red, a, t, lane);
}

// y = W.x (EPI_PLAIN) or res + W.x (EPI_RESID).  The host launches at most
// ceil(rows/RT) workgroups and W*SPL == ceil(chunks per row / 64); EXACT
// instances require chunks per row == 64*W*SPL (no clamping).  A workgroup
// walks tiles blockIdx + j*gridDim with NB fragment sets in a ring: while it
// computes one tile the loads of the next NB-1 are in flight (tiles past the
// end are clamped loads, dropped).  The exit is uniform over the workgroup,
// so every wave meets every barrier; consecutive tiles use different red
// buffers, so one barrier per tile suffices.  With PARK > 0 the tiles' wave
// partials wait in PARK LDS slots and are summed and stored after one barrier
// per PARK tiles (fewer waits for the slowest wave; the stores come later).  Scheduling barriers keep each
// tile's loads ahead of its compute and the compute ahead of the reduction:
// without them the compiler interleaved the three and reused a prefetch
// destination register, which costs a wait for every load in flight
// (measured on gfx950, q8_0 4096 x 12288: 12.0 vs 10.5 us).
template <int QT, int W, int RT, int SPL, int EPI, bool XQ, int NB, bool EXACT, int PARK = 0>
__device__ __forceinline__ void gemv_sk(const GemvArgs& a) {
    static_assert(EPI == EPI_PLAIN || EPI == EPI_RESID, "split-K forms: plain, resid");
    static_assert(!XQ || QT != Q8_0, "q8_0 runs on fp32 x");
    static_assert(NB >= 2, "a ring of at least two fragment sets");
    static_assert(PARK % NB == 0, "parked tiles come in whole ring turns");
    __shared__ float red[PARK > 0 ? PARK : NB][RT][W];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = static_cast<int>(threadIdx.x / kWave);
    const int C = chunks_per_row<QT>(a.nb);
    const uint32_t ntiles = (a.rows + RT - 1) / RT;
    const uint32_t G = gridDim.x;
    int cs[SPL];
    bool ok[SPL];
    XRaw<QT> xr[SPL];
#pragma unroll
    for (int s = 0; s < SPL; s++) {
        const int c = (wid * SPL + s) * kWave + lane;
        ok[s] = EXACT || c < C;
        cs[s] = EXACT ? c : min(c, C - 1);
        xraw_load<QT>(a.x, cs[s], xr[s]);
    }
    uint32_t t = blockIdx.x;
    Frag<QT, RT> f[NB][SPL];
    float rv[NB];
    auto issue = [&](int b, uint32_t ahead) {
        const uint32_t tc =
            static_cast<uint32_t>(min(static_cast<uint64_t>(t) + static_cast<uint64_t>(ahead) * G,
                                      static_cast<uint64_t>(ntiles - 1)));
        sk_load<QT, RT, SPL>(f[b], a, tc, cs);
        rv[b] = EPI == EPI_RESID ? a.res[sk_row<RT>(a, tc, lane)] : 0.0f;
    };
#pragma unroll
    for (int j = 0; j < NB - 1; j++) issue(j, static_cast<uint32_t>(j));
    XChunk<QT, XQ> xc[SPL];
#pragma unroll
    for (int s = 0; s < SPL; s++) xc[s] = make_xchunk<QT, XQ>(xr[s], ok[s]);
    float acc[RT];
    if constexpr (PARK > 0) {
        // Parked reduction: each tile's partials wait in LDS slot n; one
        // barrier per PARK tiles (and one at the end), then every wave sums
        // and stores the parked tiles.  Same sums in the same order as below.
        int n = 0;
        uint32_t t0 = t;
        auto flush = [&]() {
            sk_barrier();
            for (int j = 0; j < n; j++) sk_store<W, RT>(red[j], a, t0 + static_cast<uint32_t>(j) * G, lane);
            sk_barrier();
        };
        while (static_cast<uint64_t>(t) + static_cast<uint64_t>(NB - 1) * G < ntiles) {
#pragma unroll
            for (int p = 0; p < NB; p++) {
                issue((p + NB - 1) % NB, NB - 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int r = 0; r < RT; r++) acc[r] = 0.0f;
#pragma unroll
                for (int s = 0; s < SPL; s++) dot_xchunk<RT>(f[p][s], xc[s], cs[s], ok[s], acc);
                __builtin_amdgcn_sched_barrier(0);
                sk_park<W, RT, EPI>(acc, red[n + p], lane, wid, rv[p]);
                t += G;
            }
            n += NB;
            if (n == PARK) {
                flush();
                n = 0;
                t0 = t;
            }
        }
#pragma unroll
        for (int p = 0; p < NB - 1; p++) {
            if (t < ntiles) {
#pragma unroll
                for (int r = 0; r < RT; r++) acc[r] = 0.0f;
#pragma unroll
                for (int s = 0; s < SPL; s++) dot_xchunk<RT>(f[p][s], xc[s], cs[s], ok[s], acc);
                sk_park<W, RT, EPI>(acc, red[n], lane, wid, rv[p]);
                n++;
                t += G;
            }
        }
        flush();
        return;
    }
    // Whole turns of the ring (all NB tiles exist) in a loop with one exit, so
    // the compiler's wait counts stay exact across the back edge; then the
    // last fewer-than-NB tiles, whose loads are already in flight.
    while (static_cast<uint64_t>(t) + static_cast<uint64_t>(NB - 1) * G < ntiles) {
#pragma unroll
        for (int p = 0; p < NB; p++) {
            issue((p + NB - 1) % NB, NB - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RT; r++) acc[r] = 0.0f;
#pragma unroll
            for (int s = 0; s < SPL; s++) dot_xchunk<RT>(f[p][s], xc[s], cs[s], ok[s], acc);
            __builtin_amdgcn_sched_barrier(0);
            sk_finish<W, RT, EPI>(acc, red[p], a, t, lane, wid, rv[p]);
            t += G;
        }
    }
#pragma unroll
    for (int p = 0; p < NB - 1; p++) {
        if (t >= ntiles) return;
#pragma unroll
        for (int r = 0; r < RT; r++) acc[r] = 0.0f;
#pragma unroll
        for (int s = 0; s < SPL; s++) dot_xchunk<RT>(f[p][s], xc[s], cs[s], ok[s], acc);
        sk_finish<W, RT, EPI>(acc, red[p], a, t, lane, wid, rv[p]);
        t += G;
    }
}

}  // namespace

// ---- GEMV entry points ---------------------------------------------------
// zlm_gemv_<quant>_r<RT>_s<STEPS>: STEPS == ceil(chunks per row / 64) exactly
// (q4_0 and the K-quants have k/32 chunks per row, q8_0 k/16), x capacity the
// smallest of 4096/8192/16384/32768 that holds STEPS steps.
// zlm_gemv_<quant>_r1_g: the generic form for any other k up to 32768 (walks
// the row in groups of 4 steps, 8 for q8_0).
// Every instance runs 4 waves (256 threads) per workgroup.

#define ZLM_GEMV(NAME, QT, KCAP, RT, STEPS, EXACT)                                                        \
    extern "C" __global__ void __launch_bounds__(256)                                                    \
        NAME(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc, const float* __restrict__ x, \
             float* __restrict__ y, uint32_t rows, uint32_t nb) {                                        \
        GemvArgs a = {w, dsc, w, dsc, x, x, y, y, rows, nb, 0.0f, 0u};                                  \
        gemv<QT, KCAP, 4, RT, STEPS, EXACT, true, PRO_PLAIN, EPI_PLAIN>(a);                             \
    }

// Two-token instances zlm_gemv_<quant>_tok2_g<T> (T = 4, 8, 16: k <= 1024*T):
// matMul at m = 2, one pass over the weights for both tokens, one-row tiles
// (ZLM_GEMVTR, zlm_gemv_<quant>_tok2_g<T>_r<RT>: RT-row tiles, whose lanes
// read each x value once for RT rows),
// fp32 x, the row walked in groups of STEPS chunk steps (the generic loop;
// exact-step forms that issue a whole row's loads at once took 170-450 VGPRs
// with two tokens).  Both x rows fill twice the single-token LDS tile (39 KB
// at the 4096-float tier, 78 KB at 8192, 156 KB at 16384), so the workgroup
// grows with the tier (4, 8, 16 waves) to keep 16 waves per CU.
#define ZLM_GEMVT(NAME, QT, KCAP, WAVES, STEPS) ZLM_GEMVTR(NAME, QT, KCAP, WAVES, 1, STEPS)
#define ZLM_GEMVTR(NAME, QT, KCAP, WAVES, RT, STEPS)                              \
    extern "C" __global__ void __launch_bounds__(WAVES * 64) NAME(GemvArgs a) {   \
        gemv<QT, KCAP, WAVES, RT, STEPS, false, true, PRO_TOK2, EPI_TOK>(a);      \
    }
// STEPS: 2 for the 32-element chunks of q4_0 / q4_1 / q4_k, 4 for q8_0's 16
#define ZLM_GEMV_TOK2(QN, QT, STEPS)                                    \
    ZLM_GEMVT(zlm_gemv_##QN##_tok2_g4, QT, 4096, 4, STEPS)              \
    ZLM_GEMVT(zlm_gemv_##QN##_tok2_g8, QT, 8192, 8, STEPS)              \
    ZLM_GEMVT(zlm_gemv_##QN##_tok2_g16, QT, 16384, 16, STEPS)

// Int-path token instances zlm_gemv_<quant>_q8tok4_g<T> (T = 4, 8: k <=
// 1024*T): matMul at m = 3, 4.  16-wave workgroups (one float4 of each
// token's x per thread at the 4096-float tier); the tiles take 1.375 * T KiB
// per token.  Eight token slots measured slower than the tiled GEMM on most
// shapes (quantizing eight rows per workgroup and twice the LDS reads), so
// from 5 tokens the GEMM runs.
#define ZLM_GEMVQ(NAME, QT, NTOK, KCAP, STEPS) ZLM_GEMVQR(NAME, QT, NTOK, KCAP, STEPS, 1)
#define ZLM_GEMVQR(NAME, QT, NTOK, KCAP, STEPS, RT)                                \
    extern "C" __global__ void __launch_bounds__(1024) NAME(GemvArgs a) {          \
        gemv_int<QT, NTOK, KCAP, 16, STEPS, RT>(a);                                \
    }
#define ZLM_GEMV_Q8TOK(QN, QT, STEPS)                                   \
    ZLM_GEMVQ(zlm_gemv_##QN##_q8tok4_g4, QT, 4, 4096, STEPS)            \
    ZLM_GEMVQ(zlm_gemv_##QN##_q8tok4_g8, QT, 4, 8192, STEPS)
// Two-row tiles (_r2) for launches of 32768 rows and more: each lane reads a
// token's LDS words once for both rows (the nibble quants; q8_0's two LDS
// reads per token gain nothing).
// The 16384-float tier (m = 3, 4, k 8193-16384) for the quants whose
// small-M GEMM carries the min term (q4_1, q4_k).
#define ZLM_GEMV_Q8TOK16(QN, QT, STEPS) ZLM_GEMVQ(zlm_gemv_##QN##_q8tok4_g16, QT, 4, 16384, STEPS)
// Eight token slots at the 4096-float tier (m = 5..8), for the quants whose
// small-M GEMM carries the min term (q4_1, q4_k): there the GEMM's extra
// outer products cost more than the doubled LDS reads of eight slots.
#define ZLM_GEMV_Q8TOK8(QN, QT, STEPS) ZLM_GEMVQ(zlm_gemv_##QN##_q8tok8_g4, QT, 8, 4096, STEPS)
#define ZLM_GEMV_Q8TOK_R2(QN, QT, STEPS)                                \
    ZLM_GEMVQR(zlm_gemv_##QN##_q8tok4_g4_r2, QT, 4, 4096, STEPS, 2)     \
    ZLM_GEMVQR(zlm_gemv_##QN##_q8tok4_g8_r2, QT, 4, 8192, STEPS, 2)

// The fused forms take one GemvArgs: zlm_gemv_<quant>_<form>_s<STEPS> (exact
// steps) and zlm_gemv_<quant>_<form>_g<STEPS> (generic), form one of
//   pair      gate_up: act(gate.x) * (up.x), one gate and one up row per tile
//   norm      RMSNorm(x) then the GEMV
//   normpair  RMSNorm(x) then gate_up
//   resid     y = res + W.x
#define ZLM_GEMVX(NAME, QT, KCAP, RT, STEPS, EXACT, PRO, EPI)                        \
    extern "C" __global__ void __launch_bounds__(256) NAME(GemvArgs a) {            \
        gemv<QT, KCAP, 4, RT, STEPS, EXACT, true, PRO, EPI>(a);                     \
    }
// Prefetching instances zlm_gemv_<quant>_<form>_s<STEPS>_pf (launched at 8
// waves per CU) and ..._pfw16 (16 waves per CU): WAVES waves per workgroup
// (the host reads the block size from the kernel's launch bounds).  The
// ZLM_GEMVX_PFQ instances stage x as int8 planes (q4_0, q4_k, q6_k) and carry
// a q in the suffix (_pfq, _pfqw16, _tallq: 16 waves per CU from 65536 rows),
// which tells the host their summation differs from the batch kernel's.
#define ZLM_GEMVX_PF(NAME, QT, KCAP, WAVES, RT, STEPS, PRO, EPI, FENCE)                       \
    extern "C" __global__ void __launch_bounds__(WAVES * 64) NAME(GemvArgs a) {              \
        gemv<QT, KCAP, WAVES, RT, STEPS, true, true, PRO, EPI, true, FENCE>(a);             \
    }
#define ZLM_GEMVX_PFQ(NAME, QT, KCAP, WAVES, RT, STEPS, PRO, EPI, FENCE)                      \
    extern "C" __global__ void __launch_bounds__(WAVES * 64) NAME(GemvArgs a) {              \
        gemv<QT, KCAP, WAVES, RT, STEPS, true, true, PRO, EPI, true, FENCE, true>(a);       \
    }
// Split-K instances zlm_gemv_<quant>_r1_s<STEPS>_sk<RT> / _resid_s<STEPS>_sk<RT>
// (any row of STEPS chunk steps), ..._sk<RT>x (EXACT: chunks == 64*STEPS):
// W waves share a tile of RT rows (W*SPL == STEPS), one workgroup per CU.
#define ZLM_GEMV_SK(NAME, QT, W, RT, SPL, EPI, XQ, NB, EXACT)                   \
    extern "C" __global__ void __launch_bounds__(W * 64) NAME(GemvArgs a) {     \
        gemv_sk<QT, W, RT, SPL, EPI, XQ, NB, EXACT>(a);                        \
    }
// The same with the parked reduction: one barrier per PARK tiles.
#define ZLM_GEMV_SKP(NAME, QT, W, RT, SPL, EPI, XQ, NB, EXACT, PARK)           \
    extern "C" __global__ void __launch_bounds__(W * 64) NAME(GemvArgs a) {     \
        gemv_sk<QT, W, RT, SPL, EPI, XQ, NB, EXACT, PARK>(a);                  \
    }
#define ZLM_GEMVX_FORMS(QN, QT, KCAP, STEPS, EXACT, SFX)                                           \
    ZLM_GEMVX(zlm_gemv_##QN##_pair_##SFX, QT, KCAP, 2, STEPS, EXACT, PRO_PLAIN, EPI_PAIR)           \
    ZLM_GEMVX(zlm_gemv_##QN##_norm_##SFX, QT, KCAP, 1, STEPS, EXACT, PRO_NORM, EPI_PLAIN)           \
    ZLM_GEMVX(zlm_gemv_##QN##_normpair_##SFX, QT, KCAP, 2, STEPS, EXACT, PRO_NORM, EPI_PAIR)        \
    ZLM_GEMVX(zlm_gemv_##QN##_resid_##SFX, QT, KCAP, 1, STEPS, EXACT, PRO_PLAIN, EPI_RESID)

// Rows of 3-4 chunk steps (4097-8192 elements) for the 32-element-chunk
// quants: the generic loop (two chunk steps per group) over an 8192-element x
// tile, zlm_gemv_<quant>_{r1,pair,norm,normpair,resid}_g8k.  The exact-steps
// instances there hold every step's loads at once (159-264 VGPRs, one to
// three waves per SIMD); these take 62-118.  The host takes them where they
// measured faster.
#define ZLM_GEMV_G8K(QN, QT)                                                                  \
    ZLM_GEMVX(zlm_gemv_##QN##_r1_g8k, QT, 8192, 1, 2, false, PRO_PLAIN, EPI_PLAIN)            \
    ZLM_GEMVX(zlm_gemv_##QN##_pair_g8k, QT, 8192, 2, 2, false, PRO_PLAIN, EPI_PAIR)           \
    ZLM_GEMVX(zlm_gemv_##QN##_norm_g8k, QT, 8192, 1, 2, false, PRO_NORM, EPI_PLAIN)           \
    ZLM_GEMVX(zlm_gemv_##QN##_normpair_g8k, QT, 8192, 2, 2, false, PRO_NORM, EPI_PAIR)        \
    ZLM_GEMVX(zlm_gemv_##QN##_resid_g8k, QT, 8192, 1, 2, false, PRO_PLAIN, EPI_RESID)

// The gate_up pair form with two and four output rows per wave tile
// (zlm_gemv_<quant>_pair_<SFX>_r2 / _r4: RT 4 and 8, gate rows then up rows):
// the row tiles the contract's GpuVariant codes select for the fused gate_up
// (the reference's spec-constant gate_up variants, gpu/kernels/grid.zig:41-53).
#define ZLM_GEMVX_PAIR_TILES(QN, QT, KCAP, STEPS, EXACT, SFX)                                        \
    ZLM_GEMVX(zlm_gemv_##QN##_pair_##SFX##_r2, QT, KCAP, 4, STEPS, EXACT, PRO_PLAIN, EPI_PAIR)       \
    ZLM_GEMVX(zlm_gemv_##QN##_pair_##SFX##_r4, QT, KCAP, 8, STEPS, EXACT, PRO_PLAIN, EPI_PAIR)
#define ZLM_GEMVX_PAIR_TILES_Q4(QN, QT)                       \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 4096, 1, true, s1)           \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 4096, 2, true, s2)           \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 8192, 3, true, s3)           \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 8192, 4, true, s4)           \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 32768, 4, false, g)
#define ZLM_GEMVX_PAIR_TILES_Q8(QN, QT)                       \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 4096, 2, true, s2)           \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 4096, 3, true, s3)           \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 4096, 4, true, s4)           \
    ZLM_GEMVX_PAIR_TILES(QN, QT, 32768, 8, false, g)

// q4_0 / q4_k / q6_k: KCAP = 2048 * STEPS rounded up to a tier.
#define ZLM_GEMV_Q4(QN, QT)                                         \
    ZLM_GEMV_Q4_COMMON(QN, QT)                                      \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s6, QT, 16384, 2, 6, true)

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
    ZLM_GEMV(zlm_gemv_##QN##_r1_g, QT, 32768, 1, 4, false)

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
    ZLM_GEMV(zlm_gemv_##QN##_r1_g, QT, 32768, 1, 8, false)

// Fused forms: q4_0 / q4_k / q6_k at 1-4 steps (k <= 8192; q4_0 also at 6
// steps, k = 12288, where the K-quants' larger fragments would spill), q8_0
// at 2-4, 6, 8 and 12 steps, plus the generic forms.
#define ZLM_GEMVX_Q4(QN, QT)                          \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 1, true, s1)        \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 2, true, s2)        \
    ZLM_GEMVX_FORMS(QN, QT, 8192, 3, true, s3)        \
    ZLM_GEMVX_FORMS(QN, QT, 8192, 4, true, s4)        \
    ZLM_GEMVX_FORMS(QN, QT, 32768, 4, false, g)
#define ZLM_GEMVX_Q8(QN, QT)                          \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 2, true, s2)        \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 3, true, s3)        \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 4, true, s4)        \
    ZLM_GEMVX_FORMS(QN, QT, 8192, 6, true, s6)        \
    ZLM_GEMVX_FORMS(QN, QT, 8192, 8, true, s8)        \
    ZLM_GEMVX_FORMS(QN, QT, 16384, 12, true, s12)     \
    ZLM_GEMVX_FORMS(QN, QT, 32768, 8, false, g)

// f16 / bf16 (8 elements per 16-byte chunk): KCAP = 512 * STEPS rounded up to
// a tier.
#define ZLM_GEMV_F16(QN, QT)                                        \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s1, QT, 4096, 1, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s1, QT, 4096, 2, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s1, QT, 4096, 4, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s2, QT, 4096, 1, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s2, QT, 4096, 2, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r4_s2, QT, 4096, 4, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s4, QT, 4096, 1, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s4, QT, 4096, 2, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s6, QT, 4096, 1, 6, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s8, QT, 4096, 1, 8, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s8, QT, 4096, 2, 8, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s12, QT, 8192, 1, 12, true)         \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s16, QT, 8192, 1, 16, true)         \
    ZLM_GEMV(zlm_gemv_##QN##_r1_g, QT, 32768, 1, 8, false)
#define ZLM_GEMVX_F16(QN, QT)                         \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 2, true, s2)        \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 4, true, s4)        \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 8, true, s8)        \
    ZLM_GEMVX_FORMS(QN, QT, 32768, 8, false, g)

// f32 (4 elements per chunk): KCAP = 256 * STEPS rounded up to a tier.
#define ZLM_GEMV_F32(QN, QT)                                        \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s1, QT, 4096, 1, 1, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s2, QT, 4096, 1, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s2, QT, 4096, 2, 2, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s4, QT, 4096, 1, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s4, QT, 4096, 2, 4, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s8, QT, 4096, 1, 8, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r2_s8, QT, 4096, 2, 8, true)           \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s12, QT, 4096, 1, 12, true)         \
    ZLM_GEMV(zlm_gemv_##QN##_r1_s16, QT, 4096, 1, 16, true)         \
    ZLM_GEMV(zlm_gemv_##QN##_r1_g, QT, 32768, 1, 8, false)
#define ZLM_GEMVX_F32(QN, QT)                         \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 4, true, s4)        \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 8, true, s8)        \
    ZLM_GEMVX_FORMS(QN, QT, 4096, 16, true, s16)      \
    ZLM_GEMVX_FORMS(QN, QT, 32768, 8, false, g)

// zlm_gemv_<quant>_multi_s<STEPS> (exact steps) and zlm_gemv_<quant>_multi_g
// (any k up to 32768): the batch kernel over GemvMultiArgs.
#define ZLM_GEMV_MULTI(NAME, QT, KCAP, STEPS, EXACT)                                 \
    extern "C" __global__ void __launch_bounds__(256) NAME(GemvMultiArgs a) {        \
        gemv_multi<QT, KCAP, 4, STEPS, EXACT>(a);                                   \
    }
// Batch instances: q4_0 / q4_1 / q4_k / q6_k (32 elements per chunk), q8_0
// (16), f16 / bf16 (8), f32 (4); exact steps at the common k, else generic.
#define ZLM_GEMV_MULTI_Q4(QN, QT)                                   \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_s1, QT, 4096, 1, true)     \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_s2, QT, 4096, 2, true)     \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_s4, QT, 8192, 4, true)     \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_g, QT, 32768, 4, false)
#define ZLM_GEMV_MULTI_Q8(QN, QT)                                   \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_s2, QT, 4096, 2, true)     \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_s4, QT, 4096, 4, true)     \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_s8, QT, 8192, 8, true)     \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_g, QT, 32768, 8, false)
#define ZLM_GEMV_MULTI_F16(QN, QT)                                  \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_s8, QT, 4096, 8, true)     \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_g, QT, 32768, 8, false)
#define ZLM_GEMV_MULTI_F32(QN, QT)                                  \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_s16, QT, 4096, 16, true)   \
    ZLM_GEMV_MULTI(zlm_gemv_##QN##_multi_g, QT, 32768, 8, false)
