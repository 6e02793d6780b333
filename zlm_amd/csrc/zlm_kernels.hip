// zlm_kernels.hip -- CDNA4 (gfx950) kernels besides the GEMVs: layout
// conversion, dequant, the activation quantizer, the prefill GEMM and the
// decode-step glue.  Built as a device-only code object (hipcc --genco) and
// loaded by the host library with hipModuleLoad; every entry point is
// extern "C" so the host can look it up by name.
#include "gemv_impl.h"


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

