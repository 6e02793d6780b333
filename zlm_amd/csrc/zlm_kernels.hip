// zlm_kernels.hip -- CDNA4 (gfx950) kernels besides the GEMVs: layout
// conversion, dequant, the activation quantizer, the prefill GEMM and the
// decode-step glue.  Built as a device-only code object (hipcc --genco) and
// loaded by the host library with hipModuleLoad; every entry point is
// extern "C" so the host can look it up by name.
#include "gemv_impl.h"


// ---- repack: raw GGUF blocks -> aligned payload + separate f16 scales -----
// One thread per block; `bb` raw block bytes, `ns` f16 scales (1, or 2 for
// q4_1's d and m) at `soff` within the raw block; the payload is the remaining
// bytes in order, the scales go to dsc[b*ns ..].

extern "C" __global__ void __launch_bounds__(256)
    zlm_repack_split(const uint8_t* __restrict__ raw, uint8_t* __restrict__ payload, uint16_t* __restrict__ dsc,
                     uint64_t nblocks, uint32_t bb, uint32_t soff, uint32_t ns) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* src = raw + b * bb;
    const uint32_t send = soff + 2 * ns;
    uint8_t* dst = payload + b * (bb - 2 * ns);
    for (uint32_t i = 0; i < ns; i++)
        dsc[b * ns + i] = static_cast<uint16_t>(src[soff + 2 * i] | (static_cast<uint16_t>(src[soff + 2 * i + 1]) << 8));
    uint32_t o = 0;
    for (uint32_t i = 0; i < bb; i++) {
        if (i >= soff && i < send) continue;
        dst[o++] = src[i];
    }
}

// getScaleMinK4 (reference quant/k_quants.zig:24-32): the 6-bit scale and min
// of sub-block j (0..7) from the 12 packed bytes.
__device__ __forceinline__ void scale_min_k4_u8(int j, const uint8_t* q, uint32_t& sc, uint32_t& mn) {
    if (j < 4) {
        sc = q[j] & 63u;
        mn = q[j + 4] & 63u;
    } else {
        sc = (q[j + 4] & 15u) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// q4_k raw super-block (reference quant/k_quants.zig:34-72: f16 d, f16 dmin,
// 12 packed scale bytes, 128 qs bytes) -> payload [nb][128 B qs] and a 20-byte
// record per block: dword 0 = d | dmin << 16 (the raw bytes 0..3), dword 1+g =
// sc[2g] | sc[2g+1] << 8 | mn[2g] << 16 | mn[2g+1] << 24.  A GEMV lane reads
// the one dword its 32-element group needs and converts the bytes directly.
extern "C" __global__ void __launch_bounds__(256)
    zlm_repack_q4_k(const uint8_t* __restrict__ raw, uint8_t* __restrict__ payload, uint32_t* __restrict__ rec,
                    uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* src = raw + b * 144;
    const uint4* qs = reinterpret_cast<const uint4*>(src + 16);
    uint4* dst = reinterpret_cast<uint4*>(payload + b * 128);
    for (int i = 0; i < 8; i++) dst[i] = qs[i];
    uint32_t* o = rec + b * 5;
    o[0] = *reinterpret_cast<const uint32_t*>(src);
    for (int g = 0; g < 4; g++) {
        uint32_t s0, m0, s1, m1;
        scale_min_k4_u8(2 * g, src + 4, s0, m0);
        scale_min_k4_u8(2 * g + 1, src + 4, s1, m1);
        o[1 + g] = s0 | (s1 << 8) | (m0 << 16) | (m1 << 24);
    }
}

// q6_k raw super-block (reference quant/k_quants.zig: ql[128], qh[64], int8
// scales[16], f16 d; 210 bytes) -> payload [nb][128 B ql] (as is) and an
// 84-byte record per block.  GEMV chunk p (n = p/4, h = (p/2)&1, ws = p&1)
// reads ql[64n + 32ws + 16h ..+16]; its byte j = 4i + b (ql dword i) holds
// element 128n + 32ws + 16h + j in the low nibble (qh[32n + 16h + j] bits 2ws)
// and that element + 64 in the high nibble (bits 4 + 2ws).  Record bytes
// 8p + 4(i/2) + b carry those two 2-bit parts (low-nibble element at bits 0-1,
// high at 2-3 for even i; at 4-5 and 6-7 for odd i), bytes 64..65 d, bytes
// 68 + 2p and 69 + 2p the scales of the chunk's two 16-element runs,
// scales[8n + h + 2ws] and scales[8n + 4 + h + 2ws].
extern "C" __global__ void __launch_bounds__(256)
    zlm_repack_q6_k(const uint8_t* __restrict__ raw, uint8_t* __restrict__ payload, uint8_t* __restrict__ rec,
                    uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* src = raw + b * 210;
    const uint8_t *ql = src, *qh = src + 128, *sc = src + 192;
    uint8_t* dst = payload + b * 128;
    for (int i = 0; i < 128; i++) dst[i] = ql[i];
    uint8_t* o = rec + b * 84;
    for (int p = 0; p < 8; p++) {
        const int n = p >> 2, h = (p >> 1) & 1, ws = p & 1;
        for (int k = 0; k < 8; k++) o[8 * p + k] = 0;
        for (int j = 0; j < 16; j++) {
            const int i = j >> 2, bb = j & 3;
            const uint32_t q = qh[32 * n + 16 * h + j];
            const uint32_t lo2 = (q >> (2 * ws)) & 3u, hi2 = (q >> (4 + 2 * ws)) & 3u;
            o[8 * p + 4 * (i >> 1) + bb] |= static_cast<uint8_t>((lo2 | (hi2 << 2)) << (4 * (i & 1)));
        }
        o[68 + 2 * p] = sc[8 * n + h + 2 * ws];
        o[69 + 2 * p] = sc[8 * n + 4 + h + 2 * ws];
    }
    o[64] = src[208];
    o[65] = src[209];
    o[66] = 0;
    o[67] = 0;
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

// standard.dequantQ4_1Block (reference quant/standard.zig:138-148): q*d + m,
// the product and the sum rounded separately.
extern "C" __global__ void __launch_bounds__(256)
    zlm_dequant_q4_1(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc, float* __restrict__ out,
                     uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* q = w + b * 16;
    const float d = h2f(dsc[2 * b]), m = h2f(dsc[2 * b + 1]);
    float* o = out + b * 32;
    for (int j = 0; j < 16; j++) {
        o[j] = static_cast<float>(q[j] & 15) * d + m;
        o[16 + j] = static_cast<float>(q[j] >> 4) * d + m;
    }
}

// The float types, one element per "block" (reference quant/floats.zig):
// f32 as is, f16 widened exactly, bf16 as the top half of an f32.
extern "C" __global__ void __launch_bounds__(256)
    zlm_dequant_f32(const uint8_t* __restrict__ w, const uint16_t* __restrict__, float* __restrict__ out,
                    uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = reinterpret_cast<const float*>(w)[i];
}

extern "C" __global__ void __launch_bounds__(256)
    zlm_dequant_f16(const uint8_t* __restrict__ w, const uint16_t* __restrict__, float* __restrict__ out,
                    uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = h2f(reinterpret_cast<const uint16_t*>(w)[i]);
}

extern "C" __global__ void __launch_bounds__(256)
    zlm_dequant_bf16(const uint8_t* __restrict__ w, const uint16_t* __restrict__, float* __restrict__ out,
                     uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __builtin_bit_cast(float, static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(w)[i]) << 16);
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
    zlm_dequant_q4_k(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc, float* __restrict__ out,
                     uint64_t nblocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint32_t* rec = reinterpret_cast<const uint32_t*>(dsc) + b * 5;
    const float d = h2f(rec[0]), dmin = h2f(rec[0] >> 16);
    float* o = out + b * 256;
    for (int g = 0; g < 4; g++) {
        const uint32_t sm = rec[1 + g];
        const float d1 = d * ub(sm, 0), m1 = dmin * ub(sm, 2), d2 = d * ub(sm, 1), m2 = dmin * ub(sm, 3);
        const uint8_t* q = w + b * 128 + 32 * g;
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
    const uint8_t* ql = w + b * 128;
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(dsc) + b * 84;
    const float d = h2f(static_cast<uint32_t>(rec[64]) | (static_cast<uint32_t>(rec[65]) << 8));
    float* o = out + b * 256;
    for (int p = 0; p < 8; p++) {  // the GEMV's chunks (zlm_repack_q6_k)
        const int n = p >> 2, h = (p >> 1) & 1, ws = p & 1;
        const uint8_t* q = ql + 64 * n + 32 * ws + 16 * h;
        const float sa = static_cast<float>(static_cast<int8_t>(rec[68 + 2 * p]));
        const float sb = static_cast<float>(static_cast<int8_t>(rec[69 + 2 * p]));
        const int e = 128 * n + 32 * ws + 16 * h;
        for (int j = 0; j < 16; j++) {
            const int i = j >> 2;
            const uint32_t t = rec[8 * p + 4 * (i >> 1) + (j & 3)] >> (4 * (i & 1));
            const int qa = (q[j] & 15) | static_cast<int>((t & 3u) << 4);
            const int qb = (q[j] >> 4) | static_cast<int>(((t >> 2) & 3u) << 4);
            o[e + j] = static_cast<float>(qa - 32) * (d * sa);
            o[e + j + 64] = static_cast<float>(qb - 32) * (d * sb);
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
// mt*32: qx [mt][nb][32 tokens][32 B], dx [mt][nb][32 tokens] and, when `ds`
// is not null, ds = dx * f32(sum of the block's q) in the same order (the
// min-term factor of q4_1 / q4_k); padding tokens are zeros.  Eight threads
// per (token, block) slot, numbered in output order (slot i is threads 8i ..
// 8i+7), each loading one float4 of the block and writing its 4 quantized
// bytes: a wave reads 8 blocks as 128-byte runs and writes 256 contiguous
// bytes of qx; the block's amax and sum meet across the 8 lanes (max and
// integer sum: the same values in any order), so every output is bit for bit
// the one-thread-per-block quantizer's.  At 512 x 4096: 6.3 -> 5.5 us (one
// thread per slot before; numbering the threads in input order instead, so a
// wave reads 1 KiB of one token's row, measured 5.9 us).
extern "C" __global__ void __launch_bounds__(256)
    zlm_quantize_q8_tiled(const float* __restrict__ x, int8_t* __restrict__ qx, float* __restrict__ dx,
                          uint32_t m, uint32_t nb, uint32_t mt, float* __restrict__ ds) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t nslot = static_cast<uint64_t>(mt) * 32 * nb;
    const uint64_t slot = min(i / 8, nslot - 1);  // whole waves stay in the shuffles
    const uint32_t part = static_cast<uint32_t>(i % 8);
    const uint64_t tb = slot / 32;  // token tile * nb + block
    const uint32_t b = static_cast<uint32_t>(tb % nb);
    const uint32_t t = static_cast<uint32_t>(tb / nb) * 32 + static_cast<uint32_t>(slot % 32);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (t < m) v = reinterpret_cast<const float4*>(x + (static_cast<uint64_t>(t) * nb + b) * 32)[part];
    float d;
    int32_t s;
    const uint32_t wv = q8_quant4(v, d, s);
    s = sum8(s);
    if (i / 8 >= nslot) return;
    reinterpret_cast<uint32_t*>(qx + slot * 32)[part] = wv;
    if (part == 0) {
        dx[slot] = d;
        if (ds) ds[slot] = d * static_cast<float>(s);
    }
}

// The prefill GEMM's tiled weight layout, rows padded to rt*32: payload
// [rt][nb][32 rows][PB bytes] (PB = 16 for q4_0, 32 for q8_0), scales
// [rt][nb][32 rows]; padding rows have zero scales.  One thread per (row,
// block) of the padded matrix.
template <int PB>
__device__ __forceinline__ void tile_blocks(const uint8_t* __restrict__ payload, const uint16_t* __restrict__ scales,
                                            uint8_t* __restrict__ tpayload, uint16_t* __restrict__ tscales,
                                            uint32_t rows, uint32_t nb, uint32_t rt) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<uint64_t>(rt) * 32 * nb) return;
    const uint32_t r = static_cast<uint32_t>(i / nb), b = static_cast<uint32_t>(i % nb);
    const uint64_t slot = (static_cast<uint64_t>(r / 32) * nb + b) * 32 + (r % 32);
    const uint64_t src = static_cast<uint64_t>(r) * nb + b;
    uint16_t d = 0;
#pragma unroll
    for (int j = 0; j < PB / 16; j++) {
        uint4 q = make_uint4(0u, 0u, 0u, 0u);
        if (r < rows) q = reinterpret_cast<const uint4*>(payload)[src * (PB / 16) + j];
        reinterpret_cast<uint4*>(tpayload)[slot * (PB / 16) + j] = q;
    }
    if (r < rows) d = scales[src];
    tscales[slot] = d;
}

extern "C" __global__ void __launch_bounds__(256)
    zlm_tile_q4_0(const uint8_t* __restrict__ payload, const uint16_t* __restrict__ scales,
                  uint8_t* __restrict__ tpayload, uint16_t* __restrict__ tscales, uint32_t rows, uint32_t nb,
                  uint32_t rt) {
    tile_blocks<16>(payload, scales, tpayload, tscales, rows, nb, rt);
}

extern "C" __global__ void __launch_bounds__(256)
    zlm_tile_q8_0(const uint8_t* __restrict__ payload, const uint16_t* __restrict__ scales,
                  uint8_t* __restrict__ tpayload, uint16_t* __restrict__ tscales, uint32_t rows, uint32_t nb,
                  uint32_t rt) {
    tile_blocks<32>(payload, scales, tpayload, tscales, rows, nb, rt);
}

// The tiled layout of the min-carrying types (q4_1, q4_k): per 32-element
// block of a row, 16 nibble bytes in q4_0 order (byte j: element j low,
// element j+16 high) and a float2 (scale, min) such that the block's values
// are scale * nib + min: payload [rt][nb][32 rows][16 B], sm [rt][nb][32 rows].
// Padding rows are zeros.  One thread per (row, 32-element block).
//
// q4_1 (split layout, reference quant/standard.zig:138-148): the payload as
// is, (d, m).
extern "C" __global__ void __launch_bounds__(256)
    zlm_tile_q4_1(const uint8_t* __restrict__ payload, const uint16_t* __restrict__ scales,
                  uint8_t* __restrict__ tpayload, float2* __restrict__ tsm, uint32_t rows, uint32_t nb, uint32_t rt) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<uint64_t>(rt) * 32 * nb) return;
    const uint32_t r = static_cast<uint32_t>(i / nb), b = static_cast<uint32_t>(i % nb);
    const uint64_t slot = (static_cast<uint64_t>(r / 32) * nb + b) * 32 + (r % 32);
    const uint64_t src = static_cast<uint64_t>(r) * nb + b;
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    float2 sm = make_float2(0.0f, 0.0f);
    if (r < rows) {
        q = reinterpret_cast<const uint4*>(payload)[src];
        sm = make_float2(h2f(scales[2 * src]), h2f(scales[2 * src + 1]));
    }
    reinterpret_cast<uint4*>(tpayload)[slot] = q;
    tsm[slot] = sm;
}

// q4_k (the zlm_repack_q4_k layout of the 144-byte super-blocks, reference
// quant/k_quants.zig:34-72): 32-element block b of a row is sub-block j = b%8
// of super-block b/8, the low (j even) or high (j odd) nibbles of
// qs[32*(j/2) .. +32]; scale = d*sc_j, min = -(dmin*mn_j) (getScaleMinK4, the
// products of the reference's int path, quantized.zig:111-123).
extern "C" __global__ void __launch_bounds__(256)
    zlm_tile_q4_k(const uint8_t* __restrict__ payload, const uint16_t* __restrict__ records,
                  uint8_t* __restrict__ tpayload, float2* __restrict__ tsm, uint32_t rows, uint32_t nb, uint32_t rt) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<uint64_t>(rt) * 32 * nb) return;
    const uint32_t r = static_cast<uint32_t>(i / nb), b = static_cast<uint32_t>(i % nb);
    const uint64_t slot = (static_cast<uint64_t>(r / 32) * nb + b) * 32 + (r % 32);
    uint32_t packed[4] = {0u, 0u, 0u, 0u};
    float2 sm = make_float2(0.0f, 0.0f);
    if (r < rows) {
        const uint64_t sb = static_cast<uint64_t>(r) * (nb / 8) + b / 8;
        const uint32_t j = b % 8, sh = 4 * (j & 1);
        const uint32_t* rec = reinterpret_cast<const uint32_t*>(records) + sb * 5;
        const uint32_t sms = rec[1 + j / 2];
        const float sc = ub(sms, j & 1), mn = ub(sms, 2 + (j & 1));
        sm = make_float2(h2f(rec[0]) * sc, -(h2f(rec[0] >> 16) * mn));
        const uint8_t* qs = payload + sb * 128 + 32 * (j / 2);
        for (int e = 0; e < 16; e++) {
            const uint32_t lo = (qs[e] >> sh) & 15u, hi = (qs[e + 16] >> sh) & 15u;
            packed[e / 4] |= (lo | (hi << 4)) << (8 * (e % 4));
        }
    }
    reinterpret_cast<uint4*>(tpayload)[slot] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    tsm[slot] = sm;
}

// ---- device copy (16-byte granules; the traffic-counter calibration kernel) --

extern "C" __global__ void __launch_bounds__(256)
    zlm_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, uint64_t n16) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

// ---- prefill GEMM: Q4_0 / Q8_0 weights x Q8_0-quantized activations, int8 MFMA ----
//
// out[t*rows + r] = sum_b dw[r,b] * dx[t,b] * sum_j w[r,b,j] * qx[t,b,j], with
// w = nib - 8 for q4_0 and the int8 quant for q8_0 (the int paths of
// reference kernels/quantized.zig:49-55 and :149-156 over the activation
// quantizer of matvec/layout.zig:458-476, i.e. zlm_quantize_q8's output).
// q8_0 is the same kernel with the weight bytes taken as they are (lanes 0-31
// hold bytes 0..15 of a row's block, lanes 32-63 bytes 16..31, the B operand's
// k split) and no nibble factor.
//
// v_mfma_i32_32x32x32_i8 computes one 32-element block for a 32-token x
// 32-row tile: A = activations (lane l: token l%32, block elements
// 16*(l/32)..+15 of qx), B = weights (lane l: row l%32, the same elements: the
// low nibbles of the row's 16 block bytes for lanes 0-31, the high nibbles for
// 32-63), D[t = 8*(i/4) + 4*(l/32) + i%4][r = l%32].  A nibble n enters as the
// int8 16*(n-8) (n^8 in the high nibble), so each block dot is exact in int32.
// A wave owns 64 tokens (two 32-token tiles) x 32 rows.  The block's two scale
// matrices dx[t]*dw[r] (one per token tile) are outer products of vectors:
// one v_mfma_f32_32x32x1_2b_f32 (block 0 from lanes 0-31: token tile 0's dx
// by dw, block 1 from lanes 32-63: token tile 1's dx by dw) yields both, in
// the D layout of the int8 results (block 0 in result registers 0-15, block 1
// in 16-31), on the matrix pipe; the VALU does one convert and one fma per
// output.  Operand addresses are a wave-uniform base (per block, in SGPRs)
// plus a per-lane offset fixed for the whole loop, so the loads need no
// per-block address arithmetic on the VALU.  A workgroup of 4 waves owns 128
// tokens x 64 rows; padding tokens and rows of the tiled layouts are zeros and
// their outputs are not stored, blocks past the end get a zero scale.
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

struct GemmBlk {
    uint4 a0, a1, w;
    uint32_t d;      // q4_0 / q8_0: the f16 weight scale
    float x;         // dx of this lane's token tile (lanes 0-31: tile 0, 32-63: tile 1)
    float2 sm;       // q4_1 / q4_k: (scale, min)
    float s;         // q4_1 / q4_k: dx * sum(q) of this lane's token tile
};

constexpr bool gemm_has_min(int qt) { return qt == Q4_1 || qt == Q4_K; }

// Per-wave operand buffers (raw buffer resources at the wave's tile bases,
// wave-uniform) with per-lane byte offsets fixed for the whole loop; a block's
// loads add its wave-uniform byte offset in an SGPR.
struct GemmPtrs {
    __amdgpu_buffer_rsrc_t a, w, sc, x, s;  // qx, weights, scales, dx, dx*sum(q)
    uint32_t a1;                            // token tile 1's byte offset in `a`
    uint32_t oa, ow, osc, ox;               // lane byte offsets
};

// At most 168 VGPRs per wave (3 waves per SIMD): the q4_0 GEMM takes 119, so
// the 3 waves per SIMD that the 12288 x 512 launch places are all resident
// at once (the split form 120: two of its 8-wave workgroups per CU); the
// min-carrying quants' kernels 156-159.
#ifndef ZLM_GEMM_WAVES_PER_EU
#define ZLM_GEMM_WAVES_PER_EU 3
#endif

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ uint4 gemm_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

template <int QT>
__device__ __forceinline__ void gemm_load(GemmBlk& g, const GemmPtrs& p, uint32_t b) {
    constexpr uint32_t kWStride = QT == Q8_0 ? 1024 : 512;  // tiled weight bytes per block
    g.a0 = gemm_ld16(p.a, p.oa, b * 1024);
    g.a1 = gemm_ld16(p.a, p.oa, p.a1 + b * 1024);
    g.w = gemm_ld16(p.w, p.ow, b * kWStride);
    if constexpr (gemm_has_min(QT)) {
        // two dword loads (the compiler merges them into one dwordx2; the
        // 64-bit buffer-load builtin compiled to a single dword load here)
        const uint32_t sx = __builtin_amdgcn_raw_buffer_load_b32(p.sc, static_cast<int>(p.osc), static_cast<int>(b * 256), 0);
        const uint32_t sy =
            __builtin_amdgcn_raw_buffer_load_b32(p.sc, static_cast<int>(p.osc + 4), static_cast<int>(b * 256), 0);
        g.sm = make_float2(__builtin_bit_cast(float, sx), __builtin_bit_cast(float, sy));
        g.s = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(p.s, static_cast<int>(p.ox),
                                                                             static_cast<int>(b * 128), 0));
    } else {
        g.d = __builtin_amdgcn_raw_buffer_load_b16(p.sc, static_cast<int>(p.osc), static_cast<int>(b * 64), 0);
    }
    g.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(p.x, static_cast<int>(p.ox),
                                                                         static_cast<int>(b * 128), 0));
}

struct GemmI {
    v16i i0, i1;  // the block's exact int32 dots, token tiles 0 and 1
};

// A block's two int8 MFMAs (both token tiles share the unpacked weights).
// The B operand of a block's int8 MFMA from this lane's 16 weight bytes: q8_0
// as they are; q4_0 nibbles as the int8 16*(n-8) (lanes 0-31 the low
// nibbles, 32-63 the high); q4_1 / q4_k nibbles unsigned.
template <int QT>
__device__ __forceinline__ v4i gemm_unpack(const uint4 w, bool lo_half, int sh) {
    v4i bv;
    if constexpr (QT == Q8_0) {
        bv = v4i{static_cast<int>(w.x), static_cast<int>(w.y), static_cast<int>(w.z), static_cast<int>(w.w)};
    } else if constexpr (gemm_has_min(QT)) {
        const int rs = lo_half ? 0 : 4;
        bv.x = static_cast<int>((w.x >> rs) & 0x0F0F0F0Fu);
        bv.y = static_cast<int>((w.y >> rs) & 0x0F0F0F0Fu);
        bv.z = static_cast<int>((w.z >> rs) & 0x0F0F0F0Fu);
        bv.w = static_cast<int>((w.w >> rs) & 0x0F0F0F0Fu);
    } else {
        bv.x = static_cast<int>(((w.x << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
        bv.y = static_cast<int>(((w.y << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
        bv.z = static_cast<int>(((w.z << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
        bv.w = static_cast<int>(((w.w << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
    }
    return bv;
}

// A block's two int8 MFMAs (both token tiles share the unpacked weights).
template <int QT>
__device__ __forceinline__ GemmI gemm_int(const GemmBlk& g, bool lo_half, int sh) {
    const v4i bv = gemm_unpack<QT>(g.w, lo_half, sh);
    const v4i a0 = {static_cast<int>(g.a0.x), static_cast<int>(g.a0.y), static_cast<int>(g.a0.z),
                    static_cast<int>(g.a0.w)};
    const v4i a1 = {static_cast<int>(g.a1.x), static_cast<int>(g.a1.y), static_cast<int>(g.a1.z),
                    static_cast<int>(g.a1.w)};
    const v16i zi = {};
    GemmI r;
    r.i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bv, zi, 0, 0, 0);
    r.i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bv, zi, 0, 0, 0);
    return r;
}

// A block's scale matrices (and, with a min term, its accumulated min
// outer products); a block past the end gets zero scales.
template <int QT>
__device__ __forceinline__ v32f gemm_scale(const GemmBlk& g, bool valid, v32f& accm) {
    float bw;
    if constexpr (gemm_has_min(QT)) {
        bw = g.sm.x;
        // the min term sum_b (dx*sum q)[t] * min[r]: outer products the matrix
        // pipe accumulates by itself (both token tiles in one instruction)
        accm = __builtin_amdgcn_mfma_f32_32x32x1f32(valid ? g.s : 0.0f, g.sm.y, accm, 0, 0, 0);
    } else {
        bw = h2f(g.d);
    }
    // q4_0: the 16 of the nibble encoding is divided out at the store
    const v32f zf = {};
    return __builtin_amdgcn_mfma_f32_32x32x1f32(valid ? g.x : 0.0f, bw, zf, 0, 0, 0);
}

// The VALU epilogue of a block: one convert and one fma per output.
__device__ __forceinline__ void gemm_acc(const v32f& c, const GemmI& I, v16f& acc0, v16f& acc1) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
        acc0[i] = fmaf(c[i], static_cast<float>(I.i0[i]), acc0[i]);
        acc1[i] = fmaf(c[16 + i], static_cast<float>(I.i1[i]), acc1[i]);
    }
}

// Operands come from the tiled layouts (zlm_quantize_q8_tiled, zlm_tile_q4_0 /
// zlm_tile_q8_0), so each per-block load of a wave is one contiguous run: 1 KiB
// of qx per 32-token tile, 512 B (q4_0) or 1 KiB (q8_0) of weights and 64 B of
// scales per 32-row tile.
// q4_1 / q4_k take the (scale, min) tiles (zlm_tile_q4_1 / zlm_tile_q4_k) and
// the quantizer's dx*sum(q): out = sum_b scale*dx*dot(nib, q) + min*dx*sum(q).
//
// SPLIT = 2 or 4 (8- or 16-wave workgroups): each group of 4 waves takes the
// same four output tiles over its part of the row's blocks, and the other
// groups' sums reach group 0 through LDS (added in a fixed order), for small
// grids, where a lone wave per SIMD would run its block chain latency-bound.
template <int QT, int SPLIT = 1>
__device__ __forceinline__ void gemm_tiles(const uint8_t* __restrict__ wq, const void* __restrict__ wsc,
                                           const int8_t* __restrict__ qx, const float* __restrict__ dx,
                                           const float* __restrict__ ds, float* __restrict__ out, uint32_t rows,
                                           uint32_t m, uint32_t nb, uint32_t mt) {
    static_assert(SPLIT == 1 || SPLIT == 2 || SPLIT == 4, "one, two or four block ranges");
    const int lane = threadIdx.x & 63;
    const uint32_t wall = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const uint32_t wid = SPLIT == 1 ? wall : wall & 3;  // output tile
    const uint32_t kh = SPLIT == 1 ? 0u : wall >> 2;    // block range
    const uint32_t tok0 = blockIdx.y * 128 + 64 * (wid & 1);  // multiple of 32
    const uint32_t row0 = blockIdx.x * 64 + 32 * (wid >> 1);  // multiple of 32
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const uint32_t tt0 = min(tok0 / 32, mt - 1), tt1 = min(tok0 / 32 + 1, mt - 1);
    const uint32_t rt = min(row0 / 32, (rows + 31) / 32 - 1);  // a wave past the last tile re-reads it, stores nothing
    // the wave's buffers start at its first token tile / its row tile
    constexpr uint32_t kWStride = QT == Q8_0 ? 1024 : 512;
    constexpr uint32_t kScBytes = gemm_has_min(QT) ? 8 : 2;
    GemmPtrs ptr;
    ptr.a = gemm_rsrc(qx + static_cast<size_t>(tt0) * nb * 1024, (mt - tt0) * nb * 1024);
    ptr.a1 = (tt1 - tt0) * nb * 1024;
    ptr.oa = l32 * 32 + 16 * half;
    ptr.w = gemm_rsrc(wq + static_cast<size_t>(rt) * nb * kWStride, nb * kWStride);
    ptr.ow = QT == Q8_0 ? l32 * 32 + 16 * half : l32 * 16;
    ptr.sc = gemm_rsrc(static_cast<const uint8_t*>(wsc) + static_cast<size_t>(rt) * nb * 32 * kScBytes,
                       nb * 32 * kScBytes);
    ptr.osc = l32 * kScBytes;
    // lanes 0-31 read token tile 0's dx, lanes 32-63 tile 1's (the A operand
    // of the two-block outer product)
    ptr.x = gemm_rsrc(dx + static_cast<size_t>(tt0) * nb * 32, (mt - tt0) * nb * 128);
    ptr.s = gemm_rsrc(gemm_has_min(QT) ? ds + static_cast<size_t>(tt0) * nb * 32 : dx, (mt - tt0) * nb * 128);
    ptr.ox = ((half ? (tt1 - tt0) * nb * 32 : 0u) + l32) * 4;
    const int sh = half ? 0 : 4;  // q4_0: lanes 0-31 take the low nibbles, 32-63 the high
    const bool lo_half = half == 0;

    v16f acc0 = {}, acc1 = {};
    v32f accm = {};
    // Two operand sets, A and B, alternate: one set's loads are in flight
    // while the other's block is computed.  The scheduling barriers keep each
    // set's loads ahead of the compute (the scheduler would otherwise sink them
    // next to their uses), and the ping-pong needs no register copies.
    // (Issuing block b+1's MFMAs ahead of block b's epilogue -- a software
    // pipeline at 164 VGPRs -- measured the same; VALU and MFMA of different
    // waves co-issue only in part on gfx950, so the kernel stays VALU-bound.)
    // this wave's blocks [b0, b1): all of them, or one of SPLIT even-length parts
    const uint32_t nbh = SPLIT == 1 ? nb : (nb + 2 * SPLIT - 1) / (2 * SPLIT) * 2;
    const uint32_t b0 = min(kh * nbh, nb), b1 = min(b0 + nbh, nb);
    GemmBlk A, B;
    gemm_load<QT>(A, ptr, min(b0, nb - 1));
    for (uint32_t b = b0; b < b1; b += 2) {
        gemm_load<QT>(B, ptr, min(b + 1, nb - 1));
        __builtin_amdgcn_sched_barrier(0);
        {
            const GemmI I = gemm_int<QT>(A, lo_half, sh);
            gemm_acc(gemm_scale<QT>(A, b < b1, accm), I, acc0, acc1);
        }
        __builtin_amdgcn_sched_barrier(0);
        gemm_load<QT>(A, ptr, min(b + 2, nb - 1));
        __builtin_amdgcn_sched_barrier(0);
        {
            const GemmI I = gemm_int<QT>(B, lo_half, sh);
            gemm_acc(gemm_scale<QT>(B, b + 1 < b1, accm), I, acc0, acc1);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (SPLIT == 2) {
        // the second half's sums (and min terms) to the first half's waves
        constexpr int NV = gemm_has_min(QT) ? 64 : 32;
        __shared__ float red[4][NV][kWave];
        if (kh == 1) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                red[wid][i][lane] = acc0[i];
                red[wid][16 + i][lane] = acc1[i];
            }
            if constexpr (gemm_has_min(QT)) {
#pragma unroll
                for (int i = 0; i < 32; i++) red[wid][32 + i][lane] = accm[i];
            }
        }
        __syncthreads();
        if (kh == 1) return;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            acc0[i] += red[wid][i][lane];
            acc1[i] += red[wid][16 + i][lane];
        }
        if constexpr (gemm_has_min(QT)) {
#pragma unroll
            for (int i = 0; i < 32; i++) accm[i] += red[wid][32 + i][lane];
        }
    }
    if constexpr (SPLIT == 4) {
        // groups 2 and 3 add into 0 and 1, then group 1 into 0: the order is
        // fixed, (g0 + g2) + (g1 + g3)
        static_assert(!gemm_has_min(QT), "four block ranges: q4_0 / q8_0");
        __shared__ float red[2][4][32][kWave];
        if (kh >= 2) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                red[kh - 2][wid][i][lane] = acc0[i];
                red[kh - 2][wid][16 + i][lane] = acc1[i];
            }
        }
        __syncthreads();
        if (kh < 2) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                acc0[i] += red[kh][wid][i][lane];
                acc1[i] += red[kh][wid][16 + i][lane];
            }
        }
        __syncthreads();
        if (kh == 1) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                red[0][wid][i][lane] = acc0[i];
                red[0][wid][16 + i][lane] = acc1[i];
            }
        }
        __syncthreads();
        if (kh != 0) return;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            acc0[i] += red[0][wid][i][lane];
            acc1[i] += red[0][wid][16 + i][lane];
        }
    }
    constexpr float kOut = QT == Q4_0 ? 0.0625f : 1.0f;
    const uint32_t r = row0 + l32;
    if (r < rows) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t t = tok0 + 8 * (i / 4) + 4 * half + (i % 4);
            float v0 = acc0[i] * kOut, v1 = acc1[i] * kOut;
            if constexpr (gemm_has_min(QT)) {
                v0 += accm[i];
                v1 += accm[16 + i];
            }
            if (t < m) out[static_cast<size_t>(t) * rows + r] = v0;
            if (t + 32 < m) out[static_cast<size_t>(t + 32) * rows + r] = v1;
        }
    }
}

// The unsplit tiled GEMMs, for grids of three or more workgroups per CU
// (q4_0 / q8_0; configs[4] is one) or more than one (q4_1 / q4_k: nb is the
// row's 32-element block count, k/32 for both).  There the split form below
// is no faster: its 8-wave workgroups run two per CU and re-read more of the
// weight panels through L2.
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q4_0_q8(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ qx,
                     const float* __restrict__ dx, float* __restrict__ out, uint32_t rows, uint32_t m, uint32_t nb,
                     uint32_t mt) {
    gemm_tiles<Q4_0>(wq, wd, qx, dx, nullptr, out, rows, m, nb, mt);
}

extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q8_0_q8(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ qx,
                     const float* __restrict__ dx, float* __restrict__ out, uint32_t rows, uint32_t m, uint32_t nb,
                     uint32_t mt) {
    gemm_tiles<Q8_0>(wq, wd, qx, dx, nullptr, out, rows, m, nb, mt);
}

extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q4_1_q8(const uint8_t* __restrict__ wq, const float2* __restrict__ wsm, const int8_t* __restrict__ qx,
                     const float* __restrict__ dx, const float* __restrict__ ds, float* __restrict__ out,
                     uint32_t rows, uint32_t m, uint32_t nb, uint32_t mt) {
    gemm_tiles<Q4_1>(wq, wsm, qx, dx, ds, out, rows, m, nb, mt);
}

extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q4_k_q8(const uint8_t* __restrict__ wq, const float2* __restrict__ wsm, const int8_t* __restrict__ qx,
                     const float* __restrict__ dx, const float* __restrict__ ds, float* __restrict__ out,
                     uint32_t rows, uint32_t m, uint32_t nb, uint32_t mt) {
    gemm_tiles<Q4_K>(wq, wsm, qx, dx, ds, out, rows, m, nb, mt);
}

// The tiled GEMMs with each tile's blocks split over two 4-wave groups
// (gemm_tiles SPLIT = 2), for grids of two workgroups per CU (q4_0 / q8_0)
// or one (q4_1 / q4_k).
extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q4_0_q8_k2(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                        const int8_t* __restrict__ qx, const float* __restrict__ dx, float* __restrict__ out,
                        uint32_t rows, uint32_t m, uint32_t nb, uint32_t mt) {
    gemm_tiles<Q4_0, 2>(wq, wd, qx, dx, nullptr, out, rows, m, nb, mt);
}

extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q8_0_q8_k2(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                        const int8_t* __restrict__ qx, const float* __restrict__ dx, float* __restrict__ out,
                        uint32_t rows, uint32_t m, uint32_t nb, uint32_t mt) {
    gemm_tiles<Q8_0, 2>(wq, wd, qx, dx, nullptr, out, rows, m, nb, mt);
}

// Four block ranges (16-wave workgroups, 4 waves per SIMD), for grids of up
// to one workgroup per CU: q4_0 / q8_0 only, whose 121 VGPRs fit; the
// min-carrying kernels' 159 do not.
extern "C" __global__ void __launch_bounds__(1024)
    zlm_gemm_q4_0_q8_k4(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                        const int8_t* __restrict__ qx, const float* __restrict__ dx, float* __restrict__ out,
                        uint32_t rows, uint32_t m, uint32_t nb, uint32_t mt) {
    gemm_tiles<Q4_0, 4>(wq, wd, qx, dx, nullptr, out, rows, m, nb, mt);
}

extern "C" __global__ void __launch_bounds__(1024)
    zlm_gemm_q8_0_q8_k4(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                        const int8_t* __restrict__ qx, const float* __restrict__ dx, float* __restrict__ out,
                        uint32_t rows, uint32_t m, uint32_t nb, uint32_t mt) {
    gemm_tiles<Q8_0, 4>(wq, wd, qx, dx, nullptr, out, rows, m, nb, mt);
}

extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q4_1_q8_k2(const uint8_t* __restrict__ wq, const float2* __restrict__ wsm,
                        const int8_t* __restrict__ qx, const float* __restrict__ dx, const float* __restrict__ ds,
                        float* __restrict__ out, uint32_t rows, uint32_t m, uint32_t nb, uint32_t mt) {
    gemm_tiles<Q4_1, 2>(wq, wsm, qx, dx, ds, out, rows, m, nb, mt);
}

extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(ZLM_GEMM_WAVES_PER_EU)))
    zlm_gemm_q4_k_q8_k2(const uint8_t* __restrict__ wq, const float2* __restrict__ wsm,
                        const int8_t* __restrict__ qx, const float* __restrict__ dx, const float* __restrict__ ds,
                        float* __restrict__ out, uint32_t rows, uint32_t m, uint32_t nb, uint32_t mt) {
    gemm_tiles<Q4_K, 2>(wq, wsm, qx, dx, ds, out, rows, m, nb, mt);
}


// ---- small-M prefill GEMM (verify and microbatch batches, short prompts) -----
// The same int path and tiled operands as gemm_tiles, one 32-token tile per
// workgroup (grid.y: the token tiles).
// A 32-row tile is too little work for one wave over the whole row (the
// 128-token GEMM would leave most CUs idle and run a 4096-long K loop per
// wave), so the kGemmSmallWaves waves of a workgroup split the row's blocks:
// wave w takes block pairs (2w + 2*W*j, +1), the next pair's loads in flight
// while a pair computes (at these sizes the loop is bound by memory latency,
// so more waves -- shorter chains per wave -- pay).  Per pair: two int8 MFMAs (one per
// block) and one v_mfma_f32_32x32x1_2b_f32 for both blocks' scale matrices
// (lanes 0-31: the first block's dx by dw, lanes 32-63 the second's; each
// lane loads its own half's block scales).  The waves' partial sums meet in
// LDS and are added in wave order (deterministic), two output registers per
// wave.
// Waves per workgroup: 16 (128 VGPRs each at most) for q4_0 / q8_0, 8 for
// the min-carrying types (their min term holds 32 more accumulators).
template <int QT>
constexpr int gemm_small_waves() {
    return gemm_has_min(QT) ? 8 : 16;
}

template <int QT>
__device__ __forceinline__ void gemm_small(const uint8_t* __restrict__ wq, const void* __restrict__ wsc,
                                           const int8_t* __restrict__ qx, const float* __restrict__ dx,
                                           const float* __restrict__ ds, float* __restrict__ out, uint32_t rows,
                                           uint32_t m, uint32_t nb) {
    constexpr int W = gemm_small_waves<QT>();
    constexpr bool MIN = gemm_has_min(QT);
    __shared__ float red[W][MIN ? 32 : 16][kWave];
    const int lane = threadIdx.x & 63;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const uint32_t rt = blockIdx.x;  // the grid is exactly the row tiles x the token tiles
    const uint32_t tt = blockIdx.y;
    constexpr uint32_t kWStride = QT == Q8_0 ? 1024 : 512;
    constexpr uint32_t kScBytes = MIN ? 8 : 2;
    // token tile tt of the quantizer's layout: q bytes at tt * nb * 1024, scales at tt * nb * 32
    qx += static_cast<size_t>(tt) * nb * 1024;
    dx += static_cast<size_t>(tt) * nb * 32;
    if constexpr (MIN) ds += static_cast<size_t>(tt) * nb * 32;
    GemmPtrs ptr;
    ptr.a = gemm_rsrc(qx, nb * 1024);
    ptr.a1 = 0;
    ptr.oa = l32 * 32 + 16 * half;
    ptr.w = gemm_rsrc(wq + static_cast<size_t>(rt) * nb * kWStride, nb * kWStride);
    ptr.ow = QT == Q8_0 ? l32 * 32 + 16 * half : l32 * 16;
    ptr.sc = gemm_rsrc(static_cast<const uint8_t*>(wsc) + static_cast<size_t>(rt) * nb * 32 * kScBytes,
                       nb * 32 * kScBytes);
    ptr.osc = l32 * kScBytes;
    ptr.x = gemm_rsrc(dx, nb * 128);
    ptr.s = gemm_rsrc(MIN ? ds : dx, nb * 128);
    ptr.ox = l32 * 4;
    const int sh = half ? 0 : 4;
    const bool lo_half = half == 0;

    // a block pair's operands: both blocks' qx and weights, this lane's half's scales
    struct Pair {
        uint4 a0, a1, w0, w1;
        uint32_t d;
        float x, s;
        float2 sm;
    };
    auto load_pair = [&](Pair& p, uint32_t b) {
        const uint32_t b0 = min(b, nb - 1), b1 = min(b + 1, nb - 1), bh = half ? b1 : b0;
        p.a0 = gemm_ld16(ptr.a, ptr.oa, b0 * 1024);
        p.a1 = gemm_ld16(ptr.a, ptr.oa, b1 * 1024);
        p.w0 = gemm_ld16(ptr.w, ptr.ow, b0 * kWStride);
        p.w1 = gemm_ld16(ptr.w, ptr.ow, b1 * kWStride);
        if constexpr (MIN) {
            const uint32_t sx = __builtin_amdgcn_raw_buffer_load_b32(ptr.sc, static_cast<int>(ptr.osc),
                                                                     static_cast<int>(bh * 256), 0);
            const uint32_t sy = __builtin_amdgcn_raw_buffer_load_b32(ptr.sc, static_cast<int>(ptr.osc + 4),
                                                                     static_cast<int>(bh * 256), 0);
            p.sm = make_float2(__builtin_bit_cast(float, sx), __builtin_bit_cast(float, sy));
            p.s = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ptr.s, static_cast<int>(ptr.ox),
                                                                                 static_cast<int>(bh * 128), 0));
        } else {
            p.d = __builtin_amdgcn_raw_buffer_load_b16(ptr.sc, static_cast<int>(ptr.osc), static_cast<int>(bh * 64), 0);
        }
        p.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ptr.x, static_cast<int>(ptr.ox),
                                                                             static_cast<int>(bh * 128), 0));
    };
    v16f acc = {};
    v32f accm = {};
    auto compute_pair = [&](const Pair& p, uint32_t b) {
        const v4i bv0 = gemm_unpack<QT>(p.w0, lo_half, sh), bv1 = gemm_unpack<QT>(p.w1, lo_half, sh);
        const v4i a0 = {static_cast<int>(p.a0.x), static_cast<int>(p.a0.y), static_cast<int>(p.a0.z),
                        static_cast<int>(p.a0.w)};
        const v4i a1 = {static_cast<int>(p.a1.x), static_cast<int>(p.a1.y), static_cast<int>(p.a1.z),
                        static_cast<int>(p.a1.w)};
        const v16i zi = {};
        const v16i i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bv0, zi, 0, 0, 0);
        const v16i i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bv1, zi, 0, 0, 0);
        const bool valid = b + half < nb;  // this lane's half's block exists
        float bw;
        if constexpr (MIN) {
            bw = p.sm.x;
            accm = __builtin_amdgcn_mfma_f32_32x32x1f32(valid ? p.s : 0.0f, p.sm.y, accm, 0, 0, 0);
        } else {
            bw = h2f(p.d);
        }
        const v32f zf = {};
        const v32f c = __builtin_amdgcn_mfma_f32_32x32x1f32(valid ? p.x : 0.0f, bw, zf, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            acc[i] = fmaf(c[i], static_cast<float>(i0[i]), acc[i]);
            acc[i] = fmaf(c[16 + i], static_cast<float>(i1[i]), acc[i]);
        }
    };
    constexpr uint32_t kStep = 2 * W;  // blocks between a wave's consecutive pairs
    Pair A, B;
    uint32_t b = 2 * wid;
    load_pair(A, b);
    while (b < nb) {
        load_pair(B, b + kStep);
        __builtin_amdgcn_sched_barrier(0);
        compute_pair(A, b);
        __builtin_amdgcn_sched_barrier(0);
        b += kStep;
        if (b >= nb) break;
        load_pair(A, b + kStep);
        __builtin_amdgcn_sched_barrier(0);
        compute_pair(B, b);
        __builtin_amdgcn_sched_barrier(0);
        b += kStep;
    }
#pragma unroll
    for (int i = 0; i < 16; i++) red[wid][i][lane] = acc[i];
    if constexpr (MIN) {
#pragma unroll
        for (int i = 0; i < 16; i++) red[wid][16 + i][lane] = accm[i] + accm[16 + i];
    }
    __syncthreads();
    constexpr float kOut = QT == Q4_0 ? 0.0625f : 1.0f;
    const uint32_t r = rt * 32 + l32;
#pragma unroll
    for (int j = 0; j < 16 / W; j++) {
        const int i = static_cast<int>(wid) * (16 / W) + j;  // this wave's output register
        float v = 0.0f, vm = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            v += red[w][i][lane];
            if constexpr (MIN) vm += red[w][16 + i][lane];
        }
        const uint32_t t = tt * 32 + 8 * (i / 4) + 4 * half + (i % 4);
        if (r < rows && t < m) out[static_cast<size_t>(t) * rows + r] = v * kOut + vm;
    }
}

#define ZLM_GEMM_SMALL(NAME, QT, WT)                                                                          \
    extern "C" __global__ void __launch_bounds__(gemm_small_waves<QT>() * 64)                                 \
        NAME(const uint8_t* __restrict__ wq, const WT* __restrict__ ws, const int8_t* __restrict__ qx,      \
             const float* __restrict__ dx, const float* __restrict__ ds, float* __restrict__ out,           \
             uint32_t rows, uint32_t m, uint32_t nb) {                                                      \
        gemm_small<QT>(wq, ws, qx, dx, ds, out, rows, m, nb);                                              \
    }
ZLM_GEMM_SMALL(zlm_gemm_small_q4_0_q8, Q4_0, uint16_t)
ZLM_GEMM_SMALL(zlm_gemm_small_q8_0_q8, Q8_0, uint16_t)
ZLM_GEMM_SMALL(zlm_gemm_small_q4_1_q8, Q4_1, float2)
ZLM_GEMM_SMALL(zlm_gemm_small_q4_k_q8, Q4_K, float2)

// ---- decode-step glue -------------------------------------------------------
// The non-GEMV ops of one Qwen3 decode layer (reference
// architectures/impl/qwen3/block.zig:20-41), so activations stay in HBM
// between the GEMVs: per-head q/k RMSNorm + RoPE + the K/V cache append, and
// split-K attention over the fp16 cache.  KV cache layout (reference
// transformer/attention.zig:6-28): [n_kv_heads][max_seq][head_dim] f16.  The
// position is read from device memory (*pos), so a captured step can be
// replayed for another position without re-recording.

// Wave-wide sum / max, the same value in every lane, without LDS: DPP within
// each 16-lane row (quad_perm [1,0,3,2] and [2,3,0,1], then row_half_mirror
// and row_mirror, which pair a lane with one holding the other half's value
// once the smaller groups agree), then the four row results read from lanes
// 0, 16, 32, 48 and combined in that fixed order.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// qkv = [q: nh*hd | k: nkv*hd | v: nkv*hd] fp32 (the fused q/k/v GEMV's
// output).  One 64-lane workgroup per head: heads [0, nh) are q heads (out to
// q_out), [nh, nh+nkv) k heads (to the K cache at *pos), the rest v heads (to
// the V cache).  q and k: RMSNorm with the head weight (norm.zig:39-54,
// qkNormHeads :116-126), then the rotate-half RoPE (rope.zig:4-33 with the
// RopeTable frequencies :46-104: inv_freq_i = base^(-2i/hd), angle = pos *
// inv_freq_i; pair (i, i + hd/2) -> (x0 c - x1 s, x0 s + x1 c)).  Lane l owns
// pairs i = l and l + 64 (hd <= 256).  Every global load (position, head
// values, norm weights) is issued before the first use, so the kernel is one
// memory round trip.  A position at or past max_seq writes nothing.
extern "C" __global__ void __launch_bounds__(64)
    zlm_qk_norm_rope_kv(const float* __restrict__ qkv, float* __restrict__ q_out, const float* __restrict__ qn_w,
                        const float* __restrict__ kn_w, uint32_t nh, uint32_t nkv, uint32_t hd, float eps,
                        float freq_base, const int32_t* __restrict__ pos_p, _Float16* __restrict__ kc,
                        _Float16* __restrict__ vc, uint32_t max_seq) {
    const uint32_t head = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    const uint32_t half = hd / 2;
    const bool is_v = head >= nh + nkv;
    const bool is_q = head < nh;
    const float* src = qkv + static_cast<size_t>(head) * hd;  // q, k and v heads are consecutive
    const float* w = is_q ? qn_w : kn_w;
    const int32_t pos_i = *pos_p;
    float x0[2], x1[2], w0[2], w1[2];
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const uint32_t i = min(lane + kWave * p, half - 1);
        x0[p] = src[i];
        x1[p] = src[i + half];
        w0[p] = w[i];
        w1[p] = w[i + half];
    }
    const bool pos_ok = pos_i >= 0 && static_cast<uint32_t>(pos_i) < max_seq;
    const uint32_t pos = pos_ok ? static_cast<uint32_t>(pos_i) : 0u;
    if (is_v) {  // the cache append only
        _Float16* dst = vc + (static_cast<size_t>(head - nh - nkv) * max_seq + pos) * hd;
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const uint32_t i = lane + kWave * p;
            if (pos_ok && i < half) {
                dst[i] = static_cast<_Float16>(x0[p]);
                dst[i + half] = static_cast<_Float16>(x1[p]);
            }
        }
        return;
    }
    float ss = 0.0f;
#pragma unroll
    for (int p = 0; p < 2; p++) {
        if (lane + kWave * p < half) {
            ss = fmaf(x0[p], x0[p], ss);
            ss = fmaf(x1[p], x1[p], ss);
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(hd) + eps);
    const float t = static_cast<float>(pos_i);
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const uint32_t i = lane + kWave * p;
        if (i >= half) continue;
        const float a = x0[p] * inv * w0[p];
        const float b = x1[p] * inv * w1[p];
        const float angle = t * powf(freq_base, -2.0f * static_cast<float>(i) / static_cast<float>(hd));
        const float c = cosf(angle), s = sinf(angle);
        const float r0 = fmaf(b, -s, a * c);
        const float r1 = fmaf(b, c, a * s);
        if (is_q) {
            q_out[static_cast<size_t>(head) * hd + i] = r0;
            q_out[static_cast<size_t>(head) * hd + i + half] = r1;
        } else if (pos_ok) {
            _Float16* dst = kc + (static_cast<size_t>(head - nh) * max_seq + pos) * hd;
            dst[i] = static_cast<_Float16>(r0);
            dst[i + half] = static_cast<_Float16>(r1);
        }
    }
}

// Split-K decode attention, head_dim 128 (reference attention.zig:86-170, the
// per-q-head online softmax, here split over position ranges and merged by
// zlm_attn_combine).  Grid (nkv, nsplit), 256 threads.  Workgroup (h, s)
// handles the G = nh/nkv q heads of kv head h (G <= 4) over positions
// [64 s, 64 s + 64) clipped to L = min(*pos + 1, max_seq):
//   loads:   thread t loads 64 bytes of K and of V: position t/4, dims
//            32*(t%4)..+31.  The row addresses do not depend on *pos (rows
//            are clamped to the cache, positions past L masked afterwards), so
//            the K/V loads go out together with the position's own load and a
//            split costs one memory round trip;
//   scores:  thread t takes its K slice for all G heads (4 lanes reduce a dot
//            with two shuffles), score = (q.k) * scale;
//   values:  the V slices go to LDS transposed (dword column c = dims 2c, 2c+1
//            holds the 64 positions contiguously; zeros past L), wave g (< G)
//            takes head g's 64 scores: m = max, p = exp(s - m), l = sum p, and
//            lane l accumulates sum_t p_t V[t][2l..2l+1], reading its column
//            four positions per 128-bit LDS read and each weight with a
//            readlane.
// Output part[(qh*nsplit + s)*130 + d] = unnormalised acc (d < 128), then m, l.
constexpr int kAttnHd = 128;
constexpr int kAttnSplit = 64;
constexpr int kAttnPart = kAttnHd + 2;

// V tile row stride in dwords: 64 positions + 4, so the 16 lanes of one
// 128-bit LDS read pass (columns l..l+15, same positions) cover all 64 banks.
constexpr int kAttnVStride = kAttnSplit + 4;

struct alignas(16) AttnLds {
    float qs[4][kAttnHd];                          // scaled q of the G heads (zeros past G)
    float sc[4][kAttnSplit];                       // scores
    uint32_t vt[kAttnHd / 2][kAttnVStride];        // V transposed: [dim pair][position] f16 pairs
};

// Position-independent K and V loads of thread (p, qd) of split t0.
__device__ __forceinline__ void attn_load_kv(const _Float16* __restrict__ kc, const _Float16* __restrict__ vc,
                                             uint32_t h, uint32_t max_seq, uint32_t t0, uint32_t p, uint32_t qd,
                                             uint4 (&kraw)[4], uint4 (&vraw)[4]) {
    const size_t row = static_cast<size_t>(h) * max_seq + min(t0 + p, max_seq - 1);
    const _Float16* kr = kc + row * kAttnHd + 32 * qd;
    const _Float16* vr = vc + row * kAttnHd + 32 * qd;
#pragma unroll
    for (int c = 0; c < 4; c++) kraw[c] = *reinterpret_cast<const uint4*>(kr + 8 * c);
#pragma unroll
    for (int c = 0; c < 4; c++) vraw[c] = *reinterpret_cast<const uint4*>(vr + 8 * c);
}

// Thread (p, qd)'s V slice (dword columns 16 qd..+15) into the transposed
// LDS tile: zeros for a position past L (its weight is 0, and 0 * a stale NaN
// would not be), nothing for the row `skip` (the caller writes that row).
__device__ __forceinline__ void attn_stage_v(const uint4 (&vraw)[4], uint32_t p, uint32_t qd, bool valid,
                                             uint32_t skip, AttnLds& sm) {
    if (p == skip) return;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t w[4] = {vraw[c].x, vraw[c].y, vraw[c].z, vraw[c].w};
#pragma unroll
        for (int i = 0; i < 4; i++) sm.vt[16 * qd + 4 * c + i][p] = valid ? w[i] : 0u;
    }
}

// Scores of thread (p, qd)'s position for all 4 head slots into sm.sc; with
// NEWROW the position `prow` takes its K values from kn (fp32 of the f16 row
// just appended) instead of the loaded slice.
template <bool NEWROW>
__device__ __forceinline__ void attn_scores(const uint4 (&kraw)[4], uint32_t p, uint32_t qd, bool valid,
                                            uint32_t prow, const float* kn, AttnLds& sm) {
    float kf[32];  // dims 32 qd .. +31 of position p
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t wv[4] = {kraw[c].x, kraw[c].y, kraw[c].z, kraw[c].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            kf[8 * c + 2 * j] = h2f(wv[j]);
            kf[8 * c + 2 * j + 1] = h2f(wv[j] >> 16);
        }
    }
    if constexpr (NEWROW) {
        if (p == prow) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 t = lds4(kn + 32 * qd + 4 * i);
                kf[4 * i] = t.x;
                kf[4 * i + 1] = t.y;
                kf[4 * i + 2] = t.z;
                kf[4 * i + 3] = t.w;
            }
        }
    }
    float dot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 qv = lds4(&sm.qs[g][32 * qd + 4 * i]);
            dot[g] = fmaf(qv.x, kf[4 * i], dot[g]);
            dot[g] = fmaf(qv.y, kf[4 * i + 1], dot[g]);
            dot[g] = fmaf(qv.z, kf[4 * i + 2], dot[g]);
            dot[g] = fmaf(qv.w, kf[4 * i + 3], dot[g]);
        }
    }
#pragma unroll
    for (int g = 0; g < 4; g++) {
        dot[g] += __shfl_xor(dot[g], 1, kWave);
        dot[g] += __shfl_xor(dot[g], 2, kWave);
    }
    if (qd == 0) {
#pragma unroll
        for (int g = 0; g < 4; g++) sm.sc[g][p] = valid ? dot[g] : -INFINITY;
    }
}

// Wave g's softmax over its head's 64 scores and the weighted V sum from LDS;
// writes the split's partial (acc[128], m, l).  `poison` makes l NaN, so the
// merged head is NaN (a position past the launched splits: see zlm_attn_decode).
__device__ __forceinline__ void attn_values(const AttnLds& sm, uint32_t g, uint32_t lane, float* __restrict__ out,
                                            bool poison = false) {
    const float sv = sm.sc[g][lane];
    const float m = wave_max(sv);
    const float e = (sv == -INFINITY) ? 0.0f : expf(sv - m);
    const float l = wave_sum(e);
    const int eb = __builtin_bit_cast(int, e);
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int j4 = 0; j4 < kAttnSplit; j4 += 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(&sm.vt[lane][j4]);
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // position j's weight, held by lane j (0 past n)
            const float pe = __builtin_bit_cast(float, __builtin_amdgcn_readlane(eb, j4 + i));
            a0 = fmaf(pe, h2f(vw[i]), a0);
            a1 = fmaf(pe, h2f(vw[i] >> 16), a1);
        }
    }
    *reinterpret_cast<float2*>(out + 2 * lane) = make_float2(a0, a1);
    if (lane == 0) {
        out[kAttnHd] = m;
        out[kAttnHd + 1] = poison ? __builtin_nanf("") : l;
    }
}

extern "C" __global__ void __launch_bounds__(256)
    zlm_attn_partial(const float* __restrict__ q, const _Float16* __restrict__ kc, const _Float16* __restrict__ vc,
                     uint32_t nh, uint32_t nkv, const int32_t* __restrict__ pos_p, uint32_t max_seq, float scale,
                     float* __restrict__ part, uint32_t nsplit) {
    __shared__ AttnLds sm;
    const uint32_t h = blockIdx.x, s = blockIdx.y;
    const uint32_t G = nh / nkv;
    const uint32_t tid = threadIdx.x, wid = tid / kWave, lane = tid & (kWave - 1);
    const uint32_t t0 = s * kAttnSplit;
    const uint32_t p = tid / 4, qd = tid % 4;
    // q (scaled) for the G heads into LDS; thread tid holds 2 of the 4*128 values
    float qv[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t i = tid + 256u * j, g = i / kAttnHd, d = i % kAttnHd;
        qv[j] = q[static_cast<size_t>(h * G + min(g, G - 1)) * kAttnHd + d];
    }
    uint4 kraw[4], vraw[4];
    attn_load_kv(kc, vc, h, max_seq, t0, p, qd, kraw, vraw);
    const int32_t pos_i = *pos_p;
    const uint32_t L = pos_i < 0 ? 0u : min(static_cast<uint32_t>(pos_i) + 1u, max_seq);
    const uint32_t n = t0 < L ? min(static_cast<uint32_t>(kAttnSplit), L - t0) : 0u;
    const bool valid = p < n;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t i = tid + 256u * j, g = i / kAttnHd;
        sm.qs[g][i % kAttnHd] = g < G ? qv[j] * scale : 0.0f;
    }
    attn_stage_v(vraw, p, qd, valid, kAttnSplit, sm);
    __syncthreads();
    attn_scores<false>(kraw, p, qd, valid, kAttnSplit, nullptr, sm);
    __syncthreads();
    if (wid < G) attn_values(sm, wid, lane, part + (static_cast<size_t>(h * G + wid) * nsplit + s) * kAttnPart);
}

// Merge the nsplit partials of each q head: M = max m_s, w_s = exp(m_s - M)
// (0 for an empty split), out = sum w_s acc_s / sum w_s l_s.  One 256-thread
// workgroup per q head, in passes of 64 splits: lane s of every wave holds
// split s's (m, l) and w_s; wave g accumulates the pass's splits g, g+4, ...
// into lane l's dims 2l, 2l+1 (16 splits, every load issued before the first
// use, so a pass is one memory round trip), and the four waves' sums merge in
// LDS.
extern "C" __global__ void __launch_bounds__(256)
    zlm_attn_combine(const float* __restrict__ part, uint32_t nsplit, float* __restrict__ out) {
    __shared__ float2 red[4][kWave];
    const uint32_t qh = blockIdx.x, tid = threadIdx.x, wid = tid / kWave, lane = tid & (kWave - 1);
    const float* base = part + static_cast<size_t>(qh) * nsplit * kAttnPart;
    float M = -INFINITY;
    if (nsplit > kWave) {
        for (uint32_t s0 = 0; s0 < nsplit; s0 += kWave) {
            const uint32_t s = s0 + lane;
            M = fmaxf(M, wave_max(s < nsplit ? base[static_cast<size_t>(s) * kAttnPart + kAttnHd] : -INFINITY));
        }
    }
    float a0 = 0.0f, a1 = 0.0f, den = 0.0f;
    for (uint32_t s0 = 0; s0 < nsplit; s0 += kWave) {
        const uint32_t cnt = min(static_cast<uint32_t>(kWave), nsplit - s0);
        const bool sv = lane < cnt;
        const size_t sl = s0 + (sv ? lane : 0u);
        const float ms_raw = base[sl * kAttnPart + kAttnHd];
        const float ls_raw = base[sl * kAttnPart + kAttnHd + 1];
        float2 acc[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t sj = s0 + min(wid + 4u * j, cnt - 1);
            acc[j] = *reinterpret_cast<const float2*>(base + static_cast<size_t>(sj) * kAttnPart + 2 * lane);
        }
        const float ms = sv ? ms_raw : -INFINITY;
        if (nsplit <= kWave) M = wave_max(ms);
        const float w = (ms == -INFINITY) ? 0.0f : expf(ms - M);
        den += wave_sum(sv ? w * ls_raw : 0.0f);
        const int wb = __builtin_bit_cast(int, w);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t idx = wid + 4u * j;  // 0 weight past cnt
            const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(wb, idx));
            a0 = fmaf(wj, acc[j].x, a0);
            a1 = fmaf(wj, acc[j].y, a1);
        }
    }
    red[wid][lane] = make_float2(a0, a1);
    __syncthreads();
    if (wid == 0) {
        float2 t = red[0][lane];
#pragma unroll
        for (int g = 1; g < 4; g++) {
            t.x += red[g][lane].x;
            t.y += red[g][lane].y;
        }
        const float inv = 1.0f / den;
        *reinterpret_cast<float2*>(out + static_cast<size_t>(qh) * kAttnHd + 2 * lane) = make_float2(t.x * inv, t.y * inv);
    }
}

// The merge for many splits (long caches: nsplit > 64, i.e. more than 4096
// positions).  Two workgroups per q head (grid.y picks dims [64y, 64y+64),
// lane l dim 64y + l), each of nw = min(16, ceil(nsplit / 32)) waves; wave w
// takes splits [w*S, (w+1)*S), S = ceil(nsplit / nw), in chunks of 32 whose
// loads are all issued before their first use (lane j holds split j's m and
// l; every lane the chunk's 32 accumulator values of its dim), keeping a
// running maximum and rescaling its sums when a chunk raises it; the waves'
// (M, den, acc) then merge in LDS, in wave order.  One memory round trip per
// chunk instead of one per 64 splits in sequence, and each workgroup reads
// half of a head's partials.
extern "C" __global__ void __launch_bounds__(1024)
    zlm_attn_combine_wide(const float* __restrict__ part, uint32_t nsplit, float* __restrict__ out) {
    constexpr uint32_t W = 16, B = 32;
    __shared__ float rm[W], rd[W], ra[W][kWave];
    const uint32_t qh = blockIdx.x, tid = threadIdx.x, wid = tid / kWave, lane = tid & (kWave - 1);
    const uint32_t dim = kWave * blockIdx.y + lane;
    const uint32_t nw = blockDim.x / kWave;  // <= W
    const float* base = part + static_cast<size_t>(qh) * nsplit * kAttnPart;
    const uint32_t S = (nsplit + nw - 1) / nw;
    const uint32_t s_begin = min(wid * S, nsplit), s_end = min(s_begin + S, nsplit);
    float M = -INFINITY, den = 0.0f, acc_d = 0.0f;
    for (uint32_t s0 = s_begin; s0 < s_end; s0 += B) {
        const uint32_t n = min(B, s_end - s0);
        const uint32_t sl = s0 + min(lane, n - 1);
        const float ms_raw = base[static_cast<size_t>(sl) * kAttnPart + kAttnHd];
        const float ls_raw = base[static_cast<size_t>(sl) * kAttnPart + kAttnHd + 1];
        float acc[B];
#pragma unroll
        for (uint32_t j = 0; j < B; j++) acc[j] = base[static_cast<size_t>(s0 + min(j, n - 1)) * kAttnPart + dim];
        const float ms = lane < n ? ms_raw : -INFINITY;
        const float Mn = fmaxf(M, wave_max(ms));
        const float r = (M == -INFINITY) ? 0.0f : expf(M - Mn);
        const float w = (ms == -INFINITY) ? 0.0f : expf(ms - Mn);
        den = fmaf(den, r, wave_sum(lane < n ? w * ls_raw : 0.0f));
        acc_d *= r;
        const int wb = __builtin_bit_cast(int, w);
#pragma unroll
        for (uint32_t j = 0; j < B; j++)
            acc_d = fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(wb, j)), acc[j], acc_d);  // 0 past n
        M = Mn;
    }
    if (lane == 0) {
        rm[wid] = M;
        rd[wid] = den;
    }
    ra[wid][lane] = acc_d;
    __syncthreads();
    if (wid == 0) {
        float Mt = -INFINITY;
        for (uint32_t g = 0; g < nw; g++) Mt = fmaxf(Mt, rm[g]);
        float d = 0.0f, t = 0.0f;
        for (uint32_t g = 0; g < nw; g++) {
            const float e = (rm[g] == -INFINITY) ? 0.0f : expf(rm[g] - Mt);
            d = fmaf(e, rd[g], d);
            t = fmaf(e, ra[g][lane], t);
        }
        out[static_cast<size_t>(qh) * kAttnHd + dim] = t / d;
    }
}

// The decode layer's whole attention block in one launch (reference
// block.zig:24-31: q_norm/k_norm, rope, write_kv, attention), head_dim 128,
// G = nh/nkv <= 4.  Grid (nkv, nsplit), 256 threads; workgroup (h, s) owns kv
// head h's G q heads over positions [64 s, 64 s + 64) of L = *pos + 1:
//   * every global load it needs (its K and V slices, the raw q / k / v head
//     values, the norm weights, the position) is issued first, none waiting
//     on another;
//   * the cos/sin of the 64 rotary pairs at *pos go to LDS once;
//   * wave g normalises and rotates q head g (the same arithmetic as
//     zlm_qk_norm_rope_kv); the workgroup whose range holds *pos also
//     normalises and rotates k head h, appends the f16 K and V rows to the
//     caches and uses those same f16 values for position *pos (no read back:
//     the V row goes straight into the LDS V tile, the K row replaces the
//     loaded slice in the scores);
//   * scores, softmax and values as zlm_attn_partial, into the same partials,
//     which zlm_attn_combine merges.
// nsplit may cover fewer positions than the cache holds (a window: the host
// launches ceil(window / 64) splits for steps whose position is below it).  A
// position past the launched splits would leave positions out, so the first
// split then writes a NaN denominator and the heads come out NaN instead of
// silently wrong.  (Merging in the last workgroup of each kv
//     head instead, behind a device-scope fence and counter, measured 3x
//     slower on gfx950: every workgroup's release fence writes back its L2.)
extern "C" __global__ void __launch_bounds__(256)
    zlm_attn_decode(const float* __restrict__ qkv, const float* __restrict__ qn_w, const float* __restrict__ kn_w,
                    uint32_t nh, uint32_t nkv, float eps, float freq_base, const int32_t* __restrict__ pos_p,
                    _Float16* __restrict__ kc, _Float16* __restrict__ vc, uint32_t max_seq, float scale,
                    float* __restrict__ part, uint32_t nsplit) {
    __shared__ AttnLds sm;
    __shared__ float cs[kAttnHd / 2], sn[kAttnHd / 2];
    __shared__ __attribute__((aligned(16))) float kn[kAttnHd];
    const uint32_t h = blockIdx.x, s = blockIdx.y;
    const uint32_t G = nh / nkv;
    const uint32_t tid = threadIdx.x, wid = tid / kWave, lane = tid & (kWave - 1);
    constexpr uint32_t half = kAttnHd / 2;
    const uint32_t t0 = s * kAttnSplit;
    const uint32_t p = tid / 4, qd = tid % 4;

    // loads: the position, this wave's q head (raw) and norm weights, k/v of
    // the new row, the split's K and V slices
    const int32_t pos_i = *pos_p;
    const uint32_t g = min(wid, G - 1);
    const float* qh = qkv + static_cast<size_t>(h * G + g) * kAttnHd;
    const float q0 = qh[lane], q1 = qh[lane + half];
    const float wq0 = qn_w[lane], wq1 = qn_w[lane + half];
    const float* kh = qkv + static_cast<size_t>(nh + h) * kAttnHd;
    const float* vh = qkv + static_cast<size_t>(nh + nkv + h) * kAttnHd;
    const float k0 = kh[lane], k1 = kh[lane + half], wk0 = kn_w[lane], wk1 = kn_w[lane + half];
    const float v0 = vh[lane], v1 = vh[lane + half];
    uint4 kraw[4], vraw[4];
    attn_load_kv(kc, vc, h, max_seq, t0, p, qd, kraw, vraw);

    const bool pos_ok = pos_i >= 0 && static_cast<uint32_t>(pos_i) < max_seq;
    const uint32_t L = pos_i < 0 ? 0u : min(static_cast<uint32_t>(pos_i) + 1u, max_seq);
    const uint32_t n = t0 < L ? min(static_cast<uint32_t>(kAttnSplit), L - t0) : 0u;
    const bool own = pos_ok && static_cast<uint32_t>(pos_i) >= t0 && static_cast<uint32_t>(pos_i) < t0 + kAttnSplit;
    const uint32_t prow = own ? static_cast<uint32_t>(pos_i) - t0 : kAttnSplit;  // the new row's slot, or none
    const bool valid = p < n;
    if (tid < half) {
        const float angle = static_cast<float>(pos_i) *
                            powf(freq_base, -2.0f * static_cast<float>(tid) / static_cast<float>(kAttnHd));
        cs[tid] = cosf(angle);
        sn[tid] = sinf(angle);
    }
    attn_stage_v(vraw, p, qd, valid, prow, sm);
    if (own && wid == 1) {  // the new V row, as the f16 values the cache holds
        const _Float16 e0 = static_cast<_Float16>(v0), e1 = static_cast<_Float16>(v1);
        _Float16* vd = vc + (static_cast<size_t>(h) * max_seq + pos_i) * kAttnHd;
        vd[lane] = e0;
        vd[lane + half] = e1;
        // dim d sits in half d%2 of dword column d/2 at position prow
        reinterpret_cast<_Float16*>(&sm.vt[lane / 2][prow])[lane % 2] = e0;
        reinterpret_cast<_Float16*>(&sm.vt[(lane + half) / 2][prow])[lane % 2] = e1;
    }
    __syncthreads();
    // q head g: RMSNorm, rotate, scale (lane l owns the pair (l, l + 64))
    if (wid < G) {
        const float inv = 1.0f / sqrtf(wave_sum(fmaf(q0, q0, q1 * q1)) / static_cast<float>(kAttnHd) + eps);
        const float a = q0 * inv * wq0, b = q1 * inv * wq1;
        sm.qs[wid][lane] = fmaf(b, -sn[lane], a * cs[lane]) * scale;
        sm.qs[wid][lane + half] = fmaf(b, cs[lane], a * sn[lane]) * scale;
    } else {
        sm.qs[wid][lane] = 0.0f;
        sm.qs[wid][lane + half] = 0.0f;
    }
    // the new position's K row: kept as the f16 values the cache holds
    if (own && wid == 0) {
        const float inv = 1.0f / sqrtf(wave_sum(fmaf(k0, k0, k1 * k1)) / static_cast<float>(kAttnHd) + eps);
        const float a = k0 * inv * wk0, b = k1 * inv * wk1;
        const _Float16 r0 = static_cast<_Float16>(fmaf(b, -sn[lane], a * cs[lane]));
        const _Float16 r1 = static_cast<_Float16>(fmaf(b, cs[lane], a * sn[lane]));
        _Float16* kd = kc + (static_cast<size_t>(h) * max_seq + pos_i) * kAttnHd;
        kd[lane] = r0;
        kd[lane + half] = r1;
        kn[lane] = static_cast<float>(r0);
        kn[lane + half] = static_cast<float>(r1);
    }
    __syncthreads();
    attn_scores<true>(kraw, p, qd, valid, prow, kn, sm);
    __syncthreads();
    const bool past_window = L > nsplit * kAttnSplit;
    if (wid < G)
        attn_values(sm, wid, lane, part + (static_cast<size_t>(h * G + wid) * nsplit + s) * kAttnPart,
                    past_window && s == 0);
}

// ---- synthetic data on the device (benchmark and large-shape tests) ---------
// splitmix64 of (seed, index): the same counter-based generator as the
// repository's Python synthesiser, used here to fill raw GGUF blocks in HBM so
// multi-GB synthetic models need no host generation or upload.
__device__ __forceinline__ uint64_t smix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// |N(0,1)| from two uniforms (Box-Muller).
__device__ __forceinline__ float abs_normal(uint64_t r) {
    const float u1 = (static_cast<float>(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = static_cast<float>((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
    return fabsf(sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2));
}

// One thread per raw block of type `type` (2 = q4_0: f16 d + 16 random bytes;
// 8 = q8_0: f16 d + 32 int8 uniform in [-127, 127]); d = f16(|N(0,1)| * scale).
extern "C" __global__ void __launch_bounds__(256)
    zlm_synth_blocks(uint8_t* __restrict__ raw, uint32_t type, uint64_t nblocks, uint64_t seed, float scale) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint32_t bb = type == 8u ? 34u : 18u;
    uint8_t* dst = raw + b * bb;
    const uint64_t base = smix(seed ^ (b * 0xD1B54A32D192ED03ull));
    const _Float16 d = static_cast<_Float16>(abs_normal(smix(base)) * scale);
    const uint16_t db = __builtin_bit_cast(uint16_t, d);
    dst[0] = static_cast<uint8_t>(db & 0xffu);
    dst[1] = static_cast<uint8_t>(db >> 8);
    const uint32_t nq = bb - 2;
    for (uint32_t i = 0; i < nq; i += 8) {
        const uint64_t r = smix(base + 1 + i);
        for (uint32_t j = 0; j < 8 && i + j < nq; j++) {
            const uint32_t byte = static_cast<uint32_t>(r >> (8 * j)) & 0xffu;
            dst[2 + i + j] = type == 8u ? static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(byte % 255u) - 127))
                                        : static_cast<uint8_t>(byte);
        }
    }
}

// n f16 values N(0,1) * scale (signed), e.g. a KV cache's history.
extern "C" __global__ void __launch_bounds__(256)
    zlm_synth_f16(_Float16* __restrict__ out, uint64_t n, uint64_t seed, float scale) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t r = smix(seed ^ (i * 0xD1B54A32D192ED03ull));
    const float v = abs_normal(r) * scale;
    out[i] = static_cast<_Float16>((r & 1u) ? -v : v);
}
