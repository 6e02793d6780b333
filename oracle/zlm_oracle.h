/*
 * zlm_oracle.h -- CPU restatement of zlm's quantized GEMV/GEMM kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * backend and the CPU baseline timer of bench.py.  Only tests/, the smoke()
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it.
 * The product path (zlm_amd/, libzlm_gpu_hip.so) never links or calls it.
 *
 * Every function restates a routine of the Zig reference (paths relative to
 * the reference tree); the citation is on each definition in zlm_oracle.c.
 * Type codes are GGML type codes (gguf/format.zig:41-77).
 */
#ifndef ZLM_ORACLE_H
#define ZLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_F32 = 0,
    ORC_F16 = 1,
    ORC_Q4_0 = 2,
    ORC_Q4_1 = 3,
    ORC_Q8_0 = 8,
    ORC_Q4_K = 12,
    ORC_Q6_K = 14,
    ORC_BF16 = 30,
};

/* Error codes mirroring the reference's KernelError set (kernels/api.zig). */
enum {
    ORC_OK = 0,
    ORC_E_TRUNCATED = -1,     /* error.TruncatedData   */
    ORC_E_SHAPE = -2,         /* error.ShapeMismatch   */
    ORC_E_RANGE = -3,         /* error.InvalidRange    */
    ORC_E_UNSUPPORTED = -4,   /* error.UnsupportedType */
};

enum { ORC_ACT_SILU = 0, ORC_ACT_GELU = 1 };

float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

size_t orc_block_elems(uint32_t type);
size_t orc_block_bytes(uint32_t type);
int64_t orc_tensor_byte_length(uint32_t type, uint64_t n_elements);

void orc_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *d, uint8_t *m);

int orc_dequant(uint32_t type, const uint8_t *data, size_t data_len, float *out, size_t n);

int orc_matvec(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
               const float *x, float *out, size_t begin, size_t end, int lanes);
int orc_lm_head_rows(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                     const float *x, float *out, size_t begin, size_t end, int lanes);

void orc_quantize_act_q8(const float *x, size_t blocks, int8_t *qx, float *dx, int32_t *sums);
int orc_matvec_int(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                   const float *x, float *out, size_t begin, size_t end, int lanes);

int orc_matmul_rows(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                    size_t m, const float *x, float *out, size_t begin, size_t end, int lanes);
int orc_matmul_int(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                   size_t m, const float *x, float *out, size_t begin, size_t end, int lanes);

float orc_act_apply(int act, float gate, float up);
int orc_gate_up(uint32_t type, const uint8_t *wg, const uint8_t *wu, size_t w_len, size_t k,
                size_t rows, const float *x, int act, float *out, size_t begin, size_t end,
                int lanes);

void orc_range_of(size_t total, size_t parts, size_t idx, size_t *begin, size_t *end);

/* Threaded timing of the production sweep (min over `reps` of wall seconds). */
double orc_time_matvec(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                       const float *x, float *out, int threads, int reps, int lanes);
double orc_time_matmul_int(uint32_t type, const uint8_t *w, size_t w_len, size_t k,
                           size_t rows, size_t m, const float *x, float *out, int threads,
                           int reps, int lanes);

/* ---- the speed-faithful sweep (zlm_cpu_sweep.c, zlm_cpu_pool.c) ----------
 * Bit-identical to orc_matvec / orc_matvec_int at the same lanes, written as
 * zlm's ReleaseFast build runs it; lanes 8 (AVX2) or 16 (AVX-512), 0 = the
 * width zlm's simd.native picks on this host.  ORC_E_UNSUPPORTED when the
 * host lacks the width. */
int orc_fast_native_lanes(void);
int orc_fast_matvec(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                    const float *x, float *out, size_t begin, size_t end, int lanes);
int orc_fast_matvec_int(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                        const float *x, float *out, size_t begin, size_t end, int lanes);
/* One logical CPU per physical core of the process's affinity mask. */
int orc_physical_cores(int *cpus, int max);
/* The persistent pool (runtime/pool.zig): workers pinned one per physical
 * core, the caller running part 0. */
int orc_pool_start(int threads);
void orc_pool_stop(void);
int orc_pool_threads(void);
double orc_fast_time_matvec(uint32_t type, const uint8_t *w, size_t w_len, size_t k, size_t rows,
                            const float *x, float *out, int threads, int reps, int lanes);
/* The same, call r reading weight copy r % n_copies (copies past the last
 * level cache keep the weights streaming from DRAM). */
double orc_fast_time_matvec_copies(uint32_t type, const uint8_t *const *ws, int n_copies, size_t w_len,
                                   size_t k, size_t rows, const float *x, float *out, int threads, int reps,
                                   int lanes);
double orc_fast_time_matmul_int(uint32_t type, const uint8_t *w, size_t w_len, size_t k,
                                size_t rows, size_t m, const float *x, float *out, int threads,
                                int reps, int lanes);

#ifdef __cplusplus
}
#endif
#endif
