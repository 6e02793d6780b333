/*
 * zlm_gpu_hip.h -- C ABI of the MI355X (gfx950) HIP co-processor backend for
 * zlm's quantized GEMV/GEMM path.
 *
 * The first block of entry points is the reference's GPU backend contract,
 * one function per name in `required_ops` (reference
 * src/gpu/backend/root.zig:299-311), with the semantics of the Vulkan device
 * it replaces (src/gpu/backend/vulkan/root.zig:22-236):
 *   - zlm_gpu_init never fails: without a usable GPU it returns a valid, inert
 *     device whose zlm_gpu_available() is false;
 *   - nothing is thrown: `false`, ZLM_NULL_HANDLE or NULL means "did not run
 *     on the device, the caller uses the CPU kernel" (unsupported quant or
 *     shape, short buffers, allocation or driver failure);
 *   - results land in host memory: every synchronous op, and
 *     zlm_gpu_wait_resident for the asynchronous ones, copies `rows` floats
 *     into `out`;
 *   - single-threaded: one thread drives a device (the executor's).
 *
 * Quant codes: the GGML type code (reference gguf/format.zig:41-77) in bits
 * 0..7 and the GpuVariant code (reference gpu/kernels/grid.zig:14) in bits
 * 8..15.  A variant never changes the byte layout, only the kernel.
 *
 * Device kernels: GEMVs (every form) for q4_0, q4_1, q8_0, q4_k, q6_k, f32,
 * f16 and bf16 (the float types need k % 32 == 0), prefill GEMMs for q4_0,
 * q8_0, q4_1 and q4_k; any other quant or shape returns false.
 *
 * Weight bytes are always the raw GGUF blocks (row-major, `rows` rows of
 * `k / block_elems` blocks).  The device keeps its own layout in HBM.
 */
#ifndef ZLM_GPU_HIP_H
#define ZLM_GPU_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* In-flight resident dispatches (reference gpu/backend/root.zig:230 RingSize). */
#define ZLM_RING_SIZE 8
/* The null async handle (the Zig `?Handle` null). */
#define ZLM_NULL_HANDLE (-1)

/* GGML type codes (reference gguf/format.zig:41-77). */
enum {
    ZLM_GGML_F32 = 0,
    ZLM_GGML_F16 = 1,
    ZLM_GGML_Q4_0 = 2,
    ZLM_GGML_Q4_1 = 3,
    ZLM_GGML_Q8_0 = 8,
    ZLM_GGML_Q4_K = 12,
    ZLM_GGML_Q6_K = 14,
    ZLM_GGML_BF16 = 30
};

/* GpuVariant codes (reference gpu/kernels/grid.zig:14). */
enum {
    ZLM_VARIANT_PLAIN = 0,
    ZLM_VARIANT_U4 = 1,
    ZLM_VARIANT_U8 = 2,
    ZLM_VARIANT_SUB = 3,
    ZLM_VARIANT_UN2 = 4,
    ZLM_VARIANT_UN4 = 5,
    ZLM_VARIANT_W32 = 6,
    ZLM_VARIANT_W128 = 7
};

/* GateUpAct (reference gpu/backend/root.zig:225). */
enum { ZLM_ACT_SILU = 0, ZLM_ACT_GELU = 1 };

#define ZLM_QUANT(ggml_type, variant) ((uint32_t)(ggml_type) | ((uint32_t)(variant) << 8))

typedef struct zlm_device zlm_device;
typedef struct zlm_resident zlm_resident;

/* ResidentOp (reference gpu/backend/root.zig:249-254): `out` holds >= rows floats. */
typedef struct {
    zlm_resident *res;
    uint32_t quant;
    size_t rows;
    float *out;
    size_t out_len;
} zlm_resident_op;

/* Probe (reference gpu/backend/root.zig:260-295).  GB/s over raw weight bytes;
 * unmeasured fields stay 0; variants are GpuVariant codes. */
typedef struct {
    double gemv_gbps;
    double gemv_streamed_gbps;
    double matmul_gbps;
    uint8_t q4_0_variant;
    uint8_t q4_1_variant;
    uint8_t q8_0_variant;
    uint8_t q6_k_variant;
    uint8_t q4_k_variant;
    uint8_t f32_variant;
    uint8_t f16_variant;
    uint8_t bf16_variant;
    uint8_t gate_up_variant;
    uint8_t gate_up_q4_1_variant;
    uint8_t gate_up_q8_0_variant;
    double q4_0_u4_gbps;
    double q4_0_sub_gbps;
    double q4_0_un2_gbps;
    double q4_0_un4_gbps;
    double q4_0_w32_gbps;
    double q4_0_w128_gbps;
    double q4_k_gbps;
    double q4_k_u4_gbps;
    double gate_up_gbps;
    double gate_up_u4_gbps;
} zlm_probe;

/* ---- the backend contract (reference gpu/backend/root.zig:299-311) ---- */

/* Device.init (vulkan/root.zig:28-42): never NULL unless the host is out of memory. */
zlm_device *zlm_gpu_init(void);
/* Device.deinit (vulkan/root.zig:44-55); also frees the handle. */
void zlm_gpu_deinit(zlm_device *dev);
/* Device.available (vulkan/root.zig:57-59). */
bool zlm_gpu_available(const zlm_device *dev);
/* Device.backendName (vulkan/root.zig:61-66): "hip", or "off" when inert. */
const char *zlm_gpu_backend_name(const zlm_device *dev);
/* Device.deviceName (vulkan/root.zig:68-71). */
const char *zlm_gpu_device_name(const zlm_device *dev);
/* Device.isUma (vulkan/root.zig:73-76). */
bool zlm_gpu_is_uma(const zlm_device *dev);

/* Device.matVec (vulkan/root.zig:78-87): streamed GEMV, weights staged per call. */
bool zlm_gpu_mat_vec(zlm_device *dev, uint32_t quant, const void *weight, size_t weight_len, size_t rows,
                     size_t k, const float *x, size_t x_len, float *out, size_t out_len);
/* Device.matMulBatch (vulkan/root.zig:89-102): out[t*rows + r], x token-major m*k. */
bool zlm_gpu_mat_mul_batch(zlm_device *dev, uint32_t quant, const void *weight, size_t weight_len,
                           size_t rows, size_t k, size_t m, const float *x, size_t x_len, float *out,
                           size_t out_len);
/* Device.matMulResident (vulkan/root.zig:104-115). */
bool zlm_gpu_mat_mul_resident(zlm_device *dev, zlm_resident *res, uint32_t quant, size_t rows, size_t k,
                              size_t m, const float *x, size_t x_len, float *out, size_t out_len);
/* Device.matVecResident (vulkan/root.zig:117-125). */
bool zlm_gpu_mat_vec_resident(zlm_device *dev, zlm_resident *res, uint32_t quant, size_t rows, size_t k,
                              const float *x, size_t x_len, float *out, size_t out_len);
/* Device.matVecResidentAsync (vulkan/root.zig:127-136). */
int32_t zlm_gpu_mat_vec_resident_async(zlm_device *dev, zlm_resident *res, uint32_t quant, size_t rows,
                                       size_t k, const float *x, size_t x_len);
/* Device.matVecResidentBurstAsync (vulkan/root.zig:138-148).  `first` stages x
 * into the device-owned burst buffer; later members must pass the same x
 * pointer and length, or they are refused. */
int32_t zlm_gpu_mat_vec_resident_burst_async(zlm_device *dev, zlm_resident *res, uint32_t quant, size_t rows,
                                             size_t k, const float *x, size_t x_len, bool first);
/* Device.matVecGateUpResidentBurstAsync (vulkan/root.zig:150-164).  `variant`
 * (a GpuVariant code; 0 keeps the quant code's own) selects the fused kernel's
 * row tile as it does for the plain GEMV: u4/u8 four output rows per wave
 * tile, un2/un4 two, the others one.  q4_0, q4_1 and q8_0 have the wider
 * tiles (the quants the reference grid lists gate_up variants for); other
 * quants run the one-row tile for every variant.  Both MLP ops apply
 * `variant` to their gate_up part. */
int32_t zlm_gpu_mat_vec_gate_up_resident_burst_async(zlm_device *dev, zlm_resident *res_gate,
                                                     zlm_resident *res_up, uint32_t quant, size_t rows,
                                                     size_t k, const float *x, size_t x_len, uint32_t act,
                                                     uint32_t variant, bool first);
/* Device.matVecMlpResidentBurstAsync (vulkan/root.zig:166-179). */
int32_t zlm_gpu_mat_vec_mlp_resident_burst_async(zlm_device *dev, zlm_resident *res_gate, zlm_resident *res_up,
                                                 zlm_resident *res_down, uint32_t quant, size_t rows, size_t k,
                                                 size_t ffn, const float *x, size_t x_len, uint32_t act,
                                                 uint32_t variant, bool first);
/* Device.matVecMlpPairResidentBurstAsync (vulkan/root.zig:181-194). */
int32_t zlm_gpu_mat_vec_mlp_pair_resident_burst_async(zlm_device *dev, zlm_resident *res_gate,
                                                      zlm_resident *res_up, zlm_resident *res_down,
                                                      uint32_t gu_quant, uint32_t down_quant, size_t rows,
                                                      size_t k, size_t ffn, const float *x, size_t x_len,
                                                      uint32_t act, uint32_t variant, bool first);
/* Device.waitResident (vulkan/root.zig:196-202). */
bool zlm_gpu_wait_resident(zlm_device *dev, int32_t handle, float *out, size_t out_len, size_t rows);
/* Device.matVecResidentBatch (vulkan/root.zig:204-212): <= ZLM_RING_SIZE ops sharing x. */
bool zlm_gpu_mat_vec_resident_batch(zlm_device *dev, size_t k, const float *x, size_t x_len,
                                    const zlm_resident_op *ops, size_t n_ops);
/* Device.uploadResident (vulkan/root.zig:214-224). */
zlm_resident *zlm_gpu_upload_resident(zlm_device *dev, const void *bytes, size_t len);
/* Device.freeResident (vulkan/root.zig:226-230). */
void zlm_gpu_free_resident(zlm_device *dev, zlm_resident *res);
/* Device.sync (vulkan/root.zig:232-235). */
void zlm_gpu_sync(zlm_device *dev);
/* Device.probeGpu (vulkan/root.zig:237-242, generic probe gpu/backend/root.zig:357-498). */
void zlm_gpu_probe(zlm_device *dev, size_t rows, size_t k, size_t m, zlm_probe *out);

/* The per-variant rate table behind one quant's probe entry (no reference
 * counterpart; for tests and tuning logs): rates[v] = GB/s of GpuVariant v,
 * measured as zlm_gpu_probe measures it (interleaved min-of-5 contract ops on
 * fillWeights-style inputs, rows <= 12288, k <= 4096), of the resident GEMV or,
 * with gate_up, of the fused gate_up.  False, with rates zeroed, when the quant
 * is unsupported or a variant did not run. */
bool zlm_gpu_probe_rates(zlm_device *dev, uint32_t ggml_type, bool gate_up, size_t rows, size_t k, double *rates);

/* Resident.bytes (reference gpu/backend/root.zig:241-244): the raw GGUF bytes uploaded. */
uint64_t zlm_gpu_resident_bytes(const zlm_resident *res);
/* Copy a resident's raw GGUF bytes back to the host (no reference
 * counterpart; tests and diagnostics, e.g. to check weights synthesised in
 * HBM against the CPU kernels).  Only before its first op converts them to the
 * device layout; `len` must equal the resident's byte count. */
bool zlm_gpu_resident_read_raw(zlm_device *dev, const zlm_resident *res, void *dst, size_t len);

/* ---- device-level entry points (no reference counterpart) ----
 * For callers that keep activations in HBM (the decode-step harness, the
 * benchmark) and for the bit-exact checks.  All work goes to the device's one
 * HIP stream, in order. */

/* Human-readable reason of the last failed call on this device ("" if none). */
const char *zlm_gpu_last_error(const zlm_device *dev);
/* Number of compute units, 0 when inert. */
int zlm_gpu_cu_count(const zlm_device *dev);
/* Free and total HBM bytes of the device, for the caller's residency budget
 * (the plan packs its resident set into `--vram` minus a driver headroom,
 * reference plan/root.zig:36-38, and uploads it with uploadResident,
 * runtime/session.zig:452-474).  A resident holds its raw bytes until the
 * first op names its quant; the conversion to the device layout briefly holds
 * both copies. */
bool zlm_gpu_vram_info(zlm_device *dev, uint64_t *free_bytes, uint64_t *total_bytes);
/* HBM a resident holds now: its raw bytes until the first op converts them,
 * then the device layout, plus the prefill GEMM's tiled copy once the tiled
 * GEMM has run on it (more than 4 tokens, or 3-4 tokens at k > 8192, k >
 * 16384 for Q4_1 / Q4_K; fewer tokens, and 5-8 tokens where the eight-slot
 * int-path GEMV runs, read the device layout). */
uint64_t zlm_gpu_resident_device_bytes(const zlm_resident *res);
/* HBM a rows x k weight of `quant` will hold once converted (its device
 * layout), plus its GEMM tiled copy when `with_gemm` (tensors the plan also
 * runs prefill GEMMs on); 0 for an unsupported quant or shape.  For the
 * plan's --vram budget before anything is uploaded; the conversion itself
 * briefly holds the raw bytes too. */
uint64_t zlm_gpu_layout_bytes(uint32_t quant, size_t rows, size_t k, bool with_gemm);
/* Free a resident's GEMM tiled copy (a later GEMM rebuilds it); false only
 * for a null or inert device or resident. */
bool zlm_gpu_release_gemm_tiles(zlm_device *dev, zlm_resident *res);
void *zlm_gpu_dev_malloc(zlm_device *dev, size_t bytes);
void zlm_gpu_dev_free(zlm_device *dev, void *ptr);
bool zlm_gpu_dev_upload(zlm_device *dev, void *dst, const void *src, size_t bytes);
bool zlm_gpu_dev_download(zlm_device *dev, void *dst, const void *src, size_t bytes);
/* Copy `bytes` (a multiple of 16, 16-byte aligned pointers) device to device
 * with the library's own copy kernel, and wait. */
bool zlm_gpu_dev_copy(zlm_device *dev, void *dst, const void *src, size_t bytes);
/* The same copy, enqueued on the device stream without waiting. */
bool zlm_gpu_dev_copy_enqueue(zlm_device *dev, void *dst, const void *src, size_t bytes);
/* Enqueue y_dev[0..rows) = W * x_dev on the device stream; no host copies. */
bool zlm_gpu_mat_vec_enqueue(zlm_device *dev, zlm_resident *res, uint32_t quant, size_t rows, size_t k,
                             const float *x_dev, float *y_dev);
/* The device-side form of matVecResidentBatch: n <= ZLM_RING_SIZE GEMVs over
 * one x_dev (k floats), res[i] (rows[i] x k, all of one quant type) into
 * y_dev[i], enqueued as one launch (no wait) -- or as n launches of the
 * single-op kernel where that kernel sums in another order (split-K: the
 * down-projection shapes; int8-plane x: Q4_K and Q6_K at k <= 4096, the
 * q4_0 fused forms), so every row always equals the single op's bit for bit. */
bool zlm_gpu_mat_vec_batch_enqueue(zlm_device *dev, zlm_resident *const *res, uint32_t quant, const size_t *rows,
                                   size_t n, size_t k, const float *x_dev, float *const *y_dev);
/* Enqueue the matrix product out_dev[t*rows + r] (x_dev: m x k fp32,
 * token-major) over a Q4_0, Q8_0, Q4_1 or Q4_K resident, by token count:
 * m = 1 the fp GEMV; m = 2 the two-token fp GEMV (k <= 16384, else a GEMV per
 * token); m = 3, 4 at k <= 8192 (16384 for Q4_1 / Q4_K) the int-path token GEMV (q8 activations
 * quantized in its prologue, the weights read once from the device layout),
 * and its eight-slot form at m = 5..8 for Q4_1 at k <= 4096 and Q4_K there up
 * to 8192 rows; otherwise the q8 activation quantizer, then an int8-MFMA GEMM over the
 * tiled copy (built on first use): up to 32 tokens the split-K small-M
 * kernel, past that the small-M kernel over several 32-token tiles or the
 * 128 x 64 tiled GEMM (each tile's blocks split over four or two wave
 * groups on small grids), whichever the library's cost model predicts faster for
 * (rows, k, m).  A token's results do not depend on the other tokens of the
 * call within one kernel. */
bool zlm_gpu_mat_mul_enqueue(zlm_device *dev, zlm_resident *res, uint32_t quant, size_t rows, size_t k, size_t m,
                             const float *x_dev, float *out_dev);
/* Enqueue `iters` prefill GEMMs (quantizer + GEMM each), rotating over `n_res`
 * residents, between two HIP events; *ms = elapsed GPU milliseconds. */
bool zlm_gpu_time_mat_mul(zlm_device *dev, zlm_resident *const *res, size_t n_res, uint32_t quant, size_t rows,
                          size_t k, size_t m, const float *x_dev, float *out_dev, int iters, double *ms);
/* Enqueue `iters` GEMVs, rotating over `n_res` residents, between two HIP events
 * on the device stream; *ms = elapsed GPU milliseconds between the events. */
bool zlm_gpu_time_mat_vec(zlm_device *dev, zlm_resident *const *res, size_t n_res, uint32_t quant, size_t rows,
                          size_t k, const float *x_dev, float *y_dev, int iters, double *ms);
/* One GEMV of a timed sequence (device pointers).  with_next != 0 joins this
 * GEMV and the next into one batch launch (zlm_gpu_mat_vec_batch_enqueue);
 * joined GEMVs share quant type, k and x_dev. */
typedef struct {
    zlm_resident *res;
    uint32_t quant;
    size_t rows;
    size_t k;
    const float *x_dev;
    float *y_dev;
    uint32_t with_next;
} zlm_gemv_desc;
/* Enqueue descs[0..n) in order, `iters` times, between two HIP events on the
 * device stream; *ms = elapsed GPU milliseconds between the events. */
bool zlm_gpu_time_gemv_sequence(zlm_device *dev, const zlm_gemv_desc *descs, size_t n, int iters, double *ms);
/* ---- the contract path, timed as zlm's executor drives it (no reference
 * counterpart; the rates zlm would see through this ABI) ----
 * One contract GEMV per iteration: matVecResidentBurstAsync (first, host x
 * staged) + waitResident (host y), rotating over n_res residents; *us = host
 * wall microseconds per op. */
bool zlm_gpu_time_contract_gemv(zlm_device *dev, zlm_resident *const *res, size_t n_res, uint32_t quant, size_t rows,
                                size_t k, int iters, double *us);
/* The same op's host wall time split (per op, microseconds): out[0] total,
 * out[1] the submit call (x copied into the slot's pinned buffer, the copy
 * kernel and the GEMV enqueued), out[2] the waitResident call (the GPU's run
 * as far as it is not yet done, the host's wake-up, y copied out), out[3] the
 * GPU time between events around the submission (copy kernel + GEMV). */
bool zlm_gpu_time_contract_gemv_split(zlm_device *dev, zlm_resident *const *res, size_t n_res, uint32_t quant,
                                      size_t rows, size_t k, int iters, double *out);
/* One layer's projections as separate residents (the GGUF tensors zlm uploads). */
typedef struct {
    zlm_resident *q, *k, *v, *o, *gate, *up, *down;
} zlm_contract_layer;
/* `iters` decode tokens through the contract ops only, in the executor's
 * burst/drain pattern for a discrete device (reference
 * runtime/executor.zig:236-258): per layer a burst of q, k, v over one host x
 * and their drain; o as a burst of its own and its drain; the fused
 * matVecMlpPairResidentBurstAsync and its drain; then the lm_head through
 * matVecResident.  The CPU-side glue (norms, RoPE, attention, residual adds)
 * is not run, so this is the GPU part of a token; *ms per token, host wall. */
bool zlm_gpu_time_contract_decode(zlm_device *dev, const zlm_contract_layer *layers, size_t n_layers, uint32_t quant,
                                  size_t hidden, size_t q_rows, size_t kv_rows, size_t ffn, zlm_resident *lm_head,
                                  uint32_t lm_quant, size_t vocab, int iters, double *ms);

/* GEMV forms of zlm_gemv_op; every form reads x from device memory:
 *   PLAIN     y = W x
 *   PAIR      y[r] = act(W x, W_up x)[r]             (the fused gate_up)
 *   NORM      y = W n,  n = RMSNorm(x, norm_w, eps)  (norm.zig:26-37)
 *   NORMPAIR  y[r] = act(W n, W_up n)[r]
 *   RESID     y = res + W x (res may alias y) */
enum { ZLM_FORM_PLAIN = 0, ZLM_FORM_PAIR = 1, ZLM_FORM_NORM = 2, ZLM_FORM_NORMPAIR = 3, ZLM_FORM_RESID = 4 };
typedef struct {
    uint32_t form;
    uint32_t quant;     /* ZLM_QUANT(type, variant); W and W_up share it */
    zlm_resident *w;    /* rows x k (the gate for the pair forms) */
    zlm_resident *w_up; /* pair forms: the up projection, rows x k */
    size_t rows;
    size_t k;
    const float *x;      /* device, k floats */
    const float *norm_w; /* device, k floats (norm forms) */
    float eps;           /* norm forms */
    uint32_t act;        /* pair forms: ZLM_ACT_SILU or ZLM_ACT_GELU */
    const float *res;    /* device, rows floats (RESID) */
    float *y;            /* device, rows floats */
} zlm_gemv_op;
/* Enqueue one GEMV op on the device stream (no host copies, no wait). */
bool zlm_gpu_gemv_op_enqueue(zlm_device *dev, const zlm_gemv_op *op);
/* ---- decode-step glue (device buffers; the ops between a layer's GEMVs) ----
 * Per-head q/k RMSNorm + rotate-half RoPE at *pos and the K/V cache append
 * (reference transformer/norm.zig:116-160, rope.zig:4-104, attention.zig:6-28).
 * qkv = [q: n_heads*hd | k: n_kv_heads*hd | v: n_kv_heads*hd] fp32; q_out
 * receives the rotated q; caches are [n_kv_heads][max_seq][hd] f16; *pos is
 * read on the device (a position >= max_seq appends nothing).  hd even, <= 256. */
bool zlm_gpu_qk_norm_rope_kv_enqueue(zlm_device *dev, const float *qkv, float *q_out, const float *q_norm_w,
                                     const float *k_norm_w, uint32_t n_heads, uint32_t n_kv_heads,
                                     uint32_t head_dim, float eps, float freq_base, const int32_t *pos,
                                     uint16_t *k_cache, uint16_t *v_cache, uint32_t max_seq);
/* Attention of every q head over positions [0, min(*pos + 1, max_seq)) of the
 * f16 caches (reference attention.zig:86-170; GQA by n_heads / n_kv_heads <= 4,
 * head_dim 128), scores scaled by `scale`; out: n_heads*128 fp32.  Split over
 * 64-position ranges, then merged; the partials live in library scratch that
 * the first call sizes (call once before capturing it into a graph). */
bool zlm_gpu_attention_enqueue(zlm_device *dev, const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                               uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, const int32_t *pos,
                               uint32_t max_seq, float scale, float *out);

/* The fused decode attention block: q/k head norm + RoPE, the K/V append at
 * *pos and the attention over [0, *pos] in one launch (the two calls above,
 * with `scale` and the q/k norms of the same reference routines), then the
 * split merge; qkv as for zlm_gpu_qk_norm_rope_kv_enqueue, out: n_heads*128
 * fp32.  head_dim 128, n_heads / n_kv_heads <= 4.  Uses the library scratch
 * of zlm_gpu_attention_enqueue (call once before capture). */
bool zlm_gpu_attention_decode_enqueue(zlm_device *dev, const float *qkv, const float *q_norm_w,
                                      const float *k_norm_w, uint32_t n_heads, uint32_t n_kv_heads,
                                      uint32_t head_dim, float eps, float freq_base, const int32_t *pos,
                                      uint16_t *k_cache, uint16_t *v_cache, uint32_t max_seq, float scale,
                                      float *out);
/* zlm_gpu_attention_decode_enqueue over a window: positions [0, window) of
 * the caches only (ceil(window / 64) splits; 1 <= window <= max_seq, the
 * caches' stride stays max_seq).  No reference counterpart: the decode step
 * at a position well below max_seq reads only the KV it needs (a serving loop
 * captures one graph per window bucket and replays the smallest bucket above
 * the position).  A position past the launched splits (64 * ceil(window /
 * 64) positions) gives NaN heads, not a silently shortened attention. */
bool zlm_gpu_attention_decode_window_enqueue(zlm_device *dev, const float *qkv, const float *q_norm_w,
                                             const float *k_norm_w, uint32_t n_heads, uint32_t n_kv_heads,
                                             uint32_t head_dim, float eps, float freq_base, const int32_t *pos,
                                             uint16_t *k_cache, uint16_t *v_cache, uint32_t max_seq,
                                             uint32_t window, float scale, float *out);

/* zlm_gpu_attention_decode_enqueue without any allocation: no counterpart in
 * the reference.  For callers that cannot allocate device memory at call time
 * (code under HIP graph capture before any eager call, serving loops that
 * forbid hipMalloc).  Same arguments, kernels and results (bit for bit) as
 * zlm_gpu_attention_decode_enqueue; the split partials live in a fixed
 * library array of ZLM_NOALLOC_ATTN_HEAD_SPLITS head-splits (8,519,680 bytes)
 * that each GPU the library runs on holds until the process ends.  Limit:
 * n_heads * ceil(max_seq / 64) <= ZLM_NOALLOC_ATTN_HEAD_SPLITS (e.g. 32 q
 * heads up to max_seq 32768); larger shapes return false with a reason in
 * zlm_gpu_last_error.  Every call on one GPU shares that GPU's array, which
 * keeps the last call's contents: calls that overlap on one GPU (two devices
 * or streams driving the same GPU concurrently) race. */
#define ZLM_NOALLOC_ATTN_HEAD_SPLITS 16384u
bool zlm_gpu_attention_decode_enqueue_noalloc(zlm_device *dev, const float *qkv, const float *q_norm_w,
                                              const float *k_norm_w, uint32_t n_heads, uint32_t n_kv_heads,
                                              uint32_t head_dim, float eps, float freq_base, const int32_t *pos,
                                              uint16_t *k_cache, uint16_t *v_cache, uint32_t max_seq, float scale,
                                              float *out);

/* ---- HIP graphs over the device stream ----
 * Everything enqueued between capture_begin and capture_end is recorded, not
 * run.  Only the *_enqueue entry points can be captured: the host-buffer
 * contract ops (matVec*, matMul*, waitResident, uploadResident, the probe and
 * timers) fail while a capture is open.  Ops that allocate or convert layouts
 * on first use (a resident's first op, a resident's first matMul, the
 * attention and GEMM scratch) must have run once eagerly before their
 * capture; under capture they fail instead.  The library never frees or
 * replaces scratch that a captured graph references while that graph exists:
 * after capturing an attention call, an eager attention call that needs more
 * partials fails with the reason; after capturing a matMul, an eager matMul
 * that needs more activation scratch, a rebuild of a resident's GEMM tiles
 * (a matMul at another k) and zlm_gpu_release_gemm_tiles fail -- until those
 * graphs are destroyed (zlm_gpu_graph_destroy with the device that captured
 * them).  Freeing a resident (or any caller buffer) a live graph reads is the
 * caller's error. */
typedef struct zlm_graph zlm_graph;
bool zlm_gpu_capture_begin(zlm_device *dev);
zlm_graph *zlm_gpu_capture_end(zlm_device *dev);
/* Launch the graph `iters` times back to back and wait; *ms (optional) = GPU
 * milliseconds between events around the launches.  Refused (false, reason in
 * zlm_gpu_last_error) while a rocprofiler library is loaded in the process:
 * replays of the decode step under rocprofv3's kernel trace aborted inside
 * hipGraphLaunch; profile eager launches instead. */
bool zlm_gpu_graph_launch(zlm_device *dev, zlm_graph *graph, int iters, double *ms);
void zlm_gpu_graph_destroy(zlm_device *dev, zlm_graph *graph);
/* Whether a rocprofiler library appears in a /proc/<pid>/maps-format file
 * (null: this process's own map): the check behind the replay refusal. */
bool zlm_gpu_profiler_loaded(const char *maps_path);
/* What the host reads from a GEMV entry point's name before launching it
 * (no device needed): *role = the form it computes (ZLM_FORM_*), 16 the batch
 * kernel, 17 the two-token GEMV, 18 the int-path token GEMV; *struct_args =
 * it takes one GemvArgs block (else the plain GEMV's six arguments).  False
 * for a name that is not zlm_gemv_<quant>_...  Lets a test check the parse
 * against the code objects' kernel-argument metadata. */
bool zlm_gpu_kernel_convention(const char *name, int32_t *role, bool *struct_args);
/* Device bytes the library itself holds on `dev` (staging, attention and GEMM
 * scratch; not residents, not the fixed no-alloc array). */
uint64_t zlm_gpu_scratch_device_bytes(const zlm_device *dev);

/* ---- launch log (no reference counterpart; tests and diagnostics) ----
 * Every launch is checked on the host against the kernel-dispatch limits
 * (workgroup of 64..1024 work-items in whole waves; grid x workgroup below
 * 2^32 work-items in x, at most 65536 workgroups in y and z; the kernel's
 * static LDS at most 160 KiB) and fails with its parameters otherwise.  With
 * the log on, each launch's parameters are recorded (at most 65536 records;
 * enabling or disabling clears the log); zlm_gpu_launch_log_read copies up to
 * `max` records and returns how many there are. */
typedef struct {
    const char *what;     /* the op's label (static string) */
    uint32_t grid_x, grid_y, grid_z;  /* workgroups */
    uint32_t block;       /* work-items per workgroup */
    uint32_t lds_bytes;   /* the kernel's static LDS */
} zlm_launch_record;
bool zlm_gpu_launch_log(zlm_device *dev, bool enable);
size_t zlm_gpu_launch_log_read(const zlm_device *dev, zlm_launch_record *out, size_t max);

/* ---- synthetic data generated in HBM (benchmark, large-shape tests) ----
 * A resident of `n_blocks` raw GGUF blocks (q4_0: f16 d + 16 random bytes;
 * q8_0: f16 d + 32 int8 uniform in [-127, 127]) with d = |N(0,1)| * scale. */
zlm_resident *zlm_gpu_synth_resident(zlm_device *dev, uint32_t ggml_type, size_t n_blocks, uint64_t seed,
                                     float scale);
/* n f16 values N(0,1) * scale into device memory. */
bool zlm_gpu_synth_f16(zlm_device *dev, uint16_t *dst, size_t n, uint64_t seed, float scale);

/* Dequantize the first n_elements of a resident from its device layout into host `out`. */
bool zlm_gpu_dequant_resident(zlm_device *dev, zlm_resident *res, uint32_t quant, size_t n_elements, float *out);
/* Quantize host x (n floats, n % 32 == 0) to q8 blocks on the device. */
bool zlm_gpu_quantize_act_q8(zlm_device *dev, const float *x, size_t n, int8_t *qx, float *dx, int32_t *sums);

#ifdef __cplusplus
}
#endif
#endif /* ZLM_GPU_HIP_H */
