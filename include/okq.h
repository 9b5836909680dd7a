/*
 * okq.h -- C-ABI of libokq.so, the MI355X (gfx950) k-quant linear path.
 *
 * The library implements Ocelotl's quantized linear projection for the GGUF
 * block formats Q8_0 (type id 8), Q4_K (12), Q5_K (13) and Q6_K (14) with hand-written
 * HIP kernels: dequantize, a fused dequant-GEMV for decode and an MFMA
 * dequant-GEMM for prefill.  Weights stay in the GGUF layout: tensor shape
 * [ne0 = in_features, ne1 = out_features], each row one output feature made of
 * in_features / block_elems consecutive blocks.
 *
 * Conventions (mirroring the reference's kernel contract):
 *   - every entry point validates before launch and returns an okq_status; on
 *     failure okq_last_error() holds a message, and nothing was launched
 *     (crates/kernels/src/lib.rs:2443-2497, docs/design/kernels.md:96-99);
 *   - `out` buffers are caller-allocated device memory (lib.rs:106-116);
 *   - `stream` is a hipStream_t (NULL = the null stream); work is enqueued
 *     asynchronously on it;
 *   - results are deterministic: fixed reduction order, no float atomics.
 * Thread safety: all entry points may be called from several host threads; the
 * device used is the calling thread's current HIP device.  Calls on one
 * stream enqueue their kernels as one uninterrupted sequence (a per-stream
 * lock), so threads sharing a stream also share its workspace safely.
 */
#ifndef OKQ_H
#define OKQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  OKQ_E_SHAPE / E_ARG map to OcelotlError::Kernel
 * (crates/core/src/lib.rs:15-99, KernelError{backend:"hip-gfx950", message});
 * OKQ_E_TYPE maps to OcelotlError::Unsupported (lib.rs:1662-1671). */
typedef enum okq_status {
    OKQ_OK = 0,
    OKQ_E_SHAPE = 1,  /* lengths/shapes inconsistent, not block-aligned, or too large */
    OKQ_E_TYPE = 2,   /* GGML tensor type not supported by this path */
    OKQ_E_ALIGN = 3,  /* pointer misaligned for the kernel's vector loads */
    OKQ_E_NODEV = 4,  /* no HIP device, or the device is not gfx950 */
    OKQ_E_LAUNCH = 5, /* HIP runtime error at launch or copy */
    OKQ_E_ARG = 6,    /* null pointer or invalid argument value */
    OKQ_E_ALLOC = 7   /* device allocation failed */
} okq_status;

/* GGML tensor type ids, as GgmlTensorType::from_raw
 * (crates/loader/src/gguf_inspect.rs:170-206). */
enum {
    OKQ_TYPE_F32 = 0,
    OKQ_TYPE_F16 = 1,
    OKQ_TYPE_Q4_0 = 2,  /* dequantize / get_rows only */
    OKQ_TYPE_Q4_1 = 3,  /* dequantize / get_rows only */
    OKQ_TYPE_Q5_0 = 6,  /* dequantize / get_rows only */
    OKQ_TYPE_Q5_1 = 7,  /* dequantize / get_rows only */
    OKQ_TYPE_Q8_0 = 8,
    OKQ_TYPE_Q2_K = 10, /* dequantize / get_rows only */
    OKQ_TYPE_Q3_K = 11, /* dequantize / get_rows only */
    OKQ_TYPE_Q4_K = 12,
    OKQ_TYPE_Q5_K = 13,
    OKQ_TYPE_Q6_K = 14,
    OKQ_TYPE_BF16 = 30
};

/* ---- identity and errors ---------------------------------------------- */

/* Backend name, following the backend_id convention of
 * crates/kernels/src/cubecl_backend.rs:2268-2272: "hip-gfx950". */
const char *okq_backend_name(void);

/* Copies the calling thread's last error message (NUL-terminated, truncated to
 * len) and returns its full length. */
size_t okq_last_error(char *buf, size_t len);

/* ---- GGUF tensor layout (fills the byte_len = None gap of
 *      GgmlTensorType::fixed_element_size, gguf_inspect.rs:208-219) ------- */

/* Elements and bytes per block: Q8_0 32/34, Q4_K 256/144, Q6_K 256/210;
 * Q4_0 32/18, Q4_1 32/20, Q5_0 32/22, Q5_1 32/24, Q2_K 256/84, Q3_K 256/110,
 * Q5_K 256/176; and 1/4, 1/2, 1/2 for F32, F16, BF16.  OKQ_E_TYPE for
 * anything else.  The linear entry points take Q8_0, Q4_K, Q5_K and Q6_K weights;
 * okq_dequantize and okq_get_rows_q take every block format listed here. */
okq_status okq_type_info(uint32_t ggml_type, int64_t *block_elems, int64_t *block_bytes);

/* Bytes of one row of ne0 elements; OKQ_E_SHAPE if ne0 is not a positive
 * multiple of the block size. */
okq_status okq_row_bytes(uint32_t ggml_type, int64_t ne0, int64_t *out_bytes);

/* Byte length of a GGUF tensor with `n_dims` dims in ne order (shape[0] =
 * ne0, contiguous).  Overflow is OKQ_E_SHAPE (gguf_inspect.rs:331-342). */
okq_status okq_tensor_bytes(uint32_t ggml_type, const int64_t *shape, int n_dims, uint64_t *out_bytes);

/* ---- device ------------------------------------------------------------ */

/* Selects device `ordinal` for the calling thread and checks it is gfx950
 * (Device::Gpu{ordinal}, crates/core/src/lib.rs:438-441). */
okq_status okq_init(int ordinal);
okq_status okq_device_count(int *count);
okq_status okq_alloc(void **ptr, size_t bytes);
okq_status okq_free(void *ptr);
okq_status okq_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
okq_status okq_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
okq_status okq_sync(void *stream);

/* ---- compute ----------------------------------------------------------- */

/* dequantize(type, src_bytes, n_elems, out_f32): the reference defines no
 * dequant signature; this follows the linear_out_by_in style
 * (lib.rs:106-116).  n must be a multiple of the block size; src holds
 * n / block_elems blocks.  Bit-exact with the CPU oracle (every product and
 * difference rounded separately, fp16 decoded exactly as
 * crates/loader/src/safetensors_values.rs:155-183).  Every block format of
 * okq_type_info; src must be 16-byte aligned for Q4_K, 2-byte otherwise. */
okq_status okq_dequantize(uint32_t ggml_type, const void *src, int64_t n, float *dst, void *stream);

/* Quantized embedding lookup: out[j, :] = dequantize(row ids[j] of W) for
 * j < n_ids, bit-identical to okq_dequantize of that row.  W holds the GGUF
 * blocks of an [ne0, ne1] tensor (ne0 = hidden, ne1 = vocab rows), w_bytes =
 * ne1 * row_bytes(ne0); ids are in HOST memory and every id must be < ne1;
 * out: [n_ids, ne0] f32 (device).  n_ids == 0 is a no-op.  Replaces the f32
 * row copy of the reference's token embedding step
 * (crates/models/src/qwen/qwen2_5/prefill.rs:95-105, decode.rs:51-52) for a
 * quantized table such as Gemma4's Q4_K token_embd.weight [2560, 262144];
 * the id check and its message follow decode.rs:33-38. */
okq_status okq_get_rows_q(uint32_t w_type, const void *w, uint64_t w_bytes, int64_t ne0, int64_t ne1,
                          const uint32_t *ids, int64_t n_ids, float *out, void *stream);

/* Quantized counterpart of KernelBackend::linear_out_by_in
 * (crates/kernels/src/lib.rs:106-116) and linear_d (:192-202):
 *   out[r, o] = bias[o] + sum_k x[r, k] * W[o, k]
 * x: [rows, in_features] f32 (device); w: GGUF blocks of an [out_features,
 * in_features] tensor, w_bytes = out_features * row_bytes(in_features);
 * bias: [out_features] f32 or NULL; out: [rows, out_features] f32.
 * rows == 0 or out_features == 0 is a no-op.  Up to 8 rows run the fused
 * dequant-GEMV (each pass over the weights serving up to four rows), except
 * weights large enough for the MFMA kernel to repay its fixed cost: from 2 MB
 * at 6-8 rows, from 8 MB at 5 rows, and at 3-4 rows from 16 MB when
 * in_features >= 8192 or from 64 MB otherwise; more rows run the MFMA
 * dequant-GEMM (Q4_K, Q5_K, Q6_K, and Q8_0 when in_features is a multiple of 256),
 * which for up to 32 rows streams the weights once with the rows in one or
 * two MFMA tiles. */
okq_status okq_linear_out_by_in_q(const float *x, int64_t rows, int64_t in_features, uint32_t w_type,
                                  const void *w, uint64_t w_bytes, int64_t out_features, const float *bias,
                                  float *out, void *stream);

/* Same contract with bf16 activations x: [rows, in_features] (prefill,
 * decoded exactly as safetensors_values.rs:115-123). */
okq_status okq_linear_out_by_in_q_bf16(const uint16_t *x, int64_t rows, int64_t in_features, uint32_t w_type,
                                       const void *w, uint64_t w_bytes, int64_t out_features, const float *bias,
                                       float *out, void *stream);

/* okq_linear_out_by_in_q without any device allocation: the same contract,
 * dispatch and kernels (bit-identical outputs), with the MFMA kernels'
 * scratch (activation planes, split-K partials) taken from a static 64 MiB
 * device array instead of the per-stream workspace, so no call allocates or
 * frees memory (hipMalloc, hipFree, or any library routine that allocates).
 * No counterpart in the reference: it serves callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation.  Limits: a problem whose scratch exceeds 64 MiB fails with
 * OKQ_E_SHAPE before anything launches (f32 activations: every Llama-3-8B
 * shape up to 32 rows, the 128256 x 4096 output head included, whose 32-row
 * split-K partials take 62.6 MiB; the tiled GEMM while 2 x rows x
 * in_features x 2 bytes plus its sums and partials fit); every call on one device
 * shares the array and keeps the last call's contents, so calls that overlap
 * on one device (several streams or threads at once) race.  The array's
 * device address is resolved once per device by okq_init (or by the first
 * call on that device). */
okq_status okq_linear_out_by_in_q_noalloc(const float *x, int64_t rows, int64_t in_features, uint32_t w_type,
                                          const void *w, uint64_t w_bytes, int64_t out_features, const float *bias,
                                          float *out, void *stream);

/* Explicit-path variants of okq_linear_out_by_in_q (same arguments): the fused
 * dequant-GEMV (one weight pass per activation row) and the MFMA dequant-GEMM.
 * For benchmarks and tests that pin a path. */
okq_status okq_gemv(const float *x, int64_t rows, int64_t in_features, uint32_t w_type, const void *w,
                    uint64_t w_bytes, int64_t out_features, const float *bias, float *out, void *stream);
okq_status okq_gemm(const float *x, int64_t rows, int64_t in_features, uint32_t w_type, const void *w,
                    uint64_t w_bytes, int64_t out_features, const float *bias, float *out, void *stream);
okq_status okq_gemm_bf16(const uint16_t *x, int64_t rows, int64_t in_features, uint32_t w_type, const void *w,
                         uint64_t w_bytes, int64_t out_features, const float *bias, float *out, void *stream);

/* Several quantized linears that read the same activations, in one pass over
 * their weights:  out[i][r, o] = bias[i][o] + sum_k x[r, k] * W_i[o, k]  for
 * i < count (1..4), every W_i of type w_type with in_features columns and
 * out_features[i] rows (w_bytes[i] bytes).  The decode GEMV streams the
 * matrices' concatenated rows in one launch per activation row, quantizing x
 * once.  `bias` may be NULL (no bias anywhere) or hold NULL entries.  Each
 * matrix is validated like okq_gemv before anything launches.  A matrix that
 * okq_linear_out_by_in_q would not give to the GEMV at this row count (the
 * large weights of its 3-8 row rule, every weight above 8 rows) is computed
 * by the MFMA kernels
 * instead: alone through that entry
 * point's dispatch, or -- two or more of them at up to 32 rows -- together in
 * one decode-batch launch whose K split follows their combined columns.
 * Outputs equal okq_linear_out_by_in_q's on each matrix bit for bit, except
 * those of such a shared decode-batch launch, which agree within the
 * reference rule.  No counterpart in the reference,
 * whose callers compute such groups one projection at a time: the gate/up
 * pair of mlp_gated_silu (crates/kernels/src/lib.rs:150-162,
 * crates/kernels/src/mlp.rs:139-250) and the q/k/v projections of one
 * normalized hidden state. */
okq_status okq_gemv_multi(const float *x, int64_t rows, int64_t in_features, uint32_t w_type, int count,
                          const void *const *w, const uint64_t *w_bytes, const int64_t *out_features,
                          const float *const *bias, float *const *out, void *stream);

/* okq_gemv_multi for matrices of different formats: w_types[i] is matrix i's
 * GGML type (the layers of a Q4_K_M model store q/k in Q4_K and v in Q6_K).
 * Matrices of one format are grouped as okq_gemv_multi groups them; at
 * decode-batch row counts (up to 32) the Q4_K and Q6_K matrices that
 * okq_linear_out_by_in_q gives to the MFMA kernels share one decode-batch
 * launch, whose outputs agree with each matrix's own call within the
 * reference rule.  Validation and errors as okq_gemv_multi.  No counterpart in
 * the reference (its callers compute q, k and v one linear at a time). */
okq_status okq_linear_multi_q(const float *x, int64_t rows, int64_t in_features, int count, const uint32_t *w_types,
                              const void *const *w, const uint64_t *w_bytes, const int64_t *out_features,
                              const float *const *bias, float *const *out, void *stream);

/* ---- instrumentation --------------------------------------------------- */

/* ---- neighbours of the projections ------------------------------------ */

/* RMSNorm, KernelBackend::rmsnorm (crates/kernels/src/lib.rs:139-147,
 * crates/kernels/src/rmsnorm.rs:73-128): per row of x [rows, hidden],
 * out = (x * (1 / sqrt(sum(x^2) / hidden + epsilon))) * weight.  Device f32
 * buffers; weight 16-byte aligned.  Errors follow rmsnorm.rs:81-114. */
okq_status okq_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *weight, float epsilon, float *out,
                       void *stream);

/* RMSNorm followed by up to four quantized projections of the normalised
 * rows (the q/k/v of an attention block):
 *   out[i][r, o] = bias[i][o] + sum_k rmsnorm(x)[r, k] * W_i[o, k].
 * Arguments as okq_rmsnorm and okq_gemv_multi.  A single row runs the GEMV
 * with the normalisation folded into its activation prologue (no normalised
 * copy of x is written); more rows normalise into a per-stream workspace
 * first and then stream each weight once per four rows.  No counterpart in the reference, whose blocks
 * call rmsnorm and then each linear (crates/models/src/qwen/qwen2_5/prefill.rs). */
okq_status okq_rmsnorm_linear_q_multi(const float *x, int64_t rows, int64_t hidden, const float *norm_weight,
                                      float epsilon, uint32_t w_type, int count, const void *const *w,
                                      const uint64_t *w_bytes, const int64_t *out_features, const float *const *bias,
                                      float *const *out, void *stream);

/* Quantized gated-SiLU MLP, KernelBackend::mlp_gated_silu
 * (crates/kernels/src/lib.rs:150-162, crates/kernels/src/mlp.rs:139-250):
 *   out = down(silu(gate(x)) * up(x)),
 * x [rows, hidden]; gate and up [hidden -> intermediate] and down
 * [intermediate -> hidden] as GGUF blocks (rows = output features, so the
 * byte lengths are intermediate * row_bytes(hidden) and hidden *
 * row_bytes(intermediate)); gate_buf, up_buf [rows, intermediate] caller-owned
 * scratch; out [rows, hidden].  Device buffers, x/gate_buf/up_buf 16-byte
 * aligned.  Decode-sized rows (rows <= 8) run gate+up as one grouped GEMV
 * when they share a format.  A single row folds silu(gate) * up into the down
 * GEMV's prologue whenever the down weight takes the streaming GEMV (gate_buf
 * then holds gate(x)); otherwise silu(gate(x)) * up(x) is left in gate_buf,
 * as the reference does (when gate and up share one decode-batch launch that
 * splits K, by its reduction: no separate pass over the intermediate).  up_buf always holds up(x).  Treat both as scratch.  Zero rows, hidden or
 * intermediate are errors (mlp.rs:151-165). */
okq_status okq_mlp_gated_silu_q(const float *x, int64_t rows, int64_t hidden, int64_t intermediate,
                                uint32_t gate_type, const void *gate_w, uint64_t gate_bytes, uint32_t up_type,
                                const void *up_w, uint64_t up_bytes, uint32_t down_type, const void *down_w,
                                uint64_t down_bytes, float *gate_buf, float *up_buf, float *out, void *stream);

/* The next compute kernel this thread launches through okq_dequantize,
 * okq_linear_out_by_in_q*, okq_gemv or okq_gemm* records `start` and `stop`
 * (hipEvent_t, created with timing enabled) at the begin and end of its
 * dispatch (hipExtLaunchKernelGGL), so hipEventElapsedTime(start, stop) is
 * that kernel's own duration.  One-shot: cleared by the launch; pass NULLs to
 * clear.  Calls that split into several kernels time the first one.  No
 * counterpart in the reference (its benchmarks time whole phases with
 * Instant, src/main.rs:419-598). */
okq_status okq_set_launch_events(void *start, void *stop);

/* ---- data preparation -------------------------------------------------- */

/* Quantize n f32 values (device) into GGUF blocks (device), on the GPU.  The
 * reference has no quantizer; the algorithm is fixed by the CPU oracle and the
 * bytes match it exactly. */
okq_status okq_quantize(uint32_t ggml_type, const float *src, int64_t n, void *dst, void *stream);

/* dst[i] = N(0, sigma) sample number (offset + i) of stream `seed`
 * (SplitMix64 counter stream, Irwin-Hall of twelve 24-bit uniforms summed in
 * integers): identical floats on CPU and GPU. */
okq_status okq_fill_normal(uint64_t seed, int64_t offset, int64_t n, float sigma, float *dst, void *stream);

/* f32 -> bf16, round to nearest even. */
okq_status okq_f32_to_bf16(const float *src, int64_t n, uint16_t *dst, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OKQ_H */
