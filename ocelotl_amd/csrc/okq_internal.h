// okq_internal.h -- launcher declarations shared by the C-ABI layer and the
// kernel translation units.  Every launcher assumes its arguments were
// validated by okq_runtime.hip (shapes, alignment, 32-bit index ranges).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace okq {

// Optional dispatch-timing events for the next launch (see
// okq_set_launch_events).  take_launch_events() returns and clears them.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents take_launch_events();

// Launch `kernel` on s, recording the thread's pending timing events if any.
template <typename... KArgs, typename... Args>
inline void launch_timed(void (*kernel)(KArgs...), dim3 grid, dim3 block, unsigned shmem, hipStream_t s,
                         Args... args) {
  LaunchEvents ev = take_launch_events();
  if (ev.start || ev.stop) {
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, ev.start, ev.stop, 0, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
  }
}

hipError_t launch_dequantize(int type, const void *src, int64_t n, float *dst, hipStream_t s);
hipError_t launch_quantize(int type, const float *src, int64_t n, void *dst, hipStream_t s);
hipError_t launch_fill_normal(uint64_t seed, int64_t offset, int64_t n, float sigma, float *dst, hipStream_t s);
hipError_t launch_f32_to_bf16(const float *src, int64_t n, uint16_t *dst, hipStream_t s);
hipError_t launch_bf16_to_f32(const uint16_t *src, int64_t n, float *dst, hipStream_t s);

// Row gather: out[j, :] = dequant(W row ids[j]) for j < n (ids in host memory,
// each < the weight's row count).  Row ids ride in the kernel arguments,
// kGatherMaxIds per launch.
constexpr int kGatherMaxIds = 480;
struct GatherIds {
  uint32_t id[kGatherMaxIds];
};
hipError_t launch_get_rows(int type, const void *w, int64_t row_bytes, int64_t ne0, const uint32_t *ids, int64_t n,
                           float *out, hipStream_t s);

// Fused dequant-GEMV for one activation row: y[o] = bias[o] + sum_k x[k] W[o,k].
// cu_count sizes the persistent grid.
hipError_t launch_gemv(int type, const float *x, int64_t K, const void *w, int64_t N, const float *bias, float *y,
                       int cu_count, hipStream_t s);
// Several matrices of one format and K against the same activation rows in
// one launch (row-concatenated); matrices the streaming kernel cannot take
// run on their own.  count <= kGemvMaxProblems.
constexpr int kGemvMaxProblems = 4;
// Optional transform of x ahead of its quantisation: none, RMSNorm with weight
// `a` and epsilon `eps`, or the gated SiLU silu(x) * a (x = gate, a = up).
// A transform needs every matrix of the launch to pass gemv_streams.
enum GemvProKind { kProNone = 0, kProRms = 1, kProSwiGLU = 2 };
struct GemvPro {
  int kind;
  const float *a;
  float eps;
};
bool gemv_streams(int type, int64_t K, const void *w, int64_t N);
// x [rows, K] and y[i] [rows, N[i]] row-major; every pass over the weights
// serves up to four activation rows.  A prologue needs rows == 1.
hipError_t launch_gemv_multi(int type, const float *x, int64_t K, int64_t rows, int count, const void *const *w,
                             const int64_t *N, const float *const *bias, float *const *y, int cu_count,
                             hipStream_t s, const GemvPro &pro);

// The same neighbours on their own (rows of `hidden` values): RMSNorm with the
// reference's order of operations, and the gated SiLU over n values.
hipError_t launch_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *weight, float eps, float *out,
                          hipStream_t s);
hipError_t launch_swiglu(const float *gate, const float *up, int64_t n, float *out, hipStream_t s);

// MFMA dequant-GEMM: Y[M, N] = bias + X[M, K] W[N, K]^T with X f32 or bf16.
// How launch_gemm runs an (M, N, K) problem: tile rows, split-K factor and
// the workspace layout (tiled kernel: activation planes, per-32 sums, row
// scales, split-K partials; decode-batch kernel: split-K partials only),
// 256-byte aligned offsets from the workspace base.
struct GemmPlan {
  int bm;              // 32: the decode-batch kernel (M <= 32), else the tile height
  int groups;          // decode-batch kernel: column groups per K slice
  int kwaves;          // decode-batch kernel, unsplit K: waves that split a tile's K inside the workgroup;
                       // Q8_0 kernel: waves per workgroup (4 or 8)
  int ksplit;
  int wide;            // weights dequantised in registers (bf16 activations): 1 the wide kernel (Q4_K / Q5_K,
                       // 128 x 256 tiles, one workgroup per CU), 2 the pair kernel (Q4_K / Q5_K, 128 x 128
                       // tiles, two per CU), 3 the Q8_0 kernel (128 x 128 or 128 x 256 tiles),
                       // 4 the Q6_K kernel (128 x 256 tiles)
  size_t off_lo, off_sums, off_rscale, off_part, workspace;
};
GemmPlan gemm_plan(int type, int64_t M, int64_t N, int64_t K, bool x_is_bf16, int cu_count);
// `workspace` holds plan.workspace bytes (256-aligned); it is reused by later
// calls on the stream.
hipError_t launch_gemm(int type, const void *x, bool x_is_bf16, int64_t M, int64_t K, const void *w, int64_t N,
                       const float *bias, float *y, void *workspace, const GemmPlan &plan, hipStream_t s);
// Up to kDecMats matrices of one format and K that read the same activations
// in one decode-batch launch (plan: gemm_plan with N = sum of the matrices'
// rows rounded up to 16 each, which must pick the decode-batch kernel).
// swiglu (two matrices of equal rows, gate then up): when the plan splits K,
// the reduction leaves up in y[1] and silu(gate) * up in y[0].
constexpr int kDecMats = 4;
constexpr int kGemmDecodeRows = 32;  // batches up to this many rows take the decode-batch kernel
hipError_t launch_gemm_decode_multi(int type, const void *x, bool x_is_bf16, int64_t M, int64_t K, int count,
                                    const void *const *w, const int64_t *N, const float *const *bias, float *const *y,
                                    void *workspace, const GemmPlan &plan, hipStream_t s, bool swiglu = false);

// Q4_K and Q6_K matrices that read the same activations in one decode-batch
// launch: types[] lists the Q4_K matrices first, then the Q6_K ones (at least
// one of each, count <= kDecMats); the plan is gemm_plan's for their combined
// tile columns.  Each workgroup runs one format; one split-K reduction.
hipError_t launch_gemm_decode_mixed(const void *x, bool x_is_bf16, int64_t M, int64_t K, int count, const int *types,
                                    const void *const *w, const int64_t *N, const float *const *bias, float *const *y,
                                    void *workspace, const GemmPlan &plan, hipStream_t s);

// True when launch_gemm supports this (type, M, K, N): Q4_K, Q6_K and Q8_0
// with K a multiple of 256.
bool gemm_supported(int type, int64_t M, int64_t K, int64_t N);

// The Q4_K / Q5_K prefill kernel with register-dequantised weights
// (okq_gemm_wide.hip) over the pre-pass's planes: its shape limits, its
// 128 x 256 tile count, and its launch (ksplit > 1: raw partials
// [ksplit][M][N] for splitk_reduce_kernel).
bool gemm_wide_supported(int type, int64_t M, int64_t K, int64_t N);
int gemm_wide_tiles(int64_t M, int64_t N);
hipError_t launch_gemm_wide(int type, const _Float16 *xhi, const void *xsum, const float *rscale, const void *w,
                            const float *bias, float *y, int64_t M, int64_t N, int64_t K, int ksplit, float *part,
                            hipStream_t s);
// The same contraction with 128 x 128 tiles and two 4-wave workgroups per CU
// (okq_gemm_pair.hip): same shape limits, operands and partial layout.
int gemm_pair_tiles(int64_t M, int64_t N);
hipError_t launch_gemm_pair(int type, const _Float16 *xhi, const void *xsum, const float *rscale, const void *w,
                            const float *bias, float *y, int64_t M, int64_t N, int64_t K, int ksplit, float *part,
                            hipStream_t s);
// Q6_K with bf16 activations (okq_gemm_q6.hip): the pre-pass's fp16 plane and
// row scales, 128 x 256 tiles, one 8-wave workgroup per CU, the weights as
// two exact fp16 planes dequantised in registers; K a multiple of 256 split
// into ksplit <= K / 256 slices of whole super-blocks, the same partial layout.
int gemm_q6_tiles(int64_t M, int64_t N);
hipError_t launch_gemm_q6(const _Float16 *xhi, const float *rscale, const void *w, const float *bias, float *y,
                          int64_t M, int64_t N, int64_t K, int ksplit, float *part, hipStream_t s);
// Q8_0 with bf16 activations (okq_gemm_q8.hip): x [M, K] bf16 straight into
// bf16 MFMAs (no pre-pass), 128 x 32 waves tiles (waves = 4: two workgroups
// per CU; 8: one), K split in stages of 128 (ksplit <= K / 128; K a multiple
// of 256); ksplit > 1 writes unscaled partials [ksplit][M][N] for
// splitk_reduce_kernel.
int gemm_q8_tiles(int64_t M, int64_t N, int waves);
hipError_t launch_gemm_q8(const void *x, const void *w, const float *bias, float *y, int64_t M, int64_t N, int64_t K,
                          int ksplit, int waves, float *part, hipStream_t s);

}  // namespace okq
