// okq_neighbours.hip -- the f32 operations on either side of the quantized
// projections, for the paths that cannot fold them into the GEMV prologue
// (batched rows on the MFMA GEMM, rows the streaming GEMV does not take).
//
//   rmsnorm: out[r, i] = (x[r, i] * (1 / sqrt(sum_i x[r, i]^2 / hidden + eps))) * w[i]
//            (crates/kernels/src/rmsnorm.rs:73-128, same order of operations;
//            the sum of squares is reduced in a fixed tree order)
//   swiglu : out[i] = (gate[i] * (1 / (1 + exp(-gate[i])))) * up[i]
//            (crates/kernels/src/mlp.rs:77-88, :233-238)
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

// One workgroup of 256 threads per row; float4 accesses when the row allows.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, int64_t hidden,
                                                      const float *__restrict__ w, float eps,
                                                      float *__restrict__ out) {
  __shared__ float red[4];
  const float *row = x + (int64_t)blockIdx.x * hidden;
  float *orow = out + (int64_t)blockIdx.x * hidden;
  const int tid = (int)threadIdx.x;
  float ss = 0.0f;
  for (int64_t i = tid; i < hidden; i += 256) {
    const float v = row[i];
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(tot / (float)hidden + eps);
  for (int64_t i = tid; i < hidden; i += 256) orow[i] = row[i] * inv * w[i];
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float *__restrict__ gate, const float *__restrict__ up,
                                                     int64_t n, float *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float g = gate[i];
  const float sig = 1.0f / (1.0f + expf(-g));
  out[i] = (g * sig) * up[i];
}

hipError_t launch_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *weight, float eps, float *out,
                          hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  launch_timed(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0u, s, x, hidden, weight, eps, out);
  return hipGetLastError();
}

hipError_t launch_swiglu(const float *gate, const float *up, int64_t n, float *out, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  launch_timed(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0u, s, gate, up, n, out);
  return hipGetLastError();
}

}  // namespace okq
