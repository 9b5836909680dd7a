// okq_gemv.hip -- fused dequant-GEMV for decode (one activation row).
//
// Design (gfx950, wave64):
//   * A wavefront owns whole output rows; its 64 lanes split a row into
//     "units" of 64 weights that live in whole GGUF blocks:
//       Q4_K unit = (super-block, 64-weight chunk c)  : 32 B of qs + 16 B header
//       Q6_K unit = (super-block, half h, 16-run u)    : 3 x 16 B of ql/qh + scales + d
//       Q8_0 unit = a pair of 34-B blocks              : 68 B, dword aligned
//     Lane l handles units l, l+64, ... (P per lane), so each lane always
//     touches the same columns of x.
//   * The lane's columns of x are quantised once per wave to int16 (power-of-two
//     scale per 16/32-run) and split into hi/lo int8 dwords held in registers;
//     the 4/6/8-bit weight integers then contract with them by v_dot4_i32_i8.
//     Partial sums are exact integers; block scales are applied in fp32.
//   * Weight bytes are streamed once with 128-bit loads (dword-aligned windows
//     re-aligned with v_alignbyte_b32 for the 2-byte-aligned Q6_K/Q8_0 blocks).
//   * Rows are reduced across the wave with DPP + readlane in a fixed order.
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ u32x4a4 ld4(const uint8_t *p) { return *reinterpret_cast<const u32x4a4 *>(p); }
__device__ __forceinline__ u32x2a4 ld2(const uint8_t *p) { return *reinterpret_cast<const u32x2a4 *>(p); }
__device__ __forceinline__ uint32_t ld1(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

// 16 bytes starting at a (2-byte aligned, a & 3 == r) as four dwords.  Reads
// only [a - r, a + 16 + 2 - r) ⊂ [a - 2, a + 16 + 2): callers keep that range
// inside the block.
__device__ __forceinline__ void win16(const uint8_t *a, uint32_t r, uint32_t o[4]) {
  u32x4a4 v = ld4(a - r);
  uint32_t e = ld1(a + 12 + r);
  o[0] = realign(v.y, v.x, r);
  o[1] = realign(v.z, v.y, r);
  o[2] = realign(v.w, v.z, r);
  o[3] = realign(e, v.w, r);
}

// 8 bytes starting at a (a & 3 == r) as two dwords; reads [a - r, a + 8 + 2 - r).
__device__ __forceinline__ void win8(const uint8_t *a, uint32_t r, uint32_t o[2]) {
  u32x2a4 v = ld2(a - r);
  uint32_t e = ld1(a + 4 + r);
  o[0] = realign(v.y, v.x, r);
  o[1] = realign(e, v.y, r);
}

// Quantise NW*4 consecutive floats of x (16-byte aligned) into hi/lo dwords.
template <int NW>
__device__ __forceinline__ void prep_run(const float *__restrict__ xp, uint32_t *hi, uint32_t *lo, float &sx,
                                         float &xsum) {
  float v[4 * NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    float4 t = *reinterpret_cast<const float4 *>(xp + 4 * i);
    v[4 * i] = t.x;
    v[4 * i + 1] = t.y;
    v[4 * i + 2] = t.z;
    v[4 * i + 3] = t.w;
  }
  float amax = 0.0f, s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4 * NW; ++i) {
    amax = fmaxf(amax, fabsf(v[i]));
    s += v[i];
  }
  int e = x_exp(amax);
  sx = ldexpf(1.0f, e);
  xsum = s;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    int h0, l0, h1, l1, h2, l2, h3, l3;
    x_split(v[4 * i], e, h0, l0);
    x_split(v[4 * i + 1], e, h1, l1);
    x_split(v[4 * i + 2], e, h2, l2);
    x_split(v[4 * i + 3], e, h3, l3);
    hi[i] = pack4(h0, h1, h2, h3);
    lo[i] = pack4(l0, l1, l2, l3);
  }
}

// ---------------------------------------------------------------------------
// Q4_K
// ---------------------------------------------------------------------------
template <int P>
__global__ __launch_bounds__(256) void gemv_q4k_kernel(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                       const float *__restrict__ bias, float *__restrict__ y, int N,
                                                       int nb) {
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  const int nwaves = (int)((gridDim.x * blockDim.x) >> 6);
  const int U = nb * 4;
  const uint32_t c = lane & 3;
  const size_t row_bytes = (size_t)nb * kQ4KBytes;

  uint32_t xh[P][16], xl[P][16];
  float sA[P], sB[P], tA[P], tB[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    if (u < U) {
      const float *xp = x + (size_t)(u >> 2) * 256 + 64 * c;
      prep_run<8>(xp, xh[p], xl[p], sA[p], tA[p]);
      prep_run<8>(xp + 32, xh[p] + 8, xl[p] + 8, sB[p], tB[p]);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) xh[p][i] = xl[p][i] = 0u;
      sA[p] = sB[p] = tA[p] = tB[p] = 0.0f;
    }
  }

  for (int row = wave; row < N; row += nwaves) {
    const uint8_t *base = W + (size_t)row * row_bytes;
    float acc = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int u = lane + 64 * p;
      if (u < U) {
        const uint8_t *blk = base + (size_t)(u >> 2) * kQ4KBytes;
        const u32x4a4 hd = ld4(blk);
        const u32x4a4 qa = ld4(blk + 16 + 32 * c);
        const u32x4a4 qb = ld4(blk + 32 + 32 * c);
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        int ah = 0, al = 0, bh = 0, bl = 0;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          const uint32_t lo4 = q[w] & 0x0F0F0F0Fu;
          const uint32_t hi4 = (q[w] >> 4) & 0x0F0F0F0Fu;
          ah = sdot4(lo4, xh[p][w], ah);
          al = sdot4(lo4, xl[p][w], al);
          bh = sdot4(hi4, xh[p][8 + w], bh);
          bl = sdot4(hi4, xl[p][8 + w], bl);
        }
        uint32_t scA, mA, scB, mB;
        q4k_scale_min(2 * c, hd.y, hd.z, hd.w, scA, mA);
        q4k_scale_min(2 * c + 1, hd.y, hd.z, hd.w, scB, mB);
        const float d = f16_bits_hw(hd.x & 0xffffu);
        const float dmin = f16_bits_hw(hd.x >> 16);
        const float fa = (float)(ah * 256 + al);
        const float fb = (float)(bh * 256 + bl);
        acc += (d * (float)scA) * (sA[p] * fa) - (dmin * (float)mA) * tA[p];
        acc += (d * (float)scB) * (sB[p] * fb) - (dmin * (float)mB) * tB[p];
      }
    }
    const float s = wave_sum(acc);
    if (lane == 0) y[row] = s + (bias ? bias[row] : 0.0f);
  }
}

// ---------------------------------------------------------------------------
// Q6_K
// ---------------------------------------------------------------------------
template <int P>
__global__ __launch_bounds__(256) void gemv_q6k_kernel(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                       const float *__restrict__ bias, float *__restrict__ y, int N,
                                                       int nb) {
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  const int nwaves = (int)((gridDim.x * blockDim.x) >> 6);
  const int U = nb * 4;
  const uint32_t h = (lane >> 1) & 1u;
  const uint32_t u2 = lane & 1u;
  const size_t row_bytes = (size_t)nb * kQ6KBytes;

  // runs qq = 0..3: elements 128h + 32qq + 16u2 + [0, 16) of the super-block
  uint32_t xh[P][16], xl[P][16];
  float sx[P][4], xs[P][4];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    if (u < U) {
      const float *xp = x + (size_t)(u >> 2) * 256 + 128 * h + 16 * u2;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) prep_run<4>(xp + 32 * qq, xh[p] + 4 * qq, xl[p] + 4 * qq, sx[p][qq], xs[p][qq]);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) xh[p][i] = xl[p][i] = 0u;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) sx[p][qq] = xs[p][qq] = 0.0f;
    }
  }

  for (int row = wave; row < N; row += nwaves) {
    const uint8_t *base = W + (size_t)row * row_bytes;
    float acc = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int u = lane + 64 * p;
      if (u < U) {
        const uint8_t *B = base + (size_t)(u >> 2) * kQ6KBytes;
        const uint32_t r = (uint32_t)reinterpret_cast<uintptr_t>(B) & 3u;
        uint32_t L[4], Lh[4], H[4], S[2];
        win16(B + 64 * h + 16 * u2, r, L);
        win16(B + 64 * h + 32 + 16 * u2, r, Lh);
        win16(B + 128 + 32 * h + 16 * u2, r, H);
        win8(B + 192 + 8 * h, r, S);
        const float d = f16_bits_hw(*reinterpret_cast<const uint16_t *>(B + 208));
        int ah[4] = {0, 0, 0, 0}, al[4] = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t q1 = (L[w] & 0x0F0F0F0Fu) | ((H[w] << 4) & 0x30303030u);
          const uint32_t q2 = (Lh[w] & 0x0F0F0F0Fu) | ((H[w] << 2) & 0x30303030u);
          const uint32_t q3 = ((L[w] >> 4) & 0x0F0F0F0Fu) | (H[w] & 0x30303030u);
          const uint32_t q4 = ((Lh[w] >> 4) & 0x0F0F0F0Fu) | ((H[w] >> 2) & 0x30303030u);
          ah[0] = sdot4(q1, xh[p][w], ah[0]);
          al[0] = sdot4(q1, xl[p][w], al[0]);
          ah[1] = sdot4(q2, xh[p][4 + w], ah[1]);
          al[1] = sdot4(q2, xl[p][4 + w], al[1]);
          ah[2] = sdot4(q3, xh[p][8 + w], ah[2]);
          al[2] = sdot4(q3, xl[p][8 + w], al[2]);
          ah[3] = sdot4(q4, xh[p][12 + w], ah[3]);
          al[3] = sdot4(q4, xl[p][12 + w], al[3]);
        }
        const int sc0 = (int8_t)(S[0] >> (8 * u2));
        const int sc1 = (int8_t)(S[0] >> (8 * (u2 + 2)));
        const int sc2 = (int8_t)(S[1] >> (8 * u2));
        const int sc3 = (int8_t)(S[1] >> (8 * (u2 + 2)));
        const int scv[4] = {sc0, sc1, sc2, sc3};
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const float t = sx[p][qq] * (float)(ah[qq] * 256 + al[qq]) - 32.0f * xs[p][qq];
          acc += (d * (float)scv[qq]) * t;
        }
      }
    }
    const float s = wave_sum(acc);
    if (lane == 0) y[row] = s + (bias ? bias[row] : 0.0f);
  }
}

// ---------------------------------------------------------------------------
// Q8_0 (pairs of blocks: 68 B, dword aligned when the row is)
// ---------------------------------------------------------------------------
template <int P>
__global__ __launch_bounds__(256) void gemv_q8_0_kernel(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                        const float *__restrict__ bias, float *__restrict__ y, int N,
                                                        int nb) {
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  const int nwaves = (int)((gridDim.x * blockDim.x) >> 6);
  const int U = nb / 2;
  const size_t row_bytes = (size_t)nb * kQ8Bytes;

  uint32_t xh[P][16], xl[P][16];
  float s0[P], s1[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    if (u < U) {
      const float *xp = x + (size_t)u * 64;
      float t0, t1;
      prep_run<8>(xp, xh[p], xl[p], s0[p], t0);
      prep_run<8>(xp + 32, xh[p] + 8, xl[p] + 8, s1[p], t1);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) xh[p][i] = xl[p][i] = 0u;
      s0[p] = s1[p] = 0.0f;
    }
  }

  for (int row = wave; row < N; row += nwaves) {
    const uint8_t *base = W + (size_t)row * row_bytes;
    float acc = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int u = lane + 64 * p;
      if (u < U) {
        const uint8_t *pr = base + (size_t)u * (2 * kQ8Bytes);
        const u32x4a4 v0 = ld4(pr), v1 = ld4(pr + 16), v2 = ld4(pr + 32), v3 = ld4(pr + 48);
        const uint32_t v4 = ld1(pr + 64);
        const uint32_t w[17] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v2.x,
                                v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w, v4};
        int a0h = 0, a0l = 0, a1h = 0, a1l = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t q0 = realign(w[k + 1], w[k], 2u);  // block 0 quants: bytes 2..33
          const uint32_t q1 = w[9 + k];                       // block 1 quants: bytes 36..67
          a0h = sdot4(q0, xh[p][k], a0h);
          a0l = sdot4(q0, xl[p][k], a0l);
          a1h = sdot4(q1, xh[p][8 + k], a1h);
          a1l = sdot4(q1, xl[p][8 + k], a1l);
        }
        const float d0 = f16_bits_hw(w[0] & 0xffffu);
        const float d1 = f16_bits_hw(w[8] >> 16);
        acc += d0 * (s0[p] * (float)(a0h * 256 + a0l));
        acc += d1 * (s1[p] * (float)(a1h * 256 + a1l));
      }
    }
    const float s = wave_sum(acc);
    if (lane == 0) y[row] = s + (bias ? bias[row] : 0.0f);
  }
}

// ---------------------------------------------------------------------------
// General fallback (any block-aligned K, 2-byte-aligned blocks): one wave per
// row, lanes stride over elements with byte loads and fp32 FMA.  Used for
// shapes outside the fast kernels' register budget (K > 16384) and for Q8_0
// rows that are not dword aligned (an odd number of blocks per row).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float deq_elem(int type, const uint8_t *row, uint32_t k) {
  if (type == kQ8_0) {
    const uint8_t *blk = row + (size_t)(k >> 5) * kQ8Bytes;
    const float d = f16_bits_hw(*reinterpret_cast<const uint16_t *>(blk));
    return (float)(int8_t)blk[2 + (k & 31)] * d;
  } else if (type == kQ4_K) {
    const uint8_t *blk = row + (size_t)(k >> 8) * kQ4KBytes;
    const uint32_t rr = k & 255u, c = rr >> 6, hi = (rr >> 5) & 1u, l = rr & 31u;
    const uint32_t *wd = reinterpret_cast<const uint32_t *>(blk);
    uint32_t sc, m;
    q4k_scale_min(2 * c + hi, wd[1], wd[2], wd[3], sc, m);
    const float d = f16_bits_hw(wd[0] & 0xffffu), dmin = f16_bits_hw(wd[0] >> 16);
    const uint32_t q = (blk[16 + 32 * c + l] >> (4 * hi)) & 15u;
    return (d * (float)sc) * (float)q - dmin * (float)m;
  } else {
    const uint8_t *blk = row + (size_t)(k >> 8) * kQ6KBytes;
    const uint32_t rr = k & 255u, hh = rr >> 7, quarter = (rr >> 5) & 3u, l = rr & 31u;
    const uint32_t qlb = blk[64 * hh + l + ((quarter & 1u) ? 32u : 0u)];
    const uint32_t lo4 = (qlb >> ((quarter & 2u) ? 4u : 0u)) & 15u;
    const uint32_t hi2 = (blk[128 + 32 * hh + l] >> (2 * quarter)) & 3u;
    const int q = (int)(lo4 | (hi2 << 4)) - 32;
    const int sc = (int8_t)blk[192 + 8 * hh + l / 16 + 2 * quarter];
    const float d = f16_bits_hw(*reinterpret_cast<const uint16_t *>(blk + 208));
    return (d * (float)sc) * (float)q;
  }
}

__global__ __launch_bounds__(256) void gemv_generic_kernel(int type, const uint8_t *__restrict__ W,
                                                           const float *__restrict__ x,
                                                           const float *__restrict__ bias, float *__restrict__ y,
                                                           int N, int K, size_t row_bytes) {
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  const int nwaves = (int)((gridDim.x * blockDim.x) >> 6);
  for (int row = wave; row < N; row += nwaves) {
    const uint8_t *base = W + (size_t)row * row_bytes;
    float acc = 0.0f;
    for (int k = lane; k < K; k += 64) acc = fmaf(x[k], deq_elem(type, base, (uint32_t)k), acc);
    const float s = wave_sum(acc);
    if (lane == 0) y[row] = s + (bias ? bias[row] : 0.0f);
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
#define OKQ_GEMV_DISPATCH(KERNEL, P, ...)                                                        \
  switch (P) {                                                                                   \
  case 1: launch_timed(KERNEL<1>, __VA_ARGS__); break;                                     \
  case 2: launch_timed(KERNEL<2>, __VA_ARGS__); break;                                     \
  case 3: launch_timed(KERNEL<3>, __VA_ARGS__); break;                                     \
  default: launch_timed(KERNEL<4>, __VA_ARGS__); break;                                    \
  }

hipError_t launch_gemv(int type, const float *x, int64_t K, const void *w, int64_t N, const float *bias, float *y,
                       int cu_count, hipStream_t s) {
  const uint8_t *W = static_cast<const uint8_t *>(w);
  const int waves_per_cu = 16;
  int64_t max_blocks = (int64_t)cu_count * (waves_per_cu / 4);
  int64_t blocks = (N + 3) / 4;
  if (blocks > max_blocks) blocks = max_blocks;
  if (blocks < 1) blocks = 1;
  const dim3 grid((unsigned)blocks), block(256);
  const int n = (int)N;
  const uintptr_t wa = reinterpret_cast<uintptr_t>(W);
  if (type == kQ4_K) {
    const int nb = (int)(K / 256);
    const int P = (nb * 4 + 63) / 64;
    if (P <= 4 && (wa & 15u) == 0) {
      OKQ_GEMV_DISPATCH(gemv_q4k_kernel, P, grid, block, 0, s, W, x, bias, y, n, nb);
      return hipGetLastError();
    }
  } else if (type == kQ6_K) {
    const int nb = (int)(K / 256);
    const int P = (nb * 4 + 63) / 64;
    if (P <= 4 && (wa & 3u) == 0) {
      OKQ_GEMV_DISPATCH(gemv_q6k_kernel, P, grid, block, 0, s, W, x, bias, y, n, nb);
      return hipGetLastError();
    }
  } else if (type == kQ8_0) {
    const int nb = (int)(K / 32);
    const int P = (nb / 2 + 63) / 64;
    if ((nb & 1) == 0 && P <= 4 && (wa & 3u) == 0) {
      OKQ_GEMV_DISPATCH(gemv_q8_0_kernel, P, grid, block, 0, s, W, x, bias, y, n, nb);
      return hipGetLastError();
    }
  } else {
    return hipErrorInvalidValue;
  }
  const size_t row_bytes =
      (size_t)(type == kQ8_0 ? (K / 32) * kQ8Bytes : (K / 256) * (type == kQ4_K ? kQ4KBytes : kQ6KBytes));
  launch_timed(gemv_generic_kernel, grid, block, 0, s, type, W, x, bias, y, n, (int)K, row_bytes);
  return hipGetLastError();
}

}  // namespace okq
