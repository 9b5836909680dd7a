// okq_prep.hip -- bit-exact dequantize, quantize, seeded generator and
// f32->bf16 kernels.  Compiled with -ffp-contract=off: every product and
// difference is rounded on its own, in the order the GGUF spec writes it, so
// results equal the CPU oracle bit for bit.
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

// ---------------------------------------------------------------------------
// dequantize: one thread per output element (coalesced f32 stores; the block
// bytes a wave touches are shared through the cache).
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
  return (uint32_t)(*reinterpret_cast<const uint16_t *>(p));  // blocks are 2-byte aligned
}

// Element i of a run of blocks starting at `base`, in the order and rounding
// of the GGUF spec (one product or difference rounded at a time).
__device__ __forceinline__ float dq_q8_0(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 5) * kQ8Bytes;
  float d = f16_bits_exact(ld_u16(blk));
  float q = (float)(int8_t)blk[2 + (i & 31)];
  return __fmul_rn(q, d);
}

__device__ __forceinline__ float dq_q4_k(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 8) * kQ4KBytes;
  uint32_t r = (uint32_t)(i & 255);
  uint32_t c = r >> 6, hi = (r >> 5) & 1u, l = r & 31u;
  uint32_t j = 2 * c + hi;
  const uint32_t *w = reinterpret_cast<const uint32_t *>(blk);  // 144-byte blocks are 16-byte aligned
  uint32_t sc, m;
  q4k_scale_min(j, w[1], w[2], w[3], sc, m);
  float d = f16_bits_exact(w[0] & 0xffffu);
  float dmin = f16_bits_exact(w[0] >> 16);
  uint32_t q = (blk[16 + 32 * c + l] >> (4 * hi)) & 15u;
  float ds = __fmul_rn(d, (float)sc);
  float dm = __fmul_rn(dmin, (float)m);
  return __fsub_rn(__fmul_rn(ds, (float)q), dm);
}

__device__ __forceinline__ float dq_q6_k(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 8) * kQ6KBytes;
  uint32_t r = (uint32_t)(i & 255);
  uint32_t h = r >> 7, quarter = (r >> 5) & 3u, l = r & 31u;
  uint32_t qlb = blk[64 * h + l + ((quarter & 1u) ? 32u : 0u)];
  uint32_t lo4 = (qlb >> ((quarter & 2u) ? 4u : 0u)) & 15u;
  uint32_t hi2 = (blk[128 + 32 * h + l] >> (2 * quarter)) & 3u;
  int q = (int)(lo4 | (hi2 << 4)) - 32;
  int sc = (int8_t)blk[192 + 8 * h + l / 16 + 2 * quarter];
  float d = f16_bits_exact(ld_u16(blk + 208));
  return __fmul_rn(__fmul_rn(d, (float)sc), (float)q);
}

// ---- formats served by dequantize / row gather only ----------------------
// Byte loads throughout: these blocks are only 2-byte aligned.

// Fifth bit of element e (0..31) of a Q5_0 / Q5_1 block: bit e of the
// little-endian 32-bit word qh.
__device__ __forceinline__ uint32_t q5_bit(const uint8_t *qh, uint32_t e) { return (qh[e >> 3] >> (e & 7u)) & 1u; }

// The 4-bit code of element e of a 16-byte qs run: low nibbles hold
// elements 0..15, high nibbles 16..31.
__device__ __forceinline__ uint32_t nib32(const uint8_t *qs, uint32_t e) { return (qs[e & 15u] >> ((e >> 4) * 4)) & 15u; }

__device__ __forceinline__ float dq_q4_0(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 5) * kQ40Bytes;
  const uint32_t e = (uint32_t)(i & 31);
  const float d = f16_bits_exact(ld_u16(blk));
  return __fmul_rn((float)((int)nib32(blk + 2, e) - 8), d);
}

__device__ __forceinline__ float dq_q4_1(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 5) * kQ41Bytes;
  const uint32_t e = (uint32_t)(i & 31);
  const float d = f16_bits_exact(ld_u16(blk)), m = f16_bits_exact(ld_u16(blk + 2));
  return __fadd_rn(__fmul_rn((float)nib32(blk + 4, e), d), m);
}

__device__ __forceinline__ float dq_q5_0(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 5) * kQ50Bytes;
  const uint32_t e = (uint32_t)(i & 31);
  const float d = f16_bits_exact(ld_u16(blk));
  const int q = (int)(nib32(blk + 6, e) | (q5_bit(blk + 2, e) << 4)) - 16;
  return __fmul_rn((float)q, d);
}

__device__ __forceinline__ float dq_q5_1(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 5) * kQ51Bytes;
  const uint32_t e = (uint32_t)(i & 31);
  const float d = f16_bits_exact(ld_u16(blk)), m = f16_bits_exact(ld_u16(blk + 2));
  const uint32_t q = nib32(blk + 8, e) | (q5_bit(blk + 4, e) << 4);
  return __fadd_rn(__fmul_rn((float)q, d), m);
}

// Q2_K element r = 128h + 32j + s: 2-bit q = (qs[32h+s] >> 2j) & 3 and scale
// byte scales[r/16] (low nibble scale, high nibble min).
__device__ __forceinline__ float dq_q2_k(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 8) * kQ2KBytes;
  const uint32_t r = (uint32_t)(i & 255), h = r >> 7, j = (r >> 5) & 3u, s = r & 31u;
  const uint32_t sc = blk[r >> 4];
  const uint32_t q = (blk[16 + 32 * h + s] >> (2 * j)) & 3u;
  const float d = f16_bits_exact(ld_u16(blk + 80)), dmin = f16_bits_exact(ld_u16(blk + 82));
  const float dl = __fmul_rn(d, (float)(sc & 15u)), ml = __fmul_rn(dmin, (float)(sc >> 4));
  return __fsub_rn(__fmul_rn(dl, (float)q), ml);
}

// Q3_K element r = 128h + 32j + s: low two bits (qs[32h+s] >> 2j) & 3, minus 4
// when bit 4h+j of hmask[s] is clear; 6-bit scale r/16 unpacked from the 12
// packed bytes (low nibble from byte is or is-8, top two bits from byte
// 8 + is%4 at bit 2*(is/4)), biased by 32.
__device__ __forceinline__ float dq_q3_k(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 8) * kQ3KBytes;
  const uint32_t r = (uint32_t)(i & 255), h = r >> 7, j = (r >> 5) & 3u, s = r & 31u, is = r >> 4;
  const uint8_t *sb = blk + 96;
  const uint32_t lo = is < 8 ? (sb[is] & 15u) : (sb[is - 8] >> 4);
  const uint32_t hi = (sb[8 + (is & 3u)] >> (2 * (is >> 2))) & 3u;
  const int scale = (int)(lo | (hi << 4)) - 32;
  const int q = (int)((blk[32 + 32 * h + s] >> (2 * j)) & 3u) - (((blk[s] >> (4 * h + j)) & 1u) ? 0 : 4);
  const float d = f16_bits_exact(ld_u16(blk + 108));
  return __fmul_rn(__fmul_rn(d, (float)scale), (float)q);
}

// Q5_K element r = 64c + 32hi + l: the Q4_K nibble plus 16 when bit 2c+hi of
// qh[l] is set; scales and mins as Q4_K.
__device__ __forceinline__ float dq_q5_k(const uint8_t *base, int64_t i) {
  const uint8_t *blk = base + (i >> 8) * kQ5KBytes;
  const uint32_t r = (uint32_t)(i & 255), c = r >> 6, hi = (r >> 5) & 1u, l = r & 31u;
  const uint8_t *sb = blk + 4;
  const uint32_t s0 = sb[0] | (sb[1] << 8) | (sb[2] << 16) | ((uint32_t)sb[3] << 24);
  const uint32_t s1 = sb[4] | (sb[5] << 8) | (sb[6] << 16) | ((uint32_t)sb[7] << 24);
  const uint32_t s2 = sb[8] | (sb[9] << 8) | (sb[10] << 16) | ((uint32_t)sb[11] << 24);
  uint32_t sc, m;
  q4k_scale_min(2 * c + hi, s0, s1, s2, sc, m);
  const uint32_t q = ((blk[48 + 32 * c + l] >> (4 * hi)) & 15u) + (((blk[16 + l] >> (2 * c + hi)) & 1u) << 4);
  const float d = f16_bits_exact(ld_u16(blk)), dmin = f16_bits_exact(ld_u16(blk + 2));
  const float ds = __fmul_rn(d, (float)sc), dm = __fmul_rn(dmin, (float)m);
  return __fsub_rn(__fmul_rn(ds, (float)q), dm);
}

template <int kType>
__device__ __forceinline__ float dq_elem(const uint8_t *base, int64_t i) {
  if constexpr (kType == kQ8_0) return dq_q8_0(base, i);
  else if constexpr (kType == kQ4_K) return dq_q4_k(base, i);
  else if constexpr (kType == kQ6_K) return dq_q6_k(base, i);
  else if constexpr (kType == kQ4_0) return dq_q4_0(base, i);
  else if constexpr (kType == kQ4_1) return dq_q4_1(base, i);
  else if constexpr (kType == kQ5_0) return dq_q5_0(base, i);
  else if constexpr (kType == kQ5_1) return dq_q5_1(base, i);
  else if constexpr (kType == kQ2_K) return dq_q2_k(base, i);
  else if constexpr (kType == kQ3_K) return dq_q3_k(base, i);
  else return dq_q5_k(base, i);
}

template <int kType>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ src, int64_t n,
                                                     float *__restrict__ dst) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dst[i] = dq_elem<kType>(src, i);
}

// Quantized row gather (token embedding lookup): output row j is weight row
// ids[blockIdx.y] dequantized.  The ids travel in the kernel arguments, so a
// launch needs no device staging; rows are validated on the host first.
template <int kType>
__global__ __launch_bounds__(256) void get_rows_kernel(const uint8_t *__restrict__ W, int64_t row_bytes, int64_t ne0,
                                                       GatherIds ids, float *__restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= ne0) return;
  const uint8_t *row = W + (int64_t)ids.id[blockIdx.y] * row_bytes;
  out[(int64_t)blockIdx.y * ne0 + e] = dq_elem<kType>(row, e);
}

// ---------------------------------------------------------------------------
// Quantizers: one thread per block.  Step for step the algorithm of the CPU
// oracle (comparisons written as a < b ? a : b, correctly rounded division,
// round-to-nearest-even), so the bytes are identical.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float minf_(float a, float b) { return a < b ? a : b; }
__device__ __forceinline__ float maxf_(float a, float b) { return a > b ? a : b; }
__device__ __forceinline__ int clampi_(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, round to nearest even
}
__device__ __forceinline__ void st_u16(uint8_t *p, uint32_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
}

__global__ __launch_bounds__(64) void quantize_q8_0_kernel(const float *__restrict__ x, int64_t nblocks,
                                                            uint8_t *__restrict__ dst) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const float *xb = x + b * 32;
  uint8_t *blk = dst + b * kQ8Bytes;
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) amax = maxf_(amax, fabsf(xb[j]));
  float d = __fdiv_rn(amax, 127.0f);
  float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
  st_u16(blk, f32_to_f16_bits(d));
  for (int j = 0; j < 32; ++j) {
    int q = (int)__builtin_rintf(__fmul_rn(xb[j], id));
    blk[2 + j] = (uint8_t)(int8_t)clampi_(q, -127, 127);
  }
}

// Q4_K and Q5_K (kQ5): per 32-sub-block mn = min(0, min x), mx = max x,
// scale = (mx - mn) / L (L = 15 or 31 levels), mmin = -mn; d = max scale /
// 63, dmin = max mmin / 63 (fp16); 6-bit ls, lm = rint(63 * v / max);
// q = clamp(rint((x + dmin16 * lm) / (d16 * ls)), 0, L).  Q5_K keeps the
// low four bits in qs and bit 4 of element l of chunk c in bit 2c (low
// nibbles) or 2c + 1 (high nibbles) of qh[l].
template <bool kQ5>
__device__ __forceinline__ void quantize_q45_k(const float *__restrict__ xb, uint8_t *__restrict__ blk) {
  constexpr float kLevels = kQ5 ? 31.0f : 15.0f;
  constexpr int kMaxQ = kQ5 ? 31 : 15;
  float scale[8], mmin[8];
  float max_scale = 0.0f, max_min = 0.0f;
  for (int s = 0; s < 8; ++s) {
    float mn = xb[32 * s], mx = xb[32 * s];
    for (int j = 1; j < 32; ++j) {
      mn = minf_(mn, xb[32 * s + j]);
      mx = maxf_(mx, xb[32 * s + j]);
    }
    mn = minf_(mn, 0.0f);
    scale[s] = __fdiv_rn(__fsub_rn(mx, mn), kLevels);
    mmin[s] = -mn;
    max_scale = maxf_(max_scale, scale[s]);
    max_min = maxf_(max_min, mmin[s]);
  }
  float inv_scale = max_scale > 0.0f ? __fdiv_rn(63.0f, max_scale) : 0.0f;
  float inv_min = max_min > 0.0f ? __fdiv_rn(63.0f, max_min) : 0.0f;
  uint32_t ls[8], lm[8];
  for (int s = 0; s < 8; ++s) {
    ls[s] = (uint32_t)clampi_((int)__builtin_rintf(__fmul_rn(inv_scale, scale[s])), 0, 63);
    lm[s] = (uint32_t)clampi_((int)__builtin_rintf(__fmul_rn(inv_min, mmin[s])), 0, 63);
  }
  uint32_t dh = f32_to_f16_bits(__fdiv_rn(max_scale, 63.0f));
  uint32_t dminh = f32_to_f16_bits(__fdiv_rn(max_min, 63.0f));
  st_u16(blk, dh);
  st_u16(blk + 2, dminh);
  uint32_t sc[12];
  for (int j = 0; j < 4; ++j) {
    sc[j] = ls[j] | ((ls[j + 4] >> 4) << 6);
    sc[j + 4] = lm[j] | ((lm[j + 4] >> 4) << 6);
    sc[j + 8] = (ls[j + 4] & 15u) | ((lm[j + 4] & 15u) << 4);
  }
  for (int j = 0; j < 12; ++j) blk[4 + j] = (uint8_t)sc[j];
  float d16 = f16_bits_exact(dh), dmin16 = f16_bits_exact(dminh);
  uint8_t *qh = blk + 16;
  uint8_t *qs = blk + (kQ5 ? 48 : 16);
  uint32_t hbits[32];
  for (int l = 0; l < 32; ++l) hbits[l] = 0u;
  for (int c = 0; c < 4; ++c) {
    float de0 = __fmul_rn(d16, (float)ls[2 * c]), me0 = __fmul_rn(dmin16, (float)lm[2 * c]);
    float de1 = __fmul_rn(d16, (float)ls[2 * c + 1]), me1 = __fmul_rn(dmin16, (float)lm[2 * c + 1]);
    for (int l = 0; l < 32; ++l) {
      int q0 = 0, q1 = 0;
      if (de0 != 0.0f)
        q0 = clampi_((int)__builtin_rintf(__fdiv_rn(__fadd_rn(xb[64 * c + l], me0), de0)), 0, kMaxQ);
      if (de1 != 0.0f)
        q1 = clampi_((int)__builtin_rintf(__fdiv_rn(__fadd_rn(xb[64 * c + 32 + l], me1), de1)), 0, kMaxQ);
      qs[32 * c + l] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
      if (kQ5) hbits[l] |= ((uint32_t)(q0 >> 4) << (2 * c)) | ((uint32_t)(q1 >> 4) << (2 * c + 1));
    }
  }
  if (kQ5)
    for (int l = 0; l < 32; ++l) qh[l] = (uint8_t)hbits[l];
}

__global__ __launch_bounds__(64) void quantize_q4_k_kernel(const float *__restrict__ x, int64_t nblocks,
                                                            uint8_t *__restrict__ dst) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  quantize_q45_k<false>(x + b * 256, dst + b * kQ4KBytes);
}

__global__ __launch_bounds__(64) void quantize_q5_k_kernel(const float *__restrict__ x, int64_t nblocks,
                                                            uint8_t *__restrict__ dst) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  quantize_q45_k<true>(x + b * 256, dst + b * kQ5KBytes);
}

__global__ __launch_bounds__(64) void quantize_q6_k_kernel(const float *__restrict__ x, int64_t nblocks,
                                                            uint8_t *__restrict__ dst) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const float *xb = x + b * 256;
  uint8_t *blk = dst + b * kQ6KBytes;
  float scale[16];
  float max_scale = 0.0f, max_abs_scale = 0.0f;
  for (int s = 0; s < 16; ++s) {
    float mx = 0.0f, amax = 0.0f;
    for (int j = 0; j < 16; ++j) {
      float v = xb[16 * s + j];
      float a = fabsf(v);
      if (a > amax) {
        amax = a;
        mx = v;
      }
    }
    scale[s] = __fdiv_rn(-mx, 32.0f);
    float as = fabsf(scale[s]);
    if (as > max_abs_scale) {
      max_abs_scale = as;
      max_scale = scale[s];
    }
  }
  float iscale = max_scale != 0.0f ? __fdiv_rn(-128.0f, max_scale) : 0.0f;
  float d = iscale != 0.0f ? __fdiv_rn(1.0f, iscale) : 0.0f;
  uint32_t dh = f32_to_f16_bits(d);
  float d16 = f16_bits_exact(dh);
  int scs[16];
  for (int s = 0; s < 16; ++s) scs[s] = clampi_((int)__builtin_rintf(__fmul_rn(iscale, scale[s])), -128, 127);
  for (int h = 0; h < 2; ++h) {
    for (int l = 0; l < 32; ++l) {
      uint32_t L[4];
      for (int qq = 0; qq < 4; ++qq) {
        int e = 128 * h + 32 * qq + l;
        int s = e >> 4;
        float de = __fmul_rn(d16, (float)scs[s]);
        int q = 0;
        if (de != 0.0f) q = clampi_((int)__builtin_rintf(__fdiv_rn(xb[e], de)), -32, 31);
        L[qq] = (uint32_t)(q + 32);
      }
      blk[64 * h + l] = (uint8_t)((L[0] & 15u) | ((L[2] & 15u) << 4));
      blk[64 * h + 32 + l] = (uint8_t)((L[1] & 15u) | ((L[3] & 15u) << 4));
      blk[128 + 32 * h + l] = (uint8_t)((L[0] >> 4) | ((L[1] >> 4) << 2) | ((L[2] >> 4) << 4) | ((L[3] >> 4) << 6));
    }
  }
  for (int s = 0; s < 16; ++s) blk[192 + s] = (uint8_t)(int8_t)scs[s];
  st_u16(blk + 208, dh);
}

// ---------------------------------------------------------------------------
// Seeded N(0, sigma) and f32 -> bf16
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_normal_kernel(uint64_t key, int64_t offset, int64_t n, float sigma,
                                                          float *__restrict__ dst) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint64_t gi = (uint64_t)(offset + i);
  int32_t s = 0;
  for (int j = 0; j < 6; ++j) {
    uint64_t z = mix64(key + (gi * 6u + (uint64_t)j + 1u) * 0x9E3779B97F4A7C15ull);
    s += (int32_t)(z & 0xffffffu) + (int32_t)((z >> 32) & 0xffffffu);
  }
  s -= 6 * 0xffffff;
  float u = __fmul_rn((float)s, 5.9604644775390625e-08f);
  dst[i] = __fmul_rn(u, sigma);
}

__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float *__restrict__ src, int64_t n,
                                                          uint16_t *__restrict__ dst) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t u = as_u32(src[i]);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    dst[i] = (uint16_t)((u >> 16) | 0x40u);
    return;
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  dst[i] = (uint16_t)(u >> 16);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

static inline unsigned grid_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

hipError_t launch_dequantize(int type, const void *src, int64_t n, float *dst, hipStream_t s) {
  const uint8_t *p = static_cast<const uint8_t *>(src);
  const dim3 grid(grid_for(n, 256));
  switch (type) {
#define OKQ_DQ_CASE(T) \
  case T: launch_timed(dequant_kernel<T>, grid, dim3(256), 0, s, p, n, dst); break;
    OKQ_DQ_CASE(kQ8_0) OKQ_DQ_CASE(kQ4_K) OKQ_DQ_CASE(kQ6_K) OKQ_DQ_CASE(kQ4_0) OKQ_DQ_CASE(kQ4_1)
    OKQ_DQ_CASE(kQ5_0) OKQ_DQ_CASE(kQ5_1) OKQ_DQ_CASE(kQ2_K) OKQ_DQ_CASE(kQ3_K) OKQ_DQ_CASE(kQ5_K)
#undef OKQ_DQ_CASE
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_get_rows(int type, const void *w, int64_t row_bytes, int64_t ne0, const uint32_t *ids, int64_t n,
                           float *out, hipStream_t s) {
  const uint8_t *p = static_cast<const uint8_t *>(w);
  for (int64_t j0 = 0; j0 < n; j0 += kGatherMaxIds) {
    const int64_t cnt = n - j0 < kGatherMaxIds ? n - j0 : kGatherMaxIds;
    GatherIds g;
    for (int64_t j = 0; j < cnt; ++j) g.id[j] = ids[j0 + j];
    const dim3 grid(grid_for(ne0, 256), (unsigned)cnt);
    float *o = out + j0 * ne0;
    switch (type) {
#define OKQ_GR_CASE(T) \
  case T: hipLaunchKernelGGL(get_rows_kernel<T>, grid, dim3(256), 0, s, p, row_bytes, ne0, g, o); break;
      OKQ_GR_CASE(kQ8_0) OKQ_GR_CASE(kQ4_K) OKQ_GR_CASE(kQ6_K) OKQ_GR_CASE(kQ4_0) OKQ_GR_CASE(kQ4_1)
      OKQ_GR_CASE(kQ5_0) OKQ_GR_CASE(kQ5_1) OKQ_GR_CASE(kQ2_K) OKQ_GR_CASE(kQ3_K) OKQ_GR_CASE(kQ5_K)
#undef OKQ_GR_CASE
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_quantize(int type, const float *src, int64_t n, void *dst, hipStream_t s) {
  uint8_t *p = static_cast<uint8_t *>(dst);
  switch (type) {
  case kQ8_0: {
    int64_t nb = n / 32;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3(grid_for(nb, 64)), dim3(64), 0, s, src, nb, p);
    break;
  }
  case kQ4_K: {
    int64_t nb = n / 256;
    hipLaunchKernelGGL(quantize_q4_k_kernel, dim3(grid_for(nb, 64)), dim3(64), 0, s, src, nb, p);
    break;
  }
  case kQ5_K: {
    int64_t nb = n / 256;
    hipLaunchKernelGGL(quantize_q5_k_kernel, dim3(grid_for(nb, 64)), dim3(64), 0, s, src, nb, p);
    break;
  }
  case kQ6_K: {
    int64_t nb = n / 256;
    hipLaunchKernelGGL(quantize_q6_k_kernel, dim3(grid_for(nb, 64)), dim3(64), 0, s, src, nb, p);
    break;
  }
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fill_normal(uint64_t seed, int64_t offset, int64_t n, float sigma, float *dst, hipStream_t s) {
  uint64_t key = seed;
  key = (key ^ (key >> 30)) * 0xBF58476D1CE4E5B9ull;
  key = (key ^ (key >> 27)) * 0x94D049BB133111EBull;
  key = key ^ (key >> 31);
  hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, key, offset, n, sigma, dst);
  return hipGetLastError();
}

// bf16 -> f32 is exact: the bf16 bits are the high half of the f32
// (crates/loader/src/safetensors_values.rs:115-123).
__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t *__restrict__ src, int64_t n,
                                                          float *__restrict__ dst) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dst[i] = as_f32((uint32_t)src[i] << 16);
}

hipError_t launch_bf16_to_f32(const uint16_t *src, int64_t n, float *dst, hipStream_t s) {
  hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, src, n, dst);
  return hipGetLastError();
}

hipError_t launch_f32_to_bf16(const float *src, int64_t n, uint16_t *dst, hipStream_t s) {
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, src, n, dst);
  return hipGetLastError();
}

}  // namespace okq
