// okq_device.h -- device-side helpers shared by the gfx950 kernels.
//
// GGUF block layouts (public GGUF spec; the reference stops at the type tag,
// crates/loader/src/gguf_inspect.rs:170-219):
//   Q8_0  34 B / 32 weights : f16 d | i8 qs[32]
//   Q4_K 144 B / 256 weights: f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
//   Q6_K 210 B / 256 weights: u8 ql[128] | u8 qh[64] | i8 scales[16] | f16 d
// and, for dequantize / row gather only:
//   Q4_0  18 B / 32 : f16 d | u8 qs[16]
//   Q4_1  20 B / 32 : f16 d | f16 m | u8 qs[16]
//   Q5_0  22 B / 32 : f16 d | u8 qh[4] | u8 qs[16]
//   Q5_1  24 B / 32 : f16 d | f16 m | u8 qh[4] | u8 qs[16]
//   Q2_K  84 B / 256: u8 scales[16] | u8 qs[64] | f16 d | f16 dmin
//   Q3_K 110 B / 256: u8 hmask[32] | u8 qs[64] | u8 scales[12] | f16 d
//   Q5_K 176 B / 256: f16 d | f16 dmin | u8 scales[12] | u8 qh[32] | u8 qs[128]
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace okq {

constexpr int kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14;
constexpr int kQ8Bytes = 34, kQ4KBytes = 144, kQ6KBytes = 210;
// Q5_K (linear kernels too) and the formats served by dequantize / row
// gather only (gguf_inspect.rs:170-206 ids).
constexpr int kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ2_K = 10, kQ3_K = 11, kQ5_K = 13;
constexpr int kQ40Bytes = 18, kQ41Bytes = 20, kQ50Bytes = 22, kQ51Bytes = 24, kQ2KBytes = 84, kQ3KBytes = 110,
              kQ5KBytes = 176;
// Bytes per 256 weights of a row in a linear-kernel format.
__host__ __device__ constexpr int sb_bytes_of(int type) {
  return type == kQ6_K ? kQ6KBytes : type == kQ8_0 ? 8 * kQ8Bytes : type == kQ5_K ? kQ5KBytes : kQ4KBytes;
}

__device__ __forceinline__ float as_f32(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t as_u32(float f) { return __float_as_uint(f); }

// Exact binary16 -> binary32 decode written with integer ops, matching
// f16_bits_to_f32 (crates/loader/src/safetensors_values.rs:155-183) bit for
// bit, NaN payloads included.  Subnormals: frac * 2^-24 is exact in f32.
__device__ __forceinline__ float f16_bits_exact(uint32_t h) {
  uint32_t sign = (h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t frac = h & 0x3ffu;
  if (exp == 0x1f) return as_f32(sign | 0x7f800000u | (frac << 13));
  if (exp != 0) return as_f32(sign | ((exp + 112u) << 23) | (frac << 13));
  float v = __fmul_rn((float)frac, 5.9604644775390625e-08f);  // 2^-24
  return as_f32(as_u32(v) | sign);
}

// Pins a kernel argument in scalar registers at this point.  Arguments pinned
// at kernel entry are fetched in one batch of scalar loads; otherwise the
// compiler fetches each on first use, which after a branch or behind a
// computed index (a select over an argument array) becomes a chain of
// dependent round trips to the argument segment before the first load.
// The value is also marked wave-uniform (readfirstlane), so that selects over
// pinned arguments stay scalar selects rather than a lookup table in private
// memory.
template <class T>
__device__ __forceinline__ T sarg(T v) {
  asm volatile("" : "+s"(v));
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
  } else {
    static_assert(sizeof(T) == 8, "32- or 64-bit arguments");
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}

// Hardware conversion for the hot loops (exact for every non-NaN input).
__device__ __forceinline__ float f16_bits_hw(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

// Realign a window of bytes that starts r (0 or 2) bytes into dword w0:
// returns bytes [r, r+4) of (w1:w0).
__device__ __forceinline__ uint32_t realign(uint32_t w1, uint32_t w0, uint32_t r) {
  return __builtin_amdgcn_alignbyte(w1, w0, r);
}

// Signed 4 x int8 dot product accumulated into c (v_dot4_i32_i8).  The
// first product of a chain (c a constant 0) is written with clamp set: the
// compiler then keeps the three-operand form with an inline zero, where the
// accumulating two-operand form (v_dot4c) needs a move of 0 first.  Four
// int8 x int8 products cannot reach the int32 clamp, so the value is the same.
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  if (__builtin_constant_p(c) && c == 0) return __builtin_amdgcn_sdot4((int)a, (int)b, 0, true);
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// A lane's DPP neighbour under a full-row control: a quad_perm (0x00-0xFF),
// row_mirror (0x140) or row_half_mirror (0x141).  Every lane then reads a
// lane of its own 16-lane row, so neither the old value nor bound_ctrl takes
// effect and the result is a plain DPP move's.  Written as an update with
// bound_ctrl set, the compiler folds the move into the add, max or select
// that consumes it (v_add_f32_dpp, v_max_u32_dpp): one instruction instead
// of a v_mov_b32_dpp and the operation.
template <int kCtl>
__device__ __forceinline__ uint32_t dpp_row_u(uint32_t v) {
  static_assert(kCtl <= 0xFF || kCtl == 0x140 || kCtl == 0x141, "full-row DPP controls only");
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtl, 0xf, 0xf, true);
}
template <int kCtl>
__device__ __forceinline__ float dpp_row_f(float v) {
  return as_f32(dpp_row_u<kCtl>(as_u32(v)));
}

// Wave-wide sum (64 lanes) with a fixed order: DPP within rows of 16, then
// the four row sums combined with readlane.  Result is uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_row_f<0xB1>(v);   // quad_perm 1,0,3,2
  v += dpp_row_f<0x4E>(v);   // quad_perm 2,3,0,1
  v += dpp_row_f<0x141>(v);  // row_half_mirror
  v += dpp_row_f<0x140>(v);  // row_mirror
  float r0 = as_f32((uint32_t)__builtin_amdgcn_readlane((int)as_u32(v), 0));
  float r1 = as_f32((uint32_t)__builtin_amdgcn_readlane((int)as_u32(v), 16));
  float r2 = as_f32((uint32_t)__builtin_amdgcn_readlane((int)as_u32(v), 32));
  float r3 = as_f32((uint32_t)__builtin_amdgcn_readlane((int)as_u32(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Activation quantisation for the integer dot path.  A run of floats is
// scaled by a power of two 2^-e chosen so that max|x| * 2^-e <= 0.99 * 2^23,
// rounded to an integer q and split into three signed int8 limbs
// q = (hi * 256 + mi) * 256 + lo, each limb in [-128, 127] (lo = ((q + 128)
// mod 256) - 128, and the same on (q - lo) / 256).  hi stays <= 127 only
// while q <= 0x7F7F7F, so run maxima whose mantissa f exceeds 0.99 take the
// next exponent (a bf16 maximum with f = 255/256 would otherwise reach
// hi = 128).  The weights' small integers contract with every
// limb exactly through v_dot4_i32_i8.  The scaling is exact (v_ldexp_f32); the
// only approximation is the rounding of q, |error| <= 2^e / 2 <= max|x| *
// 2^-23, so one outlier channel a thousand times its run's other values
// leaves those values ~2^-13 relative precision (two limbs, 2^-15 of the
// maximum, left them ~2^-5).
__device__ __forceinline__ int x_exp(float amax) {
  int E = __builtin_amdgcn_frexp_expf(amax);    // amax = f * 2^E, f in [0.5, 1)
  float f = __builtin_amdgcn_frexp_mantf(amax);
  return (f > 0.99f) ? E - 22 : E - 23;
}

// q + 0x808080: for |q| < 2^23 the three low bytes are the limbs plus 128
// (q + 0x808080 = sum_j (limb_j + 128) 256^j with every limb_j + 128 in
// [0, 255]), so the limbs are those bytes XOR 0x80 read as int8.
__device__ __forceinline__ uint32_t x_digits(float v, int e) {
  return (uint32_t)((int)__builtin_rintf(ldexpf(v, -e)) + 0x808080);
}

// Four values' digit words -> the lo, mi and hi limb dwords (byte i = value
// i's limb): a byte transpose with v_perm_b32, then the XOR that turns each
// biased digit into its signed limb.
__device__ __forceinline__ void limbs4(uint32_t u0, uint32_t u1, uint32_t u2, uint32_t u3, uint32_t &hi,
                                       uint32_t &mi, uint32_t &lo) {
  const uint32_t a = __builtin_amdgcn_perm(u1, u0, 0x05010400u);  // u0.b0 u1.b0 u0.b1 u1.b1
  const uint32_t b = __builtin_amdgcn_perm(u3, u2, 0x05010400u);  // u2.b0 u3.b0 u2.b1 u3.b1
  const uint32_t c = __builtin_amdgcn_perm(u1, u0, 0x0C0C0602u);  // u0.b2 u1.b2 0 0
  const uint32_t d = __builtin_amdgcn_perm(u3, u2, 0x0C0C0602u);  // u2.b2 u3.b2 0 0
  lo = __builtin_amdgcn_perm(b, a, 0x05040100u) ^ 0x80808080u;
  mi = __builtin_amdgcn_perm(b, a, 0x07060302u) ^ 0x80808080u;
  hi = __builtin_amdgcn_perm(d, c, 0x05040100u) ^ 0x80808080u;
}

// Run sum of the three limb dot products (each an exact int32), in units of
// the run scale 2^e: ((h * 256 + m) * 256 + l) with h * 256 + m formed in
// int32 (|.| < 2^28 for the formats' runs), converted to f32 (exact below
// 2^24, the Q4_K case) and one fused multiply-add, so at most two roundings
// of 2^-24.  Without the low limb (l = 0) the value is exactly
// (float)(h * 256 + m) * 256: hi and mi alone are q rounded to the nearest
// multiple of 256, the 16-bit quantisation of the run (|error| <= max|x| *
// 2^-15).
__device__ __forceinline__ float limb_sum(int h, int m, int l) {
  return __builtin_fmaf((float)(h * 256 + m), 256.0f, (float)l);
}

// Q4_K 6-bit (scale, min) of sub-block j from the packed scale dwords
// s0 = bytes 0..3, s1 = bytes 4..7, s2 = bytes 8..11 (GGUF spec).
__device__ __forceinline__ void q4k_scale_min(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &sc,
                                              uint32_t &m) {
  if (j < 4) {
    sc = (s0 >> (8 * j)) & 63u;
    m = (s1 >> (8 * j)) & 63u;
  } else {
    uint32_t jj = j - 4;
    sc = ((s2 >> (8 * jj)) & 15u) | (((s0 >> (8 * jj + 6)) & 3u) << 4);
    m = ((s2 >> (8 * jj + 4)) & 15u) | (((s1 >> (8 * jj + 6)) & 3u) << 4);
  }
}

// Q4_K (scale, min) of sub-block j (any lane-dependent j < 8) without
// branches: for j < 4 both are 6-bit fields of bytes 0-7; for j >= 4 a 4-bit
// field of bytes 8-11 plus two high bits from bytes 0-7 (GGUF layout).
__device__ __forceinline__ void q4k_scale_min_sel(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &sc,
                                                  uint32_t &m) {
  const bool lowj = j < 4;
  const uint32_t jj = j & 3u;
  const uint32_t width = lowj ? 6u : 4u, himask = lowj ? 0u : 0x30u, mo = lowj ? 0u : 4u;
  sc = __builtin_amdgcn_ubfe(lowj ? s0 : s2, 8 * jj, width) | ((__builtin_amdgcn_ubfe(s0, 8 * jj + 6, 2) << 4) & himask);
  m = __builtin_amdgcn_ubfe(lowj ? s1 : s2, 8 * jj + mo, width) | ((__builtin_amdgcn_ubfe(s1, 8 * jj + 6, 2) << 4) & himask);
}

// Weight k of a row of GGUF blocks (Q8_0, Q4_K, Q5_K, Q6_K), dequantised
// exactly as the CPU oracle does it: every product and difference rounded
// on its own (__fmul_rn / __fsub_rn, so no file's FMA contraction can fuse
// them).  For the exact-f32 paths: the GEMV's generic kernel and IEEE path,
// and the prefill pre-pass's rows with infinite or NaN activations.
__device__ __forceinline__ float deq_elem(int type, const uint8_t *row, uint32_t k) {
  if (type == kQ8_0) {
    const uint8_t *blk = row + (size_t)(k >> 5) * kQ8Bytes;
    const float d = f16_bits_hw(*reinterpret_cast<const uint16_t *>(blk));
    return __fmul_rn((float)(int8_t)blk[2 + (k & 31)], d);
  } else if (type == kQ4_K || type == kQ5_K) {
    const bool q5 = type == kQ5_K;
    const uint8_t *blk = row + (size_t)(k >> 8) * (q5 ? kQ5KBytes : kQ4KBytes);
    const uint32_t rr = k & 255u, c = rr >> 6, hi = (rr >> 5) & 1u, l = rr & 31u;
    const uint32_t *wd = reinterpret_cast<const uint32_t *>(blk);
    uint32_t sc, m;
    q4k_scale_min(2 * c + hi, wd[1], wd[2], wd[3], sc, m);
    const float d = f16_bits_hw(wd[0] & 0xffffu), dmin = f16_bits_hw(wd[0] >> 16);
    uint32_t q = (blk[(q5 ? 48 : 16) + 32 * c + l] >> (4 * hi)) & 15u;
    if (q5) q |= ((blk[16 + l] >> (2 * c + hi)) & 1u) << 4;
    return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)q), __fmul_rn(dmin, (float)m));
  } else {
    const uint8_t *blk = row + (size_t)(k >> 8) * kQ6KBytes;
    const uint32_t rr = k & 255u, hh = rr >> 7, quarter = (rr >> 5) & 3u, l = rr & 31u;
    const uint32_t qlb = blk[64 * hh + l + ((quarter & 1u) ? 32u : 0u)];
    const uint32_t lo4 = (qlb >> ((quarter & 2u) ? 4u : 0u)) & 15u;
    const uint32_t hi2 = (blk[128 + 32 * hh + l] >> (2 * quarter)) & 3u;
    const int q = (int)(lo4 | (hi2 << 4)) - 32;
    const int sc = (int8_t)blk[192 + 8 * hh + l / 16 + 2 * quarter];
    const float d = f16_bits_hw(*reinterpret_cast<const uint16_t *>(blk + 208));
    return __fmul_rn(__fmul_rn(d, (float)sc), (float)q);
  }
}

}  // namespace okq
