// okq_gemm.hip -- MFMA dequant-GEMM for prefill: Y[M,N] = X[M,K] W[N,K]^T (+bias)
//
// Numerics (exact operands, f32 accumulation):
//   * A = X as fp16 after a per-row power-of-two scale 2^-s (row max into
//     [512, 1024), undone exactly in the epilogue).  A scaled bf16 value is
//     exact in fp16 down to 2^-27 of its row's maximum (bf16 carries 8
//     significant bits); f32 activations are split into an fp16 hi plane and
//     an fp16 lo plane (x ~= hi + lo to ~2^-22 relative) and contracted twice.
//   * B = the integer part of the dequantised weight, exact in fp16:
//       Q4_K: sc * q       (6-bit scale x 4-bit quant <= 945)
//       Q6_K: sc * (q - 32) (|.| <= 4096) as two planes hi + lo, hi =
//             fp16(sc * (q - 32)) and the exact remainder lo in {-1, 0, 1},
//             each contracted with A (the x_lo * lo term, below 2^-22 of the
//             result, is left out)
//     The super-block scales d and dmin are applied in f32 to the per-super-
//     block MFMA accumulators; the Q4_K min term  sum_s m_s * sum_{k in s} x_k
//     is one extra K=16 MFMA per super-block on (xsum hi, xsum lo) x m.
//   So every product inside an MFMA is exact and only f32 summation rounds.
//
// Layout / schedule (gfx950):
//   * A pre-pass (one workgroup per row) converts X once per call into a
//     workspace: fp16 planes [M][K], per-32 sums [M][K/32] as fp16 (hi, lo)
//     pairs (<= 32768 after scaling) and the row scales 2^s [M].
//   * Workgroup tile 256 x 128 (8 waves) or 128 x 128 (4 waves) when 256-row
//     tiles would leave CUs idle; each wave owns 64 x 64 = 2 x 2 MFMA 32x32x16
//     tiles.  K advances in steps of one 64-weight Q4_K chunk through a
//     software pipeline: raw loads two steps ahead in registers, the B
//     dequantisation (GGUF blocks -> fp16 sc*q) of step i+1 overlapping the
//     MFMAs of step i, double-buffered LDS, one barrier per step.
//   * Tiles are ordered so consecutive tiles (the M-tiles of one N-tile) land
//     on one XCD: workgroup b runs on XCD b % 8, so b is remapped to give each
//     XCD a contiguous range of tiles and the weight tile is re-read from that
//     XCD's L2.
#include <algorithm>
#include <type_traits>

#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

// Buffer descriptor over [base, base + bytes), bytes < 2^32.  Loads past the
// end return zeros: rows beyond M or N stage as zeros without branches.
__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload4(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }

constexpr int kBN = 128;

// ---------------------------------------------------------------------------
// pre-pass: X -> fp16 planes + per-32 sums, one workgroup per row
// ---------------------------------------------------------------------------
// Row m is scaled by 2^-s_m (exact) so that its largest |x| lies in
// [512, 1024): every fp16 value and every per-32 sum (<= 32768) is finite,
// and a bf16 value is exact in fp16 down to 2^-27 of the row maximum.  The
// GEMM epilogue multiplies the row's outputs by 2^s_m (rscale[m]), also exact.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return as_f32(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return as_f32(w & 0xffff0000u); }

template <bool kF32>
__device__ __forceinline__ void load8(const void *X, int64_t base, float v[8]) {
  if (kF32) {
    const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(X) + base);
    const float4 a = p[0], b = p[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
    const u32x4 q = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(X) + base);
    v[0] = bf16_lo(q.x), v[1] = bf16_hi(q.x), v[2] = bf16_lo(q.y), v[3] = bf16_hi(q.y);
    v[4] = bf16_lo(q.z), v[5] = bf16_hi(q.z), v[6] = bf16_lo(q.w), v[7] = bf16_hi(q.w);
  }
}

// Shared by both forms of the pre-pass: the row's scale from its max |x|,
// then the scaled fp16 planes and per-32 sums of 8 values (one chunk; fixed
// order: pairs within a thread, then the four threads of the run through DPP).
__device__ __forceinline__ int prep_exp(float amax) {
  // 2^-s with amax * 2^-s in [512, 1024); zero, inf and NaN rows keep s = 0
  return (amax > 0.0f && amax <= 3.4028235e38f) ? __builtin_amdgcn_frexp_expf(amax) - 10 : 0;
}

template <bool kF32>
__device__ __forceinline__ void prep_chunk(const float v[8], int s, bool ok, int64_t base, int m, int K, int c,
                                           int tid, _Float16 *__restrict__ xhi, _Float16 *__restrict__ xlo,
                                           h2 *__restrict__ xsum) {
  h8 hv, lv;
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float w = ldexpf(v[i], -s);
    t += w;
    const _Float16 h = (_Float16)w;
    hv[i] = h;
    lv[i] = (_Float16)(w - (float)h);
  }
  t += dpp_row_f<0xB1>(t);  // quad_perm 1,0,3,2
  t += dpp_row_f<0x4E>(t);  // quad_perm 2,3,0,1
  if (ok) {
    *reinterpret_cast<h8 *>(xhi + base) = hv;
    if (kF32) *reinterpret_cast<h8 *>(xlo + base) = lv;
    if ((tid & 3) == 0) {
      const _Float16 sh = (_Float16)t;
      h2 pair;
      pair[0] = sh;
      pair[1] = (_Float16)(t - (float)sh);
      xsum[(int64_t)m * (K / 32) + c / 4] = pair;
    }
  }
}

// The row's largest |x| as the largest magnitude bit pattern (the unsigned
// order of |x| is the float order, with NaN above infinity above every
// finite value, so one reduction also tells whether the row holds an
// infinity or a NaN: a result >= 0x7f800000).
// Within a wave: DPP inside each 16-lane row, then the four rows' lanes 0,
// 16, 32 and 48 read as scalars (six ds_bpermute shuffles instead: the calls
// 0.3-0.6 us slower).
template <int kCtl>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t a) {
  const uint32_t b = dpp_row_u<kCtl>(a);
  return a > b ? a : b;
}
__device__ __forceinline__ uint32_t block_max_bits(uint32_t a, uint32_t *red, int tid) {
  a = dpp_umax<0xB1>(a);   // quad_perm 1,0,3,2
  a = dpp_umax<0x4E>(a);   // quad_perm 2,3,0,1
  a = dpp_umax<0x141>(a);  // row_half_mirror
  a = dpp_umax<0x140>(a);  // row_mirror
  {
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)a, 0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)a, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)a, 32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)a, 48);
    const uint32_t x0 = r0 > r1 ? r0 : r1, x1 = r2 > r3 ? r2 : r3;
    a = x0 > x1 ? x0 : x1;
  }
  if ((tid & 63) == 0) red[tid >> 6] = a;
  __syncthreads();
  const uint32_t x = red[0] > red[1] ? red[0] : red[1], y = red[2] > red[3] ? red[2] : red[3];
  return x > y ? x : y;
}
__device__ __forceinline__ uint32_t abs_bits(float v) { return as_u32(v) & 0x7fffffffu; }

// Rows holding an infinity or a NaN.  The MFMA kernels cannot give them the
// reference's IEEE results: they contract sc * q and the min term apart, so
// an infinite activation meets a zero product of one part (inf * 0 = NaN)
// where the reference multiplies it by the whole weight d * sc * q - dmin * m
// (non-zero: a signed infinity).  The pre-pass computes such a row's outputs
// itself and marks its row scale NaN; the GEMM epilogues and the split-K
// reduction leave rows with a NaN scale alone.  Only the non-finite
// activations decide an output here (a finite product cannot turn an
// infinity or a NaN into anything else), so each output is the IEEE sum of
// x_k * W[o, k] over the row's non-finite positions k, then + bias[o]:
// NaN where a product is NaN or infinities of both signs meet, the
// infinity otherwise -- the reference's own values.
struct PrepIeee {
  const uint8_t *w;
  const float *bias;
  float *y;
  size_t row_bytes;
  int type, N;
};
constexpr int kIeeeCap = 1024;  // non-finite positions listed in LDS; more: every column scans the row

template <bool kF32>
__device__ __forceinline__ float x_at(const void *X, int64_t i) {
  if (kF32) return static_cast<const float *>(X)[i];
  return as_f32((uint32_t) static_cast<const uint16_t *>(X)[i] << 16);
}
__device__ __forceinline__ bool non_finite(float v) { return !(fabsf(v) <= 3.4028235e38f); }

template <bool kF32>
__device__ void prep_ieee_row(const void *__restrict__ X, int m, int K, const PrepIeee &P, int tid) {
  __shared__ int cnt;
  __shared__ int pos[kIeeeCap];
  if (tid == 0) cnt = 0;
  __syncthreads();
  const int64_t row = (int64_t)m * K;
  for (int k = tid; k < K; k += 256)
    if (non_finite(x_at<kF32>(X, row + k))) {
      const int i = atomicAdd(&cnt, 1);
      if (i < kIeeeCap) pos[i] = k;
    }
  __syncthreads();
  const int n = cnt;
  for (int o = tid; o < P.N; o += 256) {
    const uint8_t *wrow = P.w + (size_t)o * P.row_bytes;
    float acc = 0.0f;
    if (n <= kIeeeCap) {
      for (int j = 0; j < n; ++j)
        acc = __fadd_rn(acc, __fmul_rn(x_at<kF32>(X, row + pos[j]), deq_elem(P.type, wrow, (uint32_t)pos[j])));
    } else {
      for (int k = 0; k < K; ++k) {
        const float v = x_at<kF32>(X, row + k);
        if (non_finite(v)) acc = __fadd_rn(acc, __fmul_rn(v, deq_elem(P.type, wrow, (uint32_t)k)));
      }
    }
    P.y[(size_t)m * P.N + o] = __fadd_rn(acc, P.bias ? P.bias[o] : 0.0f);
  }
}

// CH > 0: each thread holds its CH chunks of 8 activations in registers
// (chunk c = tid + 256 i), so the row is read once; CH == 0: rows longer than
// 8 chunks per thread are read twice (max, then convert).
template <bool kF32, int CH>
__global__ __launch_bounds__(256) void gemm_prep_kernel(const void *__restrict__ X, int M, int K,
                                                        _Float16 *__restrict__ xhi, _Float16 *__restrict__ xlo,
                                                        h2 *__restrict__ xsum, float *__restrict__ rscale,
                                                        PrepIeee ieee) {
  __shared__ uint32_t red[4];
  const int m = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  const int chunks = K / 8;  // 8 activations per thread and pass; 4 consecutive threads = one 32-run
  const int64_t row = (int64_t)m * K;
  if constexpr (CH > 0) {
    float v[CH][8];
    uint32_t amax = 0u;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + 256 * i;
      if (c < chunks) {
        load8<kF32>(X, row + 8 * (int64_t)c, v[i]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < CH; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = amax > abs_bits(v[i][e]) ? amax : abs_bits(v[i][e]);
    const uint32_t rb = block_max_bits(amax, red, tid);
    const bool bad = rb >= 0x7f800000u;
    const int s = bad ? 0 : prep_exp(as_f32(rb));
    if (tid == 0) rscale[m] = bad ? __builtin_nanf("") : ldexpf(1.0f, s);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + 256 * i;  // chunks is a multiple of 32: runs never straddle the bound
      prep_chunk<kF32>(v[i], s, c < chunks, row + 8 * (int64_t)c, m, K, c, tid, xhi, xlo, xsum);
    }
    if (bad) prep_ieee_row<kF32>(X, m, K, ieee, tid);
    return;
  }
  // pass 1: row max |x|
  uint32_t amax = 0u;
  for (int c = tid; c < chunks; c += 256) {
    float v[8];
    load8<kF32>(X, row + 8 * (int64_t)c, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = amax > abs_bits(v[i]) ? amax : abs_bits(v[i]);
  }
  const uint32_t rb = block_max_bits(amax, red, tid);
  const bool bad = rb >= 0x7f800000u;
  const int s = bad ? 0 : prep_exp(as_f32(rb));
  if (tid == 0) rscale[m] = bad ? __builtin_nanf("") : ldexpf(1.0f, s);
  // pass 2: scaled fp16 planes and per-32 sums
  for (int c0 = 0; c0 < chunks; c0 += 256) {
    const int c = c0 + tid;
    const bool ok = c < chunks;
    float v[8];
    if (ok) {
      load8<kF32>(X, row + 8 * (int64_t)c, v);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    prep_chunk<kF32>(v, s, ok, row + 8 * (int64_t)c, m, K, c, tid, xhi, xlo, xsum);
  }
  if (bad) prep_ieee_row<kF32>(X, m, K, ieee, tid);
}

// ---------------------------------------------------------------------------
// Q4_K B staging
// ---------------------------------------------------------------------------
// 0x6400 | q is the fp16 value 1024 + q; (1024+q)*sc - 1024*sc = sc*q is one
// fused fp16 FMA whose exact result (an integer <= 945) is representable.
__device__ __forceinline__ h2 nib_pair(uint32_t spread, h2 sc2, h2 off2) {
  return __builtin_elementwise_fma(__builtin_bit_cast(h2, spread), sc2, off2);
}
// Four nibbles (one per byte of n4) -> two fp16 pairs of sc*q, in byte order.
// v_perm_b32 interleaves the bytes with the 0x64 exponent byte of 1024.
__device__ __forceinline__ void nib4(uint32_t n4, h2 sc2, h2 off2, h2 &p0, h2 &p1) {
  p0 = nib_pair(__builtin_amdgcn_perm(0x64646464u, n4, 0x04010400u), sc2, off2);
  p1 = nib_pair(__builtin_amdgcn_perm(0x64646464u, n4, 0x04030402u), sc2, off2);
}

// ---------------------------------------------------------------------------
// main kernel
// ---------------------------------------------------------------------------
constexpr int kKB = 64;         // K per pipeline step: one 64-weight Q4_K chunk
constexpr int kLDB = kKB + 8;   // LDS row pitch in halves (spreads rows over banks)

template <int BM, bool kLo, int kFmt>
struct alignas(16) GemmSmem {
  static constexpr bool kMins = kFmt == kQ4_K || kFmt == kQ5_K;
  _Float16 A[2][BM][kLDB];
  _Float16 Alo[2][kLo ? BM : 1][kLDB];
  _Float16 B[2][kBN][kLDB];
  _Float16 Blo[2][kFmt == kQ6_K || kFmt == kQ8_0 ? kBN : 1][kLDB];  // Q6_K, Q8_0: the exact remainder plane
  _Float16 xs[2][kMins ? BM : 1][16];   // per super-block parity: xsum hi/lo of sub-blocks 0..7
  _Float16 mn[2][kMins ? kBN : 1][16];  // per super-block parity: 6-bit mins, each twice
  float d[2][kBN], dmin[2][kMins ? kBN : 1];
};

// Raw global data of one pipeline step for one thread.
template <int BM, bool kLo, int kFmt>
struct StepRegs {
  u32x4 a[4], al[kLo ? 4 : 1];  // 32 activations (fp16) of one row
  u32x4 xs;                     // 4 (hi, lo) xsum pairs (first chunk of a super-block)
  u32x4 hd;                     // Q4_K header of the weight row's super-block
  u32x4 q;                      // 16 (BM=128) or 8 (BM=256, in .x/.y) qs bytes
  u32x4 qh;                     // Q5_K: the qh bytes of the same l (fifth bits)
  // Q6_K (BM = 128): dword windows (5 dwords for 16 bytes) of the ql bytes of
  // k < 32, of k >= 32 and of the qh bytes; 3 dwords around the half's 8
  // scales; d (2-byte load, first chunk of a super-block)
  uint32_t l0[kFmt == kQ6_K ? 5 : 1], l1[kFmt == kQ6_K ? 5 : 1], hq[kFmt == kQ6_K ? 5 : 1];
  uint32_t sc[kFmt == kQ6_K ? 3 : 1], dw;
  // Q8_0 (BM = 128): the dword window of this thread's 34-byte block
  uint32_t q8[kFmt == kQ8_0 ? 9 : 1];
};

// v = sc * (q - 32) for the four 6-bit values in the bytes of q4, as two
// exact fp16 planes v = hi + lo: 0x64|q is the fp16 1024 + q, minus 1056
// gives q - 32 exactly; hi = fp16(v) is exact while |v| <= 2048 and rounds to
// an even integer above (|v| <= 4096), and lo = fma(q - 32, sc, -hi) is the
// exact remainder (-1, 0 or 1).
__device__ __forceinline__ void q6_4(uint32_t q4, h2 sc2, h2 &p0, h2 &p1, h2 &l0, h2 &l1) {
  const h2 off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
  const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, q4, 0x04010400u)) + off;
  const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, q4, 0x04030402u)) + off;
  p0 = a * sc2;
  p1 = b * sc2;
  l0 = __builtin_elementwise_fma(a, sc2, -p0);
  l1 = __builtin_elementwise_fma(b, sc2, -p1);
}

// d * q for the four int8 quants in the bytes of q4, as two exact fp16 planes
// d * q = hi + lo: (q ^ 0x80) | 0x6400 is the fp16 1152 + q, minus 1152 gives
// q exactly; hi = fp16(d * q) (one rounding) and lo = fma(q, d, -hi) is the
// exact remainder.  Exact because d * q has at most 19 significant bits whose
// lowest is at least 2^-24 (d is an fp16), so the remainder fits an fp16, for
// every block with |d * q| below 65520 (|d| < 511.9, any block quantised from
// fp16-representable weights).
__device__ __forceinline__ void q8_4(uint32_t q4, h2 d2, h2 &p0, h2 &p1, h2 &l0, h2 &l1) {
  const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  const uint32_t b = q4 ^ 0x80808080u;
  const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u)) + off;
  const h2 c = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)) + off;
  p0 = a * d2;
  p1 = c * d2;
  l0 = __builtin_elementwise_fma(a, d2, -p0);
  l1 = __builtin_elementwise_fma(c, d2, -p1);
}

// BM x 128 workgroup tile, BM/32 waves arranged (BM/64) x 2, each 64 x 64.
// Software pipeline over 64-wide K steps: raw loads run two steps ahead in
// registers, the dequantisation of step i+1 overlaps the MFMAs of step i, LDS
// is double buffered, one barrier per step.
template <int BM, bool kLo, int kFmt>
__global__ __launch_bounds__(BM * 2) void gemm_kq_kernel(const _Float16 *__restrict__ xhi,
                                                         const _Float16 *__restrict__ xlo,
                                                         const h2 *__restrict__ xsum, const float *__restrict__ rscale,
                                                         const uint8_t *__restrict__ W, const float *__restrict__ bias,
                                                         float *__restrict__ Y, int M, int N, int K, int tiles_m,
                                                         int tiles, int ksplit, float *__restrict__ part) {
  constexpr int NT = BM * 2;       // threads
  constexpr int TPR = NT / kBN;    // B-staging threads per weight row (2 or 4)
  constexpr int QB = 32 / TPR;     // qs bytes per thread per step (16 or 8)
  constexpr bool kQ6 = kFmt == kQ6_K, kQ8 = kFmt == kQ8_0, kQ5 = kFmt == kQ5_K;
  static_assert(!kQ6 || QB == 16, "Q6_K staging takes 16-byte windows (BM = 128)");
  static_assert(!kQ8 || TPR == 2, "Q8_0 staging takes one 34-byte block per thread (BM = 128)");
  // bytes per 256 weights of a row: one super-block, or eight Q8_0 blocks
  constexpr uint32_t kBlk = kQ6 ? kQ6KBytes : kQ8 ? 8 * kQ8Bytes : kQ5 ? kQ5KBytes : kQ4KBytes;
  __shared__ GemmSmem<BM, kLo, kFmt> sm;
  // XCD-aware tile order: workgroup b runs on XCD b % 8; give each XCD a
  // contiguous range of tiles (consecutive tiles share an N-tile).
  // With split-K (ksplit > 1) workgroup (tile, z) covers super-blocks
  // [z * nsb_all / ksplit, (z + 1) * nsb_all / ksplit) and writes its f32
  // partial tile to part[z]; consecutive indices keep one slice z and walk
  // the M-tiles of an N-tile (they share the weight tile in L2).
  const int b = (int)blockIdx.x;
  const int jobs = tiles * ksplit;
  const int per_xcd = (jobs + 7) / 8;
  const int job = (b % 8) * per_xcd + b / 8;
  if (job >= jobs) return;
  const int z = job / tiles, tile = job % tiles;
  const int m0 = (tile % tiles_m) * BM;
  const int n0 = (tile / tiles_m) * kBN;

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int nsb_all = K / 256;
  const int sb0 = (int)((int64_t)z * nsb_all / ksplit);
  const int nsb = (int)((int64_t)(z + 1) * nsb_all / ksplit) - sb0;  // super-blocks of this slice
  const uint32_t row_bytes = (uint32_t)nsb_all * kBlk;

  const int sr = tid >> 1, sp = tid & 1;        // A: row, 32-wide half
  const int br = tid / TPR, bq = tid % TPR;     // B: weight row, byte window
  const uint32_t K32 = (uint32_t)K;
  const Rsrc rs_xh = make_rsrc(xhi, (uint32_t)((size_t)M * K * 2));
  const Rsrc rs_xl = make_rsrc(kLo ? xlo : xhi, (uint32_t)((size_t)M * K * 2));
  const Rsrc rs_xs = make_rsrc(xsum, (uint32_t)((size_t)M * (K / 32) * 4));
  const Rsrc rs_w = make_rsrc(W, (uint32_t)((size_t)N * row_bytes));
  // byte offsets of this thread's rows (past the end for rows >= M / >= N:
  // the descriptors return zeros there)
  const uint32_t a_row = (uint32_t)(m0 + sr) * K32 * 2u + 64u * (uint32_t)sp + 512u * (uint32_t)sb0;
  const uint32_t s_row = (uint32_t)(m0 + sr) * (K32 / 32u) * 4u + 16u * (uint32_t)sp + 32u * (uint32_t)sb0;
  const uint32_t w_row = (uint32_t)(n0 + br) * row_bytes + (uint32_t)sb0 * kBlk;

  // C = step & 3 is a compile-time constant at every call site, so the body
  // is straight-line code (no divergent branches around the loads: the wait
  // counters then only wait for the step actually consumed).  Steps past the
  // end read inside the next row or past the descriptor (zeros); unused.
  auto load = [&](StepRegs<BM, kLo, kFmt> &r, int step, auto Cc) {
    constexpr int c = decltype(Cc)::value;
    const int sb = step >> 2;
    const uint32_t ka = a_row + 2u * (uint32_t)(step * kKB);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.a[i] = bload4(rs_xh, ka + 16u * i);
    if (kLo) {
#pragma unroll
      for (int i = 0; i < 4; ++i) r.al[i] = bload4(rs_xl, ka + 16u * i);
    }
    if constexpr (kQ8) {
      // blocks 2c and 2c + 1 of the super-block hold this step's 64 weights;
      // thread bq stages block 2c + bq: a 9-dword window from the dword below
      // its (2-byte aligned) start
      const uint32_t B = w_row + (uint32_t)sb * kBlk + (2u * c + (uint32_t)bq) * kQ8Bytes;
      const uint32_t a = B & ~3u;
      const u32x4 v0 = bload4(rs_w, a), v1 = bload4(rs_w, a + 16u);
      r.q8[0] = v0.x, r.q8[1] = v0.y, r.q8[2] = v0.z, r.q8[3] = v0.w;
      r.q8[4] = v1.x, r.q8[5] = v1.y, r.q8[6] = v1.z, r.q8[7] = v1.w;
      r.q8[8] = __builtin_amdgcn_raw_buffer_load_b32(rs_w, a + 32u, 0, 0);
      return;
    }
    if constexpr (kQ6) {
      // chunk c of the super-block: half h = c / 2 (ql bytes 64h.., qh bytes
      // 128 + 32h..); this thread's l = 16 bq .. 16 bq + 15.  Windows start at
      // the dword below each (2-byte aligned) field.
      constexpr uint32_t h = c >> 1;
      const uint32_t B = w_row + (uint32_t)sb * kBlk;
      auto win = [&](uint32_t *dst, uint32_t at, int n) {
#pragma unroll
        for (int t = 0; t < n; ++t) dst[t] = __builtin_amdgcn_raw_buffer_load_b32(rs_w, (at & ~3u) + 4u * t, 0, 0);
      };
      // both chunks of a half use the same bytes (the second read hits the cache)
      win(r.l0, B + 64u * h + 16u * bq, 5);
      win(r.l1, B + 64u * h + 32u + 16u * bq, 5);
      win(r.hq, B + 128u + 32u * h + 16u * bq, 5);
      win(r.sc, B + 192u + 8u * h, 3);
      // d with a 2-byte load: a dword window could end past the tensor (whose
      // size is only 2-byte aligned) and the range check would zero it
      if constexpr (c == 0) r.dw = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs_w, B + 208u, 0, 0);
      return;
    }
    if constexpr (c == 0) r.xs = bload4(rs_xs, s_row + 32u * (uint32_t)sb);
    // Q4_K / Q5_K: the header, this thread's QB qs bytes of chunk c and
    // (Q5_K) the qh bytes of the same positions l
    const uint32_t blk = w_row + (uint32_t)sb * kBlk;
    r.hd = bload4(rs_w, blk);
    const uint32_t qo = blk + (kQ5 ? 48u : 16u) + 32u * (uint32_t)c + (uint32_t)(QB * bq);
    if (QB == 16) {
      r.q = bload4(rs_w, qo);
      if (kQ5) r.qh = bload4(rs_w, blk + 16u + (uint32_t)(QB * bq));
    } else {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs_w, qo, 0, 0);
      r.q = u32x4{v.x, v.y, 0u, 0u};
      if (kQ5) {
        const u32x2 h = __builtin_amdgcn_raw_buffer_load_b64(rs_w, blk + 16u + (uint32_t)(QB * bq), 0, 0);
        r.qh = u32x4{h.x, h.y, 0u, 0u};
      }
    }
  };

  auto stage = [&](const StepRegs<BM, kLo, kFmt> &r, int step, int buf, auto Cc) {
    constexpr int c = decltype(Cc)::value;
    const int sbp = (step >> 2) & 1;
    u32x4 *da = reinterpret_cast<u32x4 *>(&sm.A[buf][sr][32 * sp]);
#pragma unroll
    for (int i = 0; i < 4; ++i) da[i] = r.a[i];
    if (kLo) {
      u32x4 *dl = reinterpret_cast<u32x4 *>(&sm.Alo[buf][sr][32 * sp]);
#pragma unroll
      for (int i = 0; i < 4; ++i) dl[i] = r.al[i];
    }
    if constexpr (kQ8) {
      const uint32_t B = w_row + (uint32_t)(step >> 2) * kBlk + (2u * c + (uint32_t)bq) * kQ8Bytes;
      const uint32_t ra = B & 3u;
      uint32_t wv[9];  // bytes B + 4i .. of the block (realigned window)
#pragma unroll
      for (int t = 0; t < 8; ++t) wv[t] = __builtin_amdgcn_alignbyte(r.q8[t + 1], r.q8[t], ra);
      wv[8] = __builtin_amdgcn_alignbyte(0u, r.q8[8], ra);
      const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)(wv[0] & 0xffffu));
      const h2 d2 = {dh, dh};
      h2 hi[16], lo[16];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const uint32_t q4 = __builtin_amdgcn_alignbyte(wv[w + 1], wv[w], 2u);  // quants 4w .. 4w + 3
        q8_4(q4, d2, hi[2 * w], hi[2 * w + 1], lo[2 * w], lo[2 * w + 1]);
      }
      auto put = [&](_Float16 *dst, const h2 *v) {
        u32x4 *d4 = reinterpret_cast<u32x4 *>(dst);
#pragma unroll
        for (int t = 0; t < 4; ++t)
          d4[t] = u32x4{__builtin_bit_cast(uint32_t, v[4 * t]), __builtin_bit_cast(uint32_t, v[4 * t + 1]),
                        __builtin_bit_cast(uint32_t, v[4 * t + 2]), __builtin_bit_cast(uint32_t, v[4 * t + 3])};
      };
      put(&sm.B[buf][br][32 * bq], hi);
      put(&sm.Blo[buf][br][32 * bq], lo);
      return;
    }
    if constexpr (kQ6) {
      constexpr uint32_t cc = c & 1, h = c >> 1;
      const uint32_t B = w_row + (uint32_t)(step >> 2) * kBlk;
      // realign each window by the field's offset within its first dword
      auto bytes16 = [&](const uint32_t *w, uint32_t at, uint32_t o[4]) {
        const uint32_t ra = at & 3u;
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t] = __builtin_amdgcn_alignbyte(w[t + 1], w[t], ra);
      };
      uint32_t L0[4], L1[4], H[4];
      bytes16(r.l0, B + 64u * h + 16u * bq, L0);
      bytes16(r.l1, B + 64u * h + 32u + 16u * bq, L1);
      bytes16(r.hq, B + 128u + 32u * h + 16u * bq, H);
      // int8 scales of this thread's l-run (l / 16 = bq): index 8h + bq + 2p
      // for p = 2cc (k < 32) and 2cc + 1 (k >= 32)
      const uint32_t sat = B + 192u + 8u * h;
      const uint32_t s0 = __builtin_amdgcn_alignbyte(r.sc[1], r.sc[0], sat & 3u);
      const uint32_t s1 = __builtin_amdgcn_alignbyte(r.sc[2], r.sc[1], sat & 3u);
      const uint32_t ia = (uint32_t)bq + 4u * cc, ib = ia + 2u;  // 0..7
      const int sca = (int)__builtin_amdgcn_sbfe((int)(ia < 4 ? s0 : s1), 8 * (ia & 3u), 8u);
      const int scb = (int)__builtin_amdgcn_sbfe((int)(ib < 4 ? s0 : s1), 8 * (ib & 3u), 8u);
      const _Float16 fa = (_Float16)(float)sca, fb = (_Float16)(float)scb;
      const h2 sa = {fa, fa}, sbv = {fb, fb};
      // first: k < 32 of the chunk, second: k >= 32; r*: the remainder plane
      h2 fi[8], se[8], rf[8], rs[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t qa = ((L0[w] >> (4 * cc)) & 0x0F0F0F0Fu) | (((H[w] >> (4 * cc)) & 0x03030303u) << 4);
        const uint32_t qb = ((L1[w] >> (4 * cc)) & 0x0F0F0F0Fu) | (((H[w] >> (4 * cc + 2)) & 0x03030303u) << 4);
        q6_4(qa, sa, fi[2 * w], fi[2 * w + 1], rf[2 * w], rf[2 * w + 1]);
        q6_4(qb, sbv, se[2 * w], se[2 * w + 1], rs[2 * w], rs[2 * w + 1]);
      }
      auto put = [&](_Float16 *dst, const h2 *v) {
        u32x4 *d4 = reinterpret_cast<u32x4 *>(dst);
#pragma unroll
        for (int t = 0; t < 2; ++t)
          d4[t] = u32x4{__builtin_bit_cast(uint32_t, v[4 * t]), __builtin_bit_cast(uint32_t, v[4 * t + 1]),
                        __builtin_bit_cast(uint32_t, v[4 * t + 2]), __builtin_bit_cast(uint32_t, v[4 * t + 3])};
      };
      put(&sm.B[buf][br][16 * bq], fi);
      put(&sm.B[buf][br][32 + 16 * bq], se);
      put(&sm.Blo[buf][br][16 * bq], rf);
      put(&sm.Blo[buf][br][32 + 16 * bq], rs);
      if constexpr (c == 0) sm.d[sbp][br] = f16_bits_hw(r.dw & 0xffffu);
      return;
    }
    if constexpr (c == 0) *reinterpret_cast<u32x4 *>(&sm.xs[sbp][sr][8 * sp]) = r.xs;
    // low nibbles -> sub-block 2c (k = byte), high nibbles -> 2c+1 (k = 32 + byte)
    uint32_t sc0, mv0, sc1, mv1;
    q4k_scale_min(2 * c, r.hd.y, r.hd.z, r.hd.w, sc0, mv0);
    q4k_scale_min(2 * c + 1, r.hd.y, r.hd.z, r.hd.w, sc1, mv1);
    const _Float16 s0 = (_Float16)(float)sc0, s1 = (_Float16)(float)sc1;
    const _Float16 o0 = (_Float16)(-1024.0f * (float)sc0), o1 = (_Float16)(-1024.0f * (float)sc1);
    const h2 sc0v = {s0, s0}, sc1v = {s1, s1}, off0 = {o0, o0}, off1 = {o1, o1};
    constexpr int NW = QB / 4;
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    h2 lo[2 * NW], hi[2 * NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      // Q5_K: bit 2c of qh[l] is bit 4 of the low nibble's value, bit 2c + 1
      // of the high one's (sc * q <= 63 * 31 stays an exact fp16 integer)
      const uint32_t f0 = kQ5 ? ((qh[w] >> (2 * c)) & 0x01010101u) << 4 : 0u;
      const uint32_t f1 = kQ5 ? ((qh[w] >> (2 * c + 1)) & 0x01010101u) << 4 : 0u;
      nib4((q[w] & 0x0F0F0F0Fu) | f0, sc0v, off0, lo[2 * w], lo[2 * w + 1]);
      nib4(((q[w] >> 4) & 0x0F0F0F0Fu) | f1, sc1v, off1, hi[2 * w], hi[2 * w + 1]);
    }
    u32x4 *dlo = reinterpret_cast<u32x4 *>(&sm.B[buf][br][QB * bq]);
    u32x4 *dhi = reinterpret_cast<u32x4 *>(&sm.B[buf][br][32 + QB * bq]);
#pragma unroll
    for (int i = 0; i < NW / 2; ++i) {
      dlo[i] = u32x4{__builtin_bit_cast(uint32_t, lo[4 * i]), __builtin_bit_cast(uint32_t, lo[4 * i + 1]),
                     __builtin_bit_cast(uint32_t, lo[4 * i + 2]), __builtin_bit_cast(uint32_t, lo[4 * i + 3])};
      dhi[i] = u32x4{__builtin_bit_cast(uint32_t, hi[4 * i]), __builtin_bit_cast(uint32_t, hi[4 * i + 1]),
                     __builtin_bit_cast(uint32_t, hi[4 * i + 2]), __builtin_bit_cast(uint32_t, hi[4 * i + 3])};
    }
    if constexpr (c == 0) {
      // every staging thread of the row loaded the same header: all of them
      // store the same values (no branch, so no conservative wait counters)
      sm.d[sbp][br] = f16_bits_hw(r.hd.x & 0xffffu);
      sm.dmin[sbp][br] = f16_bits_hw(r.hd.x >> 16);
      h8 m0v, m1v;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t scj, mj;
        q4k_scale_min((uint32_t)j, r.hd.y, r.hd.z, r.hd.w, scj, mj);
        const _Float16 mh = (_Float16)(float)mj;
        if (j < 4) {
          m0v[2 * j] = mh;
          m0v[2 * j + 1] = mh;
        } else {
          m1v[2 * (j - 4)] = mh;
          m1v[2 * (j - 4) + 1] = mh;
        }
      }
      *reinterpret_cast<h8 *>(&sm.mn[sbp][br][0]) = m0v;
      *reinterpret_cast<h8 *>(&sm.mn[sbp][br][8]) = m1v;
    }
  };

  f16x acc[2][2], accs[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // MFMA slice ks, lane group g = lane/32 covers k = 32g + 8ks + [0, 8) of the
  // 64-wide step (the same k order as the direct-A kernel, so both kernels
  // give bit-identical results for a row)
  const int fr = lane & 31, fk = 8 * (lane >> 5), fk4 = 32 * (lane >> 5);
  const f16x zero = {};

  auto mma = [&](int buf, bool first) {
#pragma unroll
    for (int ks = 0; ks < kKB / 16; ++ks) {
      h8 a[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const h8 *>(&sm.A[buf][wm * 64 + 32 * i + fr][fk4 + 8 * ks]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bv[j] = *reinterpret_cast<const h8 *>(&sm.B[buf][wn * 64 + 32 * j + fr][fk4 + 8 * ks]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          accs[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bv[j], (first && ks == 0) ? zero : accs[i][j],
                                                              0, 0, 0);
      if constexpr (kQ6 || kQ8) {  // the exact remainder plane of the weights (x_lo * remainder is below 2^-22)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const h8 bl = *reinterpret_cast<const h8 *>(&sm.Blo[buf][wn * 64 + 32 * j + fr][fk4 + 8 * ks]);
#pragma unroll
          for (int i = 0; i < 2; ++i)
            accs[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bl, accs[i][j], 0, 0, 0);
        }
      }
      if (kLo) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
          a[i] = *reinterpret_cast<const h8 *>(&sm.Alo[buf][wm * 64 + 32 * i + fr][fk4 + 8 * ks]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            accs[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bv[j], accs[i][j], 0, 0, 0);
      }
    }
  };

  // end of a super-block: acc += d * accs - dmin * (xsum . m)  (Q6_K: d * accs)
  auto scale = [&](int sbp) {
    if constexpr (kQ8) {  // d is inside the B planes
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] += accs[i][j][e];
      return;
    }
    if constexpr (kQ6) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float dv = sm.d[sbp][wn * 64 + 32 * j + fr];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] = fmaf(dv, accs[i][j][e], acc[i][j][e]);
      }
      return;
    }
    h8 xa[2], mb[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) xa[i] = *reinterpret_cast<const h8 *>(&sm.xs[sbp][wm * 64 + 32 * i + fr][fk]);
#pragma unroll
    for (int j = 0; j < 2; ++j) mb[j] = *reinterpret_cast<const h8 *>(&sm.mn[sbp][wn * 64 + 32 * j + fr][fk]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int nn = wn * 64 + 32 * j + fr;
      const float dv = sm.d[sbp][nn], dm = -sm.dmin[sbp][nn];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const f16x mins = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[i], mb[j], zero, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = fmaf(dm, mins[e], fmaf(dv, accs[i][j][e], acc[i][j][e]));
      }
    }
  };

  // Pipeline over steps i = 4*sb + c: LDS buffer i&1 holds step i while the
  // register set of step i+1 is staged into the other buffer and step i+2 is
  // in flight.
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  using C2 = std::integral_constant<int, 2>;
  using C3 = std::integral_constant<int, 3>;
  StepRegs<BM, kLo, kFmt> R0, R1;
  load(R0, 0, C0{});
  load(R1, 1, C1{});
  stage(R0, 0, 0, C0{});
  __syncthreads();
  for (int sb = 0; sb < nsb; ++sb) {
    const int i = 4 * sb;
    load(R0, i + 2, C2{});
    mma(0, true);
    stage(R1, i + 1, 1, C1{});
    __syncthreads();
    load(R1, i + 3, C3{});
    mma(1, false);
    stage(R0, i + 2, 0, C2{});
    __syncthreads();
    load(R0, i + 4, C0{});
    mma(0, false);
    stage(R1, i + 3, 1, C3{});
    __syncthreads();
    load(R1, i + 5, C1{});
    mma(1, false);
    scale(sb & 1);
    stage(R0, i + 4, 0, C0{});
    __syncthreads();
  }

  // epilogue: C layout row = 8*(e/4) + 4*(lane/32) + e%4, col = lane%32
  if (ksplit > 1) {  // raw partial tile; splitk_reduce_kernel scales and adds the bias
    float *P = part + (size_t)z * M * N;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + 32 * j + fr;
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = m0 + wm * 64 + 32 * i + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
          if (row < M) P[(size_t)row * N + col] = acc[i][j][e];
        }
    }
    return;
  }
  // undo the pre-pass's per-row power-of-two scale (exact)
  float rs[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = m0 + wm * 64 + 32 * i + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
      rs[i][e] = row < M ? rscale[row] : 0.0f;
    }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + wn * 64 + 32 * j + fr;
    if (col >= N) continue;
    const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * 64 + 32 * i + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
        // a NaN scale: the pre-pass wrote this row's IEEE outputs
        if (row < M && !__builtin_isnan(rs[i][e])) Y[(size_t)row * N + col] = acc[i][j][e] * rs[i][e] + bv;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// decode batches (2 <= M <= 16): a streaming kernel with MFMA contraction
// ---------------------------------------------------------------------------
// At most 16 activation rows: every weight meets one 16-row MFMA tile, so the
// weights are dequantised by the lane that loads them straight into MFMA B
// fragments (no LDS staging, no reuse to gain), and the kernel is organised
// like the GEMV: a workgroup stages its K-slice of the activations (the
// pre-pass planes) in LDS once, then every wave streams a sequence of items
// (16-column tile, super-block) through a ring of D register sets with no
// further barrier.  Operands and scaling are those of gemm_kq_kernel (exact
// fp16 products, per-super-block f32 scaling by d and dmin).
//
// MFMA v_mfma_f32_16x16x32_f16: lane l holds A[l % 16][8 (l / 16) + 0..7],
// B[8 (l / 16) + 0..7][l % 16] and D[4 (l / 16) + 0..3][l % 16].  K order
// inside a super-block: slice t (8 per super-block) and lane group g = l / 16
// cover k = 64g + 32(t & 1) + 8(t >> 1) + [0, 8), i.e. nibble plane t & 1 of
// bytes 8(t >> 1) .. + 8 of qs chunk g -- a lane group reads only its own
// 32-byte chunk (and the header) of each block.
constexpr int kDecRows = kGemmDecodeRows;  // two 16-row MFMA groups share each B fragment above 16 rows
constexpr int kDecWaves = 16;
constexpr int64_t kDecLdsBytes = 144 * 1024;  // activations of a slice (one workgroup per CU fills its registers)
constexpr int kDecStage = 4;                // 16-byte activation pieces per thread (of 1024)
constexpr int kDecMaxTiles = 4;             // unsplit K: column tiles per wave (bias staged in LDS)

// The matrices of one decode-batch launch: matrix p owns the 16-column tiles
// [tile0[p], tile0[p + 1]) of the launch (tile0[0] = 0; unused entries
// INT32_MAX) and has n rows of weights w (w_bytes), bias `bias` (bias_bytes,
// 0 when null) and output y [M][n].  A kernel reads a matrix's record with
// scalar loads from its arguments (a wave-uniform index), once per tile it
// moves to; the byte sizes come from the host, so no select or branch
// builds the buffer descriptors.
struct DecMat {
  const uint8_t *w;
  const float *bias;
  float *y;
  int n, tile0;
  uint32_t w_bytes, bias_bytes;
};
struct DecMats {
  DecMat mat[kDecMats];
  int tile0[kDecMats];
};

typedef float f4 __attribute__((ext_vector_type(4)));

// Workgroup barrier for LDS only: waits for this wave's LDS operations, not
// for its vector-memory loads (loads issued ahead stay in flight across it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // gfx9 encoding: lgkmcnt(0), vmcnt and expcnt unconstrained
  __builtin_amdgcn_s_barrier();
}

// Activation row r of a decode-batch plane (row pitch P halves, P = 8 mod
// 256) starts at dec_row(r, P) halves: rows 8-15 of each 16-row group sit
// 64 halves (128 B) further.  A ds_read_b128 serves 32 lanes per pass over
// 512 B of banks; the pass's two lane groups read 16 rows each at k and
// k + 64, which with a plain pitch would put rows 8-15 of the first group on
// the banks of rows 0-7 of the second (measured 1.8x slower per read).  The
// shifts use kDecRowExtra halves past M * P.
constexpr int kDecRowExtra = 128;
__host__ __device__ constexpr int dec_row(int r, int P) { return r * P + 64 * ((r + 8) >> 4); }

// Byte offset of the decode-batch kernel's small LDS arrays (bias, row scales,
// row maxima): past the activation slice (planes of M * P + kDecRowExtra
// halves, per-32 sums) and, with an in-workgroup K split, past the partial
// tiles that reuse those bytes at the end ([kDecWaves][RG] x 1 KB).
__host__ __device__ constexpr size_t dec_tail_offset(int M, int P, int nsbs, int planes, bool kw_split, int RG) {
  const size_t act = ((size_t)M * P + kDecRowExtra) * 2 * planes + (size_t)M * nsbs * 32;
  const size_t red = kw_split ? (size_t)kDecWaves * RG * 1024 : 0;
  return ((act > red ? act : red) + 15) & ~(size_t)15;
}

// Per-format parts of the decode kernel: the registers of one item (one
// super-block of one 16-column tile, as seen by one lane), their loads, and
// the contraction of one super-block into the lane's 4 accumulators.
// `ar`/`arl` point at the lane's A row (hi/lo planes) at the super-block's
// first activation, `xs` at the row's xsum pairs of the super-block.
struct DecQ4K {
  static constexpr uint32_t kBlk = kQ4KBytes;
  static constexpr int kType = kQ4_K;
  static constexpr bool kSums = true;  // the min term contracts the per-32 activation sums
  // items in flight per wave: 4 with one 16-row group (the Llama shapes give
  // a wave 4 items, so all are issued at once), 3 with two (register budget)
  static constexpr int kDepth = 3, kDepth1 = 4;
  struct Item {
    u32x4 hd, q0, q1;
  };
  // lane group g reads the header and qs chunk g (bytes 32g .. 32g + 31)
  __device__ static void load(Item &it, Rsrc rs, uint32_t blk, int g) {
    it.hd = bload4(rs, blk);
    it.q0 = bload4(rs, blk + 16u + 32u * (uint32_t)g);
    it.q1 = bload4(rs, blk + 32u + 32u * (uint32_t)g);
  }
  // slice t: k = 64g + 32(t & 1) + 8(t >> 1) + [0, 8) (nibble plane t & 1 of
  // bytes 8(t >> 1) .. of chunk g); the min term is one more MFMA on
  // (xsum hi, xsum lo) x m (lane groups 2, 3 contribute zeros)
  template <bool kLo, int RG>
  __device__ static void contract(const Item &it, const _Float16 *const *ar, const _Float16 *const *arl,
                                  const _Float16 *const *xs, const float *rsc, int g, f4 *acc) {
    const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    h2 scv[2], offv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t sc, mv;
      q4k_scale_min_sel(2u * (uint32_t)g + (uint32_t)j, it.hd.y, it.hd.z, it.hd.w, sc, mv);
      const _Float16 sh = (_Float16)(uint16_t)sc, oh = sh * (_Float16)-1024.0f;
      scv[j] = h2{sh, sh};
      offv[j] = h2{oh, oh};
    }
    h8 mb;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t sc, mv;
      q4k_scale_min_sel((4u * (uint32_t)g + (uint32_t)j) & 7u, it.hd.y, it.hd.z, it.hd.w, sc, mv);
      const _Float16 mh = g < 2 ? (_Float16)(uint16_t)mv : (_Float16)0.0f;
      mb[2 * j] = mh;
      mb[2 * j + 1] = mh;
    }
    f4 accs[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) accs[q] = zero4;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int nib = t & 1, p8 = t >> 1;
      const u32x4 pc = (p8 >> 1) ? it.q1 : it.q0;
      const uint32_t d0 = (p8 & 1) ? pc.z : pc.x, d1 = (p8 & 1) ? pc.w : pc.y;
      const uint32_t n0v = nib ? (d0 >> 4) & 0x0F0F0F0Fu : d0 & 0x0F0F0F0Fu;
      const uint32_t n1v = nib ? (d1 >> 4) & 0x0F0F0F0Fu : d1 & 0x0F0F0F0Fu;
      h2 p0, p1, p2, p3;
      nib4(n0v, scv[nib], offv[nib], p0, p1);
      nib4(n1v, scv[nib], offv[nib], p2, p3);
      const h8 bv = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      const int ka = 64 * g + 32 * nib + 8 * p8;
#pragma unroll
      for (int q = 0; q < RG; ++q) {
        const h8 ah = *reinterpret_cast<const h8 *>(ar[q] + ka);
        accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bv, accs[q], 0, 0, 0);
        if (kLo) {
          const h8 al = *reinterpret_cast<const h8 *>(arl[q] + ka);
          accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bv, accs[q], 0, 0, 0);
        }
      }
    }
    const float dv = f16_bits_hw(it.hd.x & 0xffffu), dm = -f16_bits_hw(it.hd.x >> 16);
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      const h8 xa = g < 2 ? *reinterpret_cast<const h8 *>(xs[q] + 8 * g) : h8{};
      const f4 mins = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, mb, zero4, 0, 0, 0);
      const f4 s4 = *reinterpret_cast<const f4 *>(rsc + 16 * q);  // the rows' 2^s (exact products)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[q][v] = fmaf(s4[v], fmaf(dm, mins[v], dv * accs[q][v]), acc[q][v]);
    }
  }
};

// Q5_K: DecQ4K with the fifth bit of every weight from qh (bit 2g + nibble
// plane of qh[l] for byte l of qs chunk g); sc * q <= 63 * 31 stays an exact
// fp16 integer.  A lane group reads the header, all 32 qh bytes and its qs
// chunk: 20 registers per item, so the ring is one item shorter.
struct DecQ5K {
  static constexpr uint32_t kBlk = kQ5KBytes;
  static constexpr int kType = kQ5_K;
  static constexpr bool kSums = true;
  static constexpr int kDepth = 2, kDepth1 = 3;
  struct Item {
    u32x4 hd, h0, h1, q0, q1;
  };
  __device__ static void load(Item &it, Rsrc rs, uint32_t blk, int g) {
    it.hd = bload4(rs, blk);
    it.h0 = bload4(rs, blk + 16u);
    it.h1 = bload4(rs, blk + 32u);
    it.q0 = bload4(rs, blk + 48u + 32u * (uint32_t)g);
    it.q1 = bload4(rs, blk + 64u + 32u * (uint32_t)g);
  }
  template <bool kLo, int RG>
  __device__ static void contract(const Item &it, const _Float16 *const *ar, const _Float16 *const *arl,
                                  const _Float16 *const *xs, const float *rsc, int g, f4 *acc) {
    const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    h2 scv[2], offv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t sc, mv;
      q4k_scale_min_sel(2u * (uint32_t)g + (uint32_t)j, it.hd.y, it.hd.z, it.hd.w, sc, mv);
      const _Float16 sh = (_Float16)(uint16_t)sc, oh = sh * (_Float16)-1024.0f;
      scv[j] = h2{sh, sh};
      offv[j] = h2{oh, oh};
    }
    h8 mb;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t sc, mv;
      q4k_scale_min_sel((4u * (uint32_t)g + (uint32_t)j) & 7u, it.hd.y, it.hd.z, it.hd.w, sc, mv);
      const _Float16 mh = g < 2 ? (_Float16)(uint16_t)mv : (_Float16)0.0f;
      mb[2 * j] = mh;
      mb[2 * j + 1] = mh;
    }
    f4 accs[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) accs[q] = zero4;
    const uint32_t hsh = 2u * (uint32_t)g;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int nib = t & 1, p8 = t >> 1;
      const u32x4 pc = (p8 >> 1) ? it.q1 : it.q0;
      const u32x4 hc = (p8 >> 1) ? it.h1 : it.h0;
      const uint32_t d0 = (p8 & 1) ? pc.z : pc.x, d1 = (p8 & 1) ? pc.w : pc.y;
      const uint32_t e0 = (p8 & 1) ? hc.z : hc.x, e1 = (p8 & 1) ? hc.w : hc.y;
      const uint32_t f0 = ((e0 >> (hsh + (uint32_t)nib)) & 0x01010101u) << 4;
      const uint32_t f1 = ((e1 >> (hsh + (uint32_t)nib)) & 0x01010101u) << 4;
      const uint32_t n0v = (nib ? (d0 >> 4) & 0x0F0F0F0Fu : d0 & 0x0F0F0F0Fu) | f0;
      const uint32_t n1v = (nib ? (d1 >> 4) & 0x0F0F0F0Fu : d1 & 0x0F0F0F0Fu) | f1;
      h2 p0, p1, p2, p3;
      nib4(n0v, scv[nib], offv[nib], p0, p1);
      nib4(n1v, scv[nib], offv[nib], p2, p3);
      const h8 bv = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      const int ka = 64 * g + 32 * nib + 8 * p8;
#pragma unroll
      for (int q = 0; q < RG; ++q) {
        const h8 ah = *reinterpret_cast<const h8 *>(ar[q] + ka);
        accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bv, accs[q], 0, 0, 0);
        if (kLo) {
          const h8 al = *reinterpret_cast<const h8 *>(arl[q] + ka);
          accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bv, accs[q], 0, 0, 0);
        }
      }
    }
    const float dv = f16_bits_hw(it.hd.x & 0xffffu), dm = -f16_bits_hw(it.hd.x >> 16);
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      const h8 xa = g < 2 ? *reinterpret_cast<const h8 *>(xs[q] + 8 * g) : h8{};
      const f4 mins = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, mb, zero4, 0, 0, 0);
      const f4 s4 = *reinterpret_cast<const f4 *>(rsc + 16 * q);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[q][v] = fmaf(s4[v], fmaf(dm, mins[v], dv * accs[q][v]), acc[q][v]);
    }
  }
};

// kDw: d is taken from the scales' last dword (bytes 208-211 of the block
// from the dword below it: d sits at its byte r), one load fewer per item.
// That dword reaches 2 bytes into the next block when the block starts on a
// dword, so the launcher takes this form only for tensors whose last block
// starts 2 bytes off one (a size that is a multiple of 4: an even number of
// blocks); otherwise d comes with a 2-byte load of its own (a dword around
// it could end past the tensor, where the range check zeroes it).
template <bool kDw>
struct DecQ6KT {
  static constexpr uint32_t kBlk = kQ6KBytes;
  static constexpr int kType = kQ6_K;
  static constexpr bool kSums = false;
  static constexpr int kDepth = 2, kDepth1 = 2;
  // Slice t = (half hh = t >> 2, quarter qq = t & 3); lane group g covers
  // l = 8g .. 8g + 7 of it: k = 128hh + 32qq + 8g + [0, 8), i.e. ql bytes
  // 64hh + 32(qq & 1) + 8g .. (nibble qq >> 1), qh bytes 128 + 32hh + 8g ..
  // (bits 2qq), scale byte 8hh + 2qq + (g >> 1).  Blocks are 2-byte aligned:
  // each 8-byte field is read as a 3-dword window from the dword below it
  // and realigned by r = block & 3.
  struct Item {
    u32x3 ql[4], qh[2];  // ql: (hh, qq & 1) = (0,0) (0,1) (1,0) (1,1)
    u32x4 sc4;
    uint32_t sc1, dw, r;
  };
  __device__ static void load(Item &it, Rsrc rs, uint32_t blk, int g) {
    const uint32_t r = blk & 3u, a = blk - r;
#pragma unroll
    for (int p = 0; p < 4; ++p)
      it.ql[p] = __builtin_amdgcn_raw_buffer_load_b96(rs, a + 64u * (uint32_t)(p >> 1) + 32u * (uint32_t)(p & 1) + 8u * (uint32_t)g, 0, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h)
      it.qh[h] = __builtin_amdgcn_raw_buffer_load_b96(rs, a + 128u + 32u * (uint32_t)h + 8u * (uint32_t)g, 0, 0);
    it.sc4 = bload4(rs, a + 192u);
    it.sc1 = __builtin_amdgcn_raw_buffer_load_b32(rs, a + 208u, 0, 0);
    if constexpr (!kDw) it.dw = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, blk + 208u, 0, 0);
    it.r = r;
  }
  template <bool kLo, int RG>
  __device__ static void contract(const Item &it, const _Float16 *const *ar, const _Float16 *const *arl,
                                  const _Float16 *const *, const float *rsc, int g, f4 *acc) {
    const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t r = it.r;
    uint32_t L[4][2], H[2][2];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      L[p][0] = __builtin_amdgcn_alignbyte(it.ql[p].y, it.ql[p].x, r);
      L[p][1] = __builtin_amdgcn_alignbyte(it.ql[p].z, it.ql[p].y, r);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      H[h][0] = __builtin_amdgcn_alignbyte(it.qh[h].y, it.qh[h].x, r);
      H[h][1] = __builtin_amdgcn_alignbyte(it.qh[h].z, it.qh[h].y, r);
    }
    const uint32_t S[4] = {__builtin_amdgcn_alignbyte(it.sc4.y, it.sc4.x, r),
                           __builtin_amdgcn_alignbyte(it.sc4.z, it.sc4.y, r),
                           __builtin_amdgcn_alignbyte(it.sc4.w, it.sc4.z, r),
                           __builtin_amdgcn_alignbyte(it.sc1, it.sc4.w, r)};
    const uint32_t gb = (uint32_t)g >> 1;
    f4 accs[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) accs[q] = zero4;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int hh = t >> 2, qq = t & 3;
      const uint32_t *lq = L[2 * hh + (qq & 1)];
      const uint32_t *hq = H[hh];
      const int sh4 = 4 * (qq >> 1), sh2 = 2 * qq;
      const uint32_t q0 = ((lq[0] >> sh4) & 0x0F0F0F0Fu) | (((hq[0] >> sh2) & 0x03030303u) << 4);
      const uint32_t q1 = ((lq[1] >> sh4) & 0x0F0F0F0Fu) | (((hq[1] >> sh2) & 0x03030303u) << 4);
      const int sc = __builtin_amdgcn_sbfe((int)S[2 * hh + (qq >> 1)], 8u * (2u * (uint32_t)(qq & 1) + gb), 8u);
      const _Float16 sf = (_Float16)(float)sc;
      const h2 sc2 = {sf, sf};
      h2 p0, p1, p2, p3, l0, l1, l2, l3;
      q6_4(q0, sc2, p0, p1, l0, l1);
      q6_4(q1, sc2, p2, p3, l2, l3);
      const h8 bh = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      const h8 bl = {l0[0], l0[1], l1[0], l1[1], l2[0], l2[1], l3[0], l3[1]};
      const int ka = 128 * hh + 32 * qq + 8 * g;
#pragma unroll
      for (int q = 0; q < RG; ++q) {
        const h8 ah = *reinterpret_cast<const h8 *>(ar[q] + ka);
        accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, accs[q], 0, 0, 0);
        accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, accs[q], 0, 0, 0);
        if (kLo) {  // the x_lo * remainder term (below 2^-22 of the result) is left out, as in the tiled kernel
          const h8 al = *reinterpret_cast<const h8 *>(arl[q] + ka);
          accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, accs[q], 0, 0, 0);
        }
      }
    }
    const float dv = f16_bits_hw(kDw ? (it.sc1 >> (8u * r)) & 0xffffu : it.dw & 0xffffu);
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      const f4 s4 = *reinterpret_cast<const f4 *>(rsc + 16 * q);  // the rows' 2^s (exact products)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[q][v] = fmaf(dv * s4[v], accs[q][v], acc[q][v]);
    }
  }
};

using DecQ6K = DecQ6KT<false>;
using DecQ6KW = DecQ6KT<true>;

// Q8_0: an item is 256 weights of a column, eight 34-byte blocks (272 bytes,
// 2-byte aligned).  Lane group g covers blocks 2g and 2g + 1 (k = 64g ..
// 64g + 63); slice t (8 per item) is k = 64g + 8t + [0, 8), quants 8(t & 3) ..
// of block 2g + (t >> 2).  The lane reads its 68 bytes as an 18-dword window
// from the dword below them and realigns it; d is folded into two exact fp16
// B planes (q8_4), so the item needs no scaling afterwards.
struct DecQ80 {
  static constexpr uint32_t kBlk = 8 * kQ8Bytes;
  static constexpr int kType = kQ8_0;
  static constexpr bool kSums = false;
  static constexpr int kDepth = 2, kDepth1 = 3;
  struct Item {
    u32x4 w0, w1, w2, w3;
    u32x2 w4;
    uint32_t r;
  };
  __device__ static void load(Item &it, Rsrc rs, uint32_t blk, int g) {
    const uint32_t S = blk + 68u * (uint32_t)g, r = S & 3u, a = S - r;
    it.w0 = bload4(rs, a);
    it.w1 = bload4(rs, a + 16u);
    it.w2 = bload4(rs, a + 32u);
    it.w3 = bload4(rs, a + 48u);
    it.w4 = __builtin_amdgcn_raw_buffer_load_b64(rs, a + 64u, 0, 0);
    it.r = r;
  }
  template <bool kLo, int RG>
  __device__ static void contract(const Item &it, const _Float16 *const *ar, const _Float16 *const *arl,
                                  const _Float16 *const *, const float *rsc, int g, f4 *acc) {
    const uint32_t raw[18] = {it.w0.x, it.w0.y, it.w0.z, it.w0.w, it.w1.x, it.w1.y, it.w1.z, it.w1.w, it.w2.x,
                              it.w2.y, it.w2.z, it.w2.w, it.w3.x, it.w3.y, it.w3.z, it.w3.w, it.w4.x, it.w4.y};
    uint32_t w[17];  // bytes 4i .. 4i + 3 of the lane's 68 bytes
#pragma unroll
    for (int i = 0; i < 17; ++i) w[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], it.r);
    // block 2g: d in bytes 0-1, quants in bytes 2-33; block 2g + 1: d in bytes
    // 34-35, quants in bytes 36-67 (dword aligned)
    const _Float16 d0 = __builtin_bit_cast(_Float16, (uint16_t)(w[0] & 0xffffu));
    const _Float16 d1 = __builtin_bit_cast(_Float16, (uint16_t)(w[8] >> 16));
    const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f4 accs[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) accs[q] = zero4;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int blk = t >> 2, o = 2 * (t & 3);  // dword of the 8 quants within the block's quants
      const uint32_t qa = blk ? w[9 + o] : __builtin_amdgcn_alignbyte(w[o + 1], w[o], 2u);
      const uint32_t qb = blk ? w[10 + o] : __builtin_amdgcn_alignbyte(w[o + 2], w[o + 1], 2u);
      const _Float16 dh = blk ? d1 : d0;
      const h2 d2 = {dh, dh};
      h2 p0, p1, p2, p3, l0, l1, l2, l3;
      q8_4(qa, d2, p0, p1, l0, l1);
      q8_4(qb, d2, p2, p3, l2, l3);
      const h8 bh = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      const h8 bl = {l0[0], l0[1], l1[0], l1[1], l2[0], l2[1], l3[0], l3[1]};
      const int ka = 64 * g + 8 * t;
#pragma unroll
      for (int q = 0; q < RG; ++q) {
        const h8 ah = *reinterpret_cast<const h8 *>(ar[q] + ka);
        accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, accs[q], 0, 0, 0);
        accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, accs[q], 0, 0, 0);
        if (kLo) {  // the x_lo * remainder term (below 2^-22 of the result) is left out
          const h8 al = *reinterpret_cast<const h8 *>(arl[q] + ka);
          accs[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, accs[q], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      const f4 s4 = *reinterpret_cast<const f4 *>(rsc + 16 * q);  // the rows' 2^s (exact products)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[q][v] = fmaf(s4[v], accs[q][v], acc[q][v]);
    }
  }
};

// The activations arrive raw (f32 when kLo, else bf16): every workgroup
// converts its own K slice, so no pre-pass launch precedes the kernel.  Each
// row of the slice is scaled by 2^-s so its largest |x| lies in [512, 1024)
// (rows of zeros, infinities or NaNs keep s = 0), as the tiled kernel's
// pre-pass scales whole rows; the slice's outputs are multiplied back by 2^s
// (exact), so split-K partials leave the kernel unscaled and
// splitk_reduce_kernel only sums them in slice order and adds the bias.
// (Reducing in the kernel instead -- the last workgroup of a column group to
// count its arrival sums the partials -- measured 1.5-2x slower at the C5
// shapes than the separate reduction launch: with plain stores the
// device-scope release is an L2 write-back per workgroup; with write-through
// partials the last workgroup still reads every slice of its group alone, at
// one CU's bandwidth.)
//
// One launch may serve up to kDecMats matrices of one format and K that read
// the same activations (gate/up): their 16-column tiles are numbered
// consecutively (`DecMats`), and each tile finds its matrix from the tile
// boundaries and reads the matrix's record (weights, bias, output, sizes)
// with a wave-uniform scalar load.  Split-K partials are laid out
// over the concatenated tile columns, [ksplit][M][ntiles * 16].
// Index arithmetic stays off the scalar ALU, which one CU's 16 waves share:
// the grid is (column group, K slice), the host passes the slice partition
// (slice z holds base + (z < rem) super-blocks) and the power of two kw as a
// shift, and the ring walks its items with counters instead of divisions.
// The body of one decode-batch workgroup for format F: column group grp of
// `groups` over the tiles [tbase, tbase + ntl) of the launch (one format's
// tiles; `ntiles` counts every tile of the launch, the partials' width).
template <class F, bool kLo, int RG, bool kW>
__device__ __forceinline__ void dec_run(const void *__restrict__ X, const DecMats &mats, int ntiles, int M, int K,
                                        int sl_base, int sl_rem, int kw_shift_arg, float *__restrict__ part,
                                        int grp, int groups, int tbase, int ntl) {
  // kW: an in-workgroup K split (unsplit K across workgroups, one 16-row group)
  const int kw_shift = kW ? kw_shift_arg : 0, kw = 1 << kw_shift;
  const int ksplit = (int)gridDim.y;
  constexpr int D = RG == 1 ? F::kDepth1 : F::kDepth;
  extern __shared__ __align__(16) unsigned char dsm[];
  constexpr int nt = kDecWaves * 64;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int z = (int)blockIdx.y;
  const int nsb_all = (int)((uint32_t)K >> 8);
  const int sb0 = z * sl_base + (z < sl_rem ? z : sl_rem);
  const int nsbs = sl_base + (z < sl_rem ? 1 : 0);
  const int Ks = nsbs * 256, P = Ks + 8;  // slice width, LDS row pitch (halves)
  // LDS: Ah and Al (kLo) of M rows at dec_row(r, P), xs [nsbs][M][16] (a
  // row's 32-byte records of consecutive rows adjacent: the 32 lanes reading
  // them hit 32 distinct 16-byte bank groups); with kw > 1 the same bytes
  // hold the waves' partial tiles once the activations are consumed
  _Float16 *Ah = reinterpret_cast<_Float16 *>(dsm);
  _Float16 *Al = Ah + (size_t)M * P + kDecRowExtra;
  _Float16 *Xs = Ah + ((size_t)M * P + kDecRowExtra) * (kLo ? 2 : 1);
  // unsplit K: the bias of every wave's tiles (tile ti of wave w at
  // [ti][16 w .. 16 w + 15]); the power-of-two scale of every (super-block,
  // row) of the slice
  float *Bs = reinterpret_cast<float *>(dsm + dec_tail_offset(M, P, nsbs, kLo ? 2 : 1, kW, RG));  // [kDecMaxTiles][256]
  float *Rsb = Bs + kDecMaxTiles * 256;  // [nsbs][kDecRows]: the 2^s of each (super-block, row)
  // bit r: row r of the slice holds an infinity or a NaN
  uint32_t *Dbad = reinterpret_cast<uint32_t *>(Rsb + nsbs * kDecRows);

  // 1. this wave's items.  The kDecWaves waves form T = kDecWaves / kw tile
  //    slots of kw waves each.  Column group grp owns a contiguous block of
  //    the tiles, the blocks balanced to within one tile (so no CU holds a
  //    round more than another); slot ts's tile of round ti is tile
  //    ti * T + ts of the block, and wave kp of the slot takes the slice's
  //    super-blocks kp, kp + kw, ... (kw > 1 only with unsplit K: the slot's
  //    waves then sum their partial tiles through LDS at the end).  Item
  //    (ti, jj) is round ti's super-block kp + kw jj, jj < cnt.  Tile numbers
  //    are local to the workgroup's format (tiles [tbase, tbase + ntl) of the
  //    launch); gtile() gives the launch's tile number (matrix, partials).
  // (all wave-uniform: readfirstlane keeps them, and the matrix records and
  // weight descriptors built from them, in scalar registers -- a descriptor
  // the compiler takes for divergent costs a waterfall loop per load)
  static_assert(kDecWaves == 16, "T = 16 >> kw_shift");
  const int T = kDecWaves >> kw_shift, ts = wave >> kw_shift, kp = wave & (kw - 1);
  const int qg = __builtin_amdgcn_readfirstlane(ntl / groups), rg = ntl - qg * groups;
  const int t0g = grp * qg + (grp < rg ? grp : rg), ntg = qg + (grp < rg ? 1 : 0);  // the group's block
  const int cnt = __builtin_amdgcn_readfirstlane(nsbs > kp ? (nsbs - kp + kw - 1) >> kw_shift : 0);  // items per tile
  const int mytiles =
      __builtin_amdgcn_readfirstlane(ts < ntg && cnt > 0 ? (ntg - ts + T - 1) >> (4 - kw_shift) : 0);
  // the local tile of round ti (wave-uniform)
  auto ltile = [&](int ti) { return __builtin_amdgcn_readfirstlane(t0g + ti * T + ts); };
  // a local tile's launch tile (tiles past the end: the format's last one)
  auto gtile = [&](int t) { return tbase + (t < ntl ? t : ntl - 1); };
  const int nitems = mytiles * cnt;
  const int cn = lane & 15, g = lane >> 4;
  const uint32_t row_bytes = (uint32_t)nsb_all * F::kBlk;
  // the matrix of a tile (tiles past the end map to the last matrix): the
  // tile boundaries stay in SGPRs (t >= st as the sign of st - 1 - t: shifts,
  // not compares and selects), the matrix's record is a scalar load
  const int st1 = mats.tile0[1], st2 = mats.tile0[2], st3 = mats.tile0[3];
  auto ge = [](int t, int st) { return (int)((uint32_t)(st - 1 - t) >> 31); };
  auto mat_of = [&](int t) { return ge(t, st1) + ge(t, st2) + ge(t, st3); };
  // A rows of the lane's row groups.  Lanes whose 16-row group reaches past
  // M read row M - 1: they only produce MFMA output rows >= M, which are
  // never stored, so no zero row needs staging.
  int arow[RG];
#pragma unroll
  for (int q = 0; q < RG; ++q) arow[q] = (lane & 15) + 16 * q < M ? (lane & 15) + 16 * q : M - 1;

  using Item = typename F::Item;
  // item positions advance by counters: (ti, jj) -> next item
  auto advance = [&](int &ti, int &jj) {
    const bool wrap = jj + 1 == cnt;
    jj = wrap ? 0 : jj + 1;
    ti += wrap ? 1 : 0;
  };
  // The weights of the wave's tile of round ti: the matrix's descriptor and
  // this lane's byte offset of its column's first super-block of the slice.
  // Rows past the matrix (and rounds past the wave's tiles) read past the tensor:
  // zeros.  Set once per tile, so an item's load costs one address add.
  struct WTile {
    Rsrc rs;
    uint32_t base;
  };
  auto wtile = [&](int ti) {
    const int lt = ltile(ti), tile = gtile(lt), m = mat_of(tile);
    const DecMat &mt = mats.mat[m];
    const uint32_t n = (uint32_t)((tile - mt.tile0) * 16 + cn);
    WTile wt;
    wt.rs = make_rsrc(mt.w, mt.w_bytes);
    wt.base = ti < mytiles ? n * row_bytes + (uint32_t)sb0 * F::kBlk : mt.w_bytes;
    return wt;
  };
  WTile lw = wtile(0);
  int l_ti = 0, l_jj = 0;  // the next item to load
  auto load_next = [&](Item &it) {
    F::load(it, lw.rs, lw.base + (uint32_t)(kp + (l_jj << kw_shift)) * F::kBlk, g);
    if (++l_jj == cnt) {
      l_jj = 0;
      lw = wtile(++l_ti);
    }
  };
  // 2. the activations of the slice: this thread's pieces of 8 consecutive
  //    activations of one row (at most kDecStage; pieces past the last row
  //    read past x and are not stored) are loaded first, then the first D items'
  //    weights; the conversion waits for the activations only (the
  //    vector-memory counter completes in order) and the weights stay in
  //    flight across the barriers.
  const int pr = Ks / 8;  // pieces per row
  const uint32_t x_end = (uint32_t)((size_t)M * K * (kLo ? 4 : 2));
  const Rsrc rs_x = make_rsrc(X, x_end);
  // piece i of this thread is piece tid + i * nt of the slice: row pc_r[i],
  // piece pc_c[i] of the row (one division per thread; each step adds
  // divmod(nt, pr) with a carry)
  int pc_r[kDecStage], pc_c[kDecStage];
  {
    const int dq = nt / pr, dr = nt - dq * pr;
    int r = tid / pr, c = tid - r * pr;
#pragma unroll
    for (int i = 0; i < kDecStage; ++i) {
      pc_r[i] = r;
      pc_c[i] = c;
      c += dr;
      r += dq + (c >= pr ? 1 : 0);
      c -= c >= pr ? pr : 0;
    }
  }
  u32x4 xa[kDecStage], xb[kLo ? kDecStage : 1];  // f32: 2 x 4 values; bf16: 8 values
#pragma unroll
  for (int i = 0; i < kDecStage; ++i) {
    const int r = pc_r[i], c = pc_c[i];
    const uint32_t e = (uint32_t)r * (uint32_t)K + (uint32_t)sb0 * 256u + 8u * (uint32_t)c;  // first activation
    if (kLo) {
      xa[i] = bload4(rs_x, r < M ? e * 4u : x_end);
      xb[i] = bload4(rs_x, r < M ? e * 4u + 16u : x_end);
    } else {
      xa[i] = bload4(rs_x, r < M ? e * 2u : x_end);
    }
  }
  // bias of the wave's tiles (unsplit K only; split K adds it in the
  // reduction): lanes 0-15 of each wave load the 16 values of its tile ti
  uint32_t bbits[kDecMaxTiles] = {};
  if (ksplit == 1) {
#pragma unroll
    for (int ti = 0; ti < kDecMaxTiles; ++ti) {
      const int lt = ltile(ti), tile = gtile(lt), m = mat_of(tile);
      const DecMat &mt = mats.mat[m];
      // columns past the matrix fall past bias_bytes: the range check reads 0
      const uint32_t col = (uint32_t)((tile - mt.tile0) * 16 + lane);
      bbits[ti] = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(mt.bias, mt.bias_bytes),
                                                       lane < 16 && ti < mytiles ? col * 4u : mt.bias_bytes, 0, 0);
    }
  }
  // the non-finite row mask starts empty (written before the barrier below,
  // and waited for, so that no wave's staging can set a bit ahead of it)
  if (tid == 0) {
    *Dbad = 0u;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  }
  // A CU returns vector loads in issue order: this bare barrier (no memory
  // fence) puts every activation load of the workgroup ahead of every weight
  // load, so no wave's activations queue behind another wave's weights.
  __builtin_amdgcn_s_barrier();
  // The weights go out once the wave's first activations have arrived (after
  // its first piece below), so that the rest of the conversion overlaps their
  // latency; issued before that, they delay the activations themselves.  With
  // two 16-row groups only waves with more than D items do so (measured: the
  // 1-2 item waves of the small projections lose more to the weights
  // competing with their staging than they gain); theirs go out after the
  // staging.  The closing barrier itself waits for LDS only, but with the
  // issue a per-wave choice the compiler's wait counts after it hold on
  // both paths: an early wave's last piece waits for its weights too (exact
  // counts, from issuing on every wave, measured no faster).
  const bool early = RG == 1 || nitems > D;
  Item S[D];
  if (ksplit == 1 && lane < 16) {
#pragma unroll
    for (int ti = 0; ti < kDecMaxTiles; ++ti) Bs[ti * 256 + wave * 16 + lane] = __uint_as_float(bbits[ti]);
  }
  auto piece = [&](int i, float v[8]) {
    if (kLo) {
      v[0] = as_f32(xa[i].x), v[1] = as_f32(xa[i].y), v[2] = as_f32(xa[i].z), v[3] = as_f32(xa[i].w);
      v[4] = as_f32(xb[i].x), v[5] = as_f32(xb[i].y), v[6] = as_f32(xb[i].z), v[7] = as_f32(xb[i].w);
    } else {
      v[0] = bf16_lo(xa[i].x), v[1] = bf16_hi(xa[i].x), v[2] = bf16_lo(xa[i].y), v[3] = bf16_hi(xa[i].y);
      v[4] = bf16_lo(xa[i].z), v[5] = bf16_hi(xa[i].z), v[6] = bf16_lo(xa[i].w), v[7] = bf16_hi(xa[i].w);
    }
  };
  // Scaled fp16 planes and per-32 sums, one pass: each (row, super-block) of
  // the slice is scaled by its own 2^-s (its largest |x| into [512, 1024);
  // zero, inf and NaN blocks keep s = 0), applied back in f32 with the
  // super-block's d.  The 32 pieces of lanes 0-31 (32-63) are one row's
  // super-block (pieces per row are a multiple of 32), so its max is a
  // half-wave reduction: DPP within each 16-lane row, readlane across the
  // two.  Pieces past the last row are skipped (a uniform bound).
  auto umax_u32 = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
  auto dmax = [&](uint32_t a, auto ctl) {
    return umax_u32(a, dpp_row_u<decltype(ctl)::value>(a));
  };
#pragma unroll
  for (int i = 0; i < kDecStage; ++i) {
    if (i * nt >= M * pr) break;
    const int r = pc_r[i], c = pc_c[i];
    float v[8];
    piece(i, v);
    // the largest |x| as the largest magnitude bit pattern: for |x| the
    // unsigned order is the float order, with NaN above infinity above every
    // finite value (a float max would drop NaNs)
    uint32_t a = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) a = umax_u32(a, as_u32(v[e]) & 0x7fffffffu);
    a = dmax(a, std::integral_constant<int, 0xB1>{});   // quad_perm 1,0,3,2
    a = dmax(a, std::integral_constant<int, 0x4E>{});   // quad_perm 2,3,0,1
    a = dmax(a, std::integral_constant<int, 0x141>{});  // row_half_mirror
    a = dmax(a, std::integral_constant<int, 0x140>{});  // row_mirror
    const uint32_t h0 = umax_u32((uint32_t)__builtin_amdgcn_readlane((int)a, 0), (uint32_t)__builtin_amdgcn_readlane((int)a, 16));
    const uint32_t h1 = umax_u32((uint32_t)__builtin_amdgcn_readlane((int)a, 32), (uint32_t)__builtin_amdgcn_readlane((int)a, 48));
    const uint32_t abits = lane < 32 ? h0 : h1;
    const bool nonfin = abits >= 0x7f800000u;  // the block holds an infinity or a NaN
    const float amax = as_f32(abits);
    const int sx = (amax > 0.0f && !nonfin) ? __builtin_amdgcn_frexp_expf(amax) - 10 : 0;
    // hi = fp16 of w = x * 2^-sx rounded to nearest, lo = fp16 of the exact
    // residue w - hi (rounded to nearest once), so hi + lo = w to 2^-22
    // relative.  Sums (Q4_K): the 8 values of a piece in order, then the 4
    // pieces of a run (4 consecutive lanes) through DPP.  Fast path (every
    // block of the wave has |sx| <= 100, so 2^-sx is a normal f32 and the raw
    // values and their sums stay far from overflow): one v_fma_mix per fp16
    // value, and the sum taken on the raw values and then scaled (a power of
    // two, exact).  Otherwise v_ldexp on every value.
    h8 hv, lv;
    float t = 0.0f;
    if (__builtin_amdgcn_ballot_w64(sx < -100 || sx > 100) == 0) {
      const float sc = ldexpf(1.0f, -sx);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (F::kSums) t += v[e];
        const _Float16 h = (_Float16)(v[e] * sc);
        hv[e] = h;
        if (kLo) lv[e] = (_Float16)__builtin_fmaf(v[e], sc, -(float)h);
      }
      if (F::kSums) t *= sc;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float w = ldexpf(v[e], -sx);
        if (F::kSums) t += w;
        const _Float16 h = (_Float16)w;
        hv[e] = h;
        if (kLo) lv[e] = (_Float16)(w - (float)h);
      }
    }
    if (F::kSums) {
      t += dpp_row_f<0xB1>(t);  // quad_perm 1,0,3,2
      t += dpp_row_f<0x4E>(t);  // quad_perm 2,3,0,1
    }
    if (r < M) {
      *reinterpret_cast<h8 *>(Ah + dec_row(r, P) + 8 * c) = hv;
      if (kLo) *reinterpret_cast<h8 *>(Al + dec_row(r, P) + 8 * c) = lv;
      if (F::kSums && (c & 3) == 0) {
        const _Float16 sh = (_Float16)t;
        h2 pair;
        pair[0] = sh;
        pair[1] = (_Float16)(t - (float)sh);
        *reinterpret_cast<h2 *>(Xs + ((size_t)(c >> 5) * M + r) * 16 + 2 * ((c >> 2) & 7)) = pair;
      }
      // a NaN scale marks a block holding an infinity or a NaN: the row's
      // outputs of this slice are recomputed in IEEE f32 at the end
      if ((c & 31) == 0) {
        Rsb[(c >> 5) * kDecRows + r] = nonfin ? __builtin_nanf("") : ldexpf(1.0f, sx);
        if (nonfin) atomicOr(Dbad, 1u << r);
      }
    }
    if (early && i == 0) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < D; ++j) load_next(S[j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  lds_barrier();
  if (!early) {
#pragma unroll
    for (int j = 0; j < D; ++j) load_next(S[j]);
  }

  const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[RG];
#pragma unroll
  for (int q = 0; q < RG; ++q) acc[q] = zero4;
  // outputs: range-checked buffer stores (out-of-range lanes are dropped by
  // the hardware, so no branch surrounds them), scale and bias from LDS
  const int ncat = ntiles * 16;  // partial columns: the concatenated tiles
  const uint32_t part_end = (uint32_t)((size_t)ksplit * M * ncat * 4);
  const Rsrc rs_part = make_rsrc(part, part_end);
  // a finished tile (round ti of this wave's slot): scaled back by the rows'
  // 2^s, plus the bias (unsplit K), or the raw partial of slice z
  auto store = [&](int ti, const f4 *vals) {
    const int tile = gtile(ltile(ti)), m = mat_of(tile);
    const DecMat &mt = mats.mat[m];
    const int nm = mt.n, col = (tile - mt.tile0) * 16 + cn;
    const float bv = ksplit == 1 ? Bs[(ti < kDecMaxTiles ? ti : 0) * 256 + wave * 16 + cn] : 0.0f;
    // unsplit: the matrix's own output; split: the concatenated partials
    const uint32_t out_end = ksplit > 1 ? part_end : (uint32_t)((size_t)M * nm * 4);
    const Rsrc rs_out = ksplit > 1 ? rs_part : make_rsrc(mt.y, out_end);
    // element offsets in 32 bits (both ranges are below 4 GiB), selected
    // rather than branched on: row 4g + v of row group q is base + (16q + v)
    // * pitch; lanes past the matrix's rows or columns store to out_end
    const uint32_t pitch = ksplit > 1 ? (uint32_t)ncat : (uint32_t)nm;
    const uint32_t base = ksplit > 1 ? ((uint32_t)z * (uint32_t)M + 4u * (uint32_t)g) * (uint32_t)ncat +
                                           (uint32_t)tile * 16u + (uint32_t)cn
                                     : 4u * (uint32_t)g * (uint32_t)nm + (uint32_t)col;
    const bool col_ok = col < nm;
#pragma unroll
    for (int q = 0; q < RG; ++q) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * q + 4 * g + v;
        const float val = vals[q][v] + bv;  // rows >= M: the range check drops their stores
        const uint32_t e = base + (uint32_t)(16 * q + v) * pitch;
        const uint32_t off = col_ok && row < M ? e * 4u : out_end;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), rs_out, off, 0, 0);
      }
    }
  };
  auto consume = [&](const Item &it, int ti, int jj) {
    const int sbl = kp + (jj << kw_shift);
    const _Float16 *ar[RG], *arl[RG], *xs[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      ar[q] = Ah + dec_row(arow[q], P) + sbl * 256;
      arl[q] = Al + dec_row(arow[q], P) + sbl * 256;
      xs[q] = Xs + ((size_t)sbl * M + arow[q]) * 16;
    }
    F::template contract<kLo, RG>(it, ar, arl, xs, Rsb + sbl * kDecRows + 4 * g, g, acc);
    // the tile's last super-block: write it out (kw > 1: a slot has at most
    // one tile, and acc keeps this wave's part of it for the LDS sum below)
    if (jj == cnt - 1 && kw == 1) {
      store(ti, acc);
#pragma unroll
      for (int q = 0; q < RG; ++q) acc[q] = zero4;
    }
  };

  // Rows of this slice holding an infinity or a NaN (Dbad) get the IEEE f32
  // value of their products over the slice instead of the MFMA result, which
  // contracts sc * q and the min term apart (an infinity meets a zero part:
  // NaN, where the reference multiplies it by a non-zero weight).  Only the
  // non-finite activations decide it: the sum of x_k * W[col, k] over them,
  // weights dequantised exactly; split K: this slice's partial (the
  // reduction's f32 sum of slices keeps IEEE semantics), unsplit: plus the
  // bias.  Rare inputs: one lane per (row, column), a plain loop.
  auto ieee_fix = [&](int ti, uint32_t bad) {
    const int tile = gtile(ltile(ti)), m = mat_of(tile);
    const DecMat &mt = mats.mat[m];
    const int nm = mt.n, col = (tile - mt.tile0) * 16 + cn;
    if (col >= nm) return;
    const uint8_t *wrow = mt.w + (size_t)col * row_bytes;
    const int k0 = sb0 * 256, k1 = (sb0 + nsbs) * 256;
    for (int q = 0; q < RG; ++q)
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * q + 4 * g + v;
        if (row >= M || !((bad >> row) & 1u)) continue;
        float t = 0.0f;
        for (int k = k0; k < k1; ++k) {
          const float xv = x_at<kLo>(X, (int64_t)row * K + k);
          if (non_finite(xv)) t = __fadd_rn(t, __fmul_rn(xv, deq_elem(F::kType, wrow, (uint32_t)k)));
        }
        if (ksplit > 1)
          part[((size_t)z * M + row) * (size_t)ncat + (size_t)tile * 16 + cn] = t;
        else
          mt.y[(size_t)row * nm + col] = __fadd_rn(t, mt.bias ? mt.bias[col] : 0.0f);
      }
  };

  // 3. the ring: consume slot j, refill it D items ahead; loads stay
  //    unconditional (items past the end read past the tensor: zeros).
  int c_ti = 0, c_jj = 0;  // the next item to consume
  int u0 = 0;
  for (; u0 + D < nitems; u0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      consume(S[j], c_ti, c_jj);
      advance(c_ti, c_jj);
      load_next(S[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j)
    if (u0 + j < nitems) {
      consume(S[j], c_ti, c_jj);
      advance(c_ti, c_jj);
    }
  if constexpr (!kW) {
    const uint32_t bad = *Dbad;  // set during the staging, before its barrier
    if (bad != 0u)
      for (int ti = 0; ti < mytiles; ++ti) ieee_fix(ti, bad);
    return;
  }
  // 4. kw > 1: the kw waves of each slot hold partial sums of its one tile
  //    over disjoint super-blocks.  Once every wave is past the activations,
  //    their LDS holds the partials [wave][RG][lane][4]; the slot's first
  //    wave sums them in wave order (a fixed order: deterministic) and writes
  //    the tile.
  __syncthreads();
  f4 *Red = reinterpret_cast<f4 *>(dsm);
  if (mytiles > 0) {
#pragma unroll
    for (int q = 0; q < RG; ++q) Red[(wave * RG + q) * 64 + lane] = acc[q];
  }
  __syncthreads();
  if (kp != 0 || mytiles == 0) return;
  for (int k2 = 1; k2 < kw; ++k2)
#pragma unroll
    for (int q = 0; q < RG; ++q) acc[q] += Red[((wave + k2) * RG + q) * 64 + lane];
  store(0, acc);
  const uint32_t bad = *Dbad;
  if (bad != 0u) ieee_fix(0, bad);
}

// One format (F1 == F2: every workgroup) or two: workgroups below g_split run
// F1 over the launch's first nt1 tiles (its first matrices), the rest run F2
// over the others.  Both read the same activations; the split-K partials of
// both go to one array over the concatenated tiles.
template <class F1, class F2, bool kLo, int RG, bool kW>
__global__ __launch_bounds__(kDecWaves * 64) void gemm_decode_kernel(const void *__restrict__ X_arg, DecMats mats,
                                                                     int ntiles_arg, int M_arg, int K_arg,
                                                                     int sl_base_arg, int sl_rem_arg,
                                                                     int kw_shift_arg, float *__restrict__ part_arg,
                                                                     int g_split_arg, int nt1_arg) {
  // every argument in scalar registers up front (one batch of argument loads)
  const void *const X = sarg(X_arg);
  float *const part = sarg(part_arg);
  const int ntiles = sarg(ntiles_arg), M = sarg(M_arg), K = sarg(K_arg);
  const int sl_base = sarg(sl_base_arg), sl_rem = sarg(sl_rem_arg);
  const int kw_shift = kW ? sarg(kw_shift_arg) : 0;
  const int b = (int)blockIdx.x, groups = (int)gridDim.x;
  if constexpr (std::is_same<F1, F2>::value) {
    dec_run<F1, kLo, RG, kW>(X, mats, ntiles, M, K, sl_base, sl_rem, kw_shift, part, b, groups, 0, ntiles);
  } else {
    const int g_split = sarg(g_split_arg), nt1 = sarg(nt1_arg);
    if (b < g_split)
      dec_run<F1, kLo, RG, kW>(X, mats, ntiles, M, K, sl_base, sl_rem, kw_shift, part, b, g_split, 0, nt1);
    else
      dec_run<F2, kLo, RG, kW>(X, mats, ntiles, M, K, sl_base, sl_rem, kw_shift, part, b - g_split, groups - g_split,
                               nt1, ntiles - nt1);
  }
}

// Sum of the split-K partials in slice order (deterministic), then the row
// scale (tiled kernel; the decode-batch kernel's partials are unscaled:
// rscale == nullptr) and the bias: Y[m, n] = (sum_z P[z][m, n]) * rscale[m] + bias[n].
// Grid: 256-column blocks x rows (a row stride of gridDim.y beyond 65535
// rows), so no thread divides its index.  The partials are read through a
// range-checked buffer resource with 32-bit offsets (K is split only for
// output grids under 3/4 of the CUs' tiles: at most 8 slices of a few
// million floats), KB slices per batch, the split rounded up to 2, 4 or 8,
// slices past it pointed at the end, where they read zeros without a branch.
template <int KB>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ part, int ksplit, int M, int N,
                                                            const float *__restrict__ rscale,
                                                            const float *__restrict__ bias, float *__restrict__ Y) {
  const int n = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (n >= N) return;
  const uint32_t total = (uint32_t)M * (uint32_t)N, end = (uint32_t)ksplit * total * 4u;
  const Rsrc rs = make_rsrc(part, end);
  const float bn = bias ? bias[n] : 0.0f;
  for (int m = (int)blockIdx.y; m < M; m += (int)gridDim.y) {
    const float rs_m = rscale ? rscale[m] : 1.0f;
    if (__builtin_isnan(rs_m)) continue;  // the pre-pass wrote this row's IEEE outputs
    const uint32_t i = (uint32_t)m * (uint32_t)N + (uint32_t)n;
    // every slice's load of a batch in flight at once; the sum runs in slice
    // order from -0.0 (x + -0.0 == x, so p0 + p1 + ...; the zeros past the
    // split change no sum but an exact -0, which the bias term below turns
    // into +0 either way)
    float acc = -0.0f;
    for (int z0 = 0; z0 < ksplit; z0 += KB) {
      float v[KB];
#pragma unroll
      for (int d = 0; d < KB; ++d) {
        const uint32_t off = z0 + d < ksplit ? ((uint32_t)(z0 + d) * total + i) * 4u : end;
        v[d] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
      }
#pragma unroll
      for (int d = 0; d < KB; ++d) acc += v[d];
    }
    Y[(size_t)i] = __builtin_fmaf(acc, rs_m, bn);  // rs_m a power of two: the product is exact
  }
}

// The same sums, four consecutive outputs and RR rows per thread (N a
// multiple of 4, Y 16-byte aligned: every partial and output row holds whole
// 16-byte pieces): each slice's 16-byte loads of all RR rows in flight at
// once, a quarter of the threads and an RR-th of the workgroups of
// splitk_reduce_kernel.  Per output the same operations in the same order:
// the slice-order sum from -0.0, then acc * rscale + bias as one FMA (the
// power-of-two scale makes the product exact, so this is the rounding of
// the separate multiply and add).  Grid: 1024-column blocks x RR-row blocks.
constexpr int kReduceRows = 2;  // rows per thread of splitk_reduce4_kernel
template <int KB, int RR>
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(const float *__restrict__ part, int ksplit, int M, int N,
                                                             const float *__restrict__ rscale,
                                                             const float *__restrict__ bias, float *__restrict__ Y) {
  const int n = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 4;
  if (n >= N) return;
  const uint32_t total = (uint32_t)M * (uint32_t)N, end = (uint32_t)ksplit * total * 4u;
  const Rsrc rs = make_rsrc(part, end);
  const int m0 = (int)blockIdx.y * RR;
  f4 acc[RR];
#pragma unroll
  for (int r = 0; r < RR; ++r) acc[r] = f4{-0.0f, -0.0f, -0.0f, -0.0f};
  for (int z0 = 0; z0 < ksplit; z0 += KB) {
    u32x4 v[RR][KB];
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
      for (int d = 0; d < KB; ++d) {
        const uint32_t i = (uint32_t)(m0 + r) * (uint32_t)N + (uint32_t)n;
        const bool in = z0 + d < ksplit && m0 + r < M;
        v[r][d] = bload4(rs, in ? ((uint32_t)(z0 + d) * total + i) * 4u : end);
      }
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
      for (int d = 0; d < KB; ++d) {
        acc[r].x += __uint_as_float(v[r][d].x);
        acc[r].y += __uint_as_float(v[r][d].y);
        acc[r].z += __uint_as_float(v[r][d].z);
        acc[r].w += __uint_as_float(v[r][d].w);
      }
  }
  const float b0 = bias ? bias[n] : 0.0f, b1 = bias ? bias[n + 1] : 0.0f;
  const float b2 = bias ? bias[n + 2] : 0.0f, b3 = bias ? bias[n + 3] : 0.0f;
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    const int m = m0 + r;
    if (m >= M) break;
    const float s = rscale ? rscale[m] : 1.0f;
    if (__builtin_isnan(s)) continue;  // the pre-pass wrote this row's IEEE outputs
    f4 o;
    o.x = __builtin_fmaf(acc[r].x, s, b0);
    o.y = __builtin_fmaf(acc[r].y, s, b1);
    o.z = __builtin_fmaf(acc[r].z, s, b2);
    o.w = __builtin_fmaf(acc[r].w, s, b3);
    *reinterpret_cast<f4 *>(Y + (size_t)m * N + n) = o;
  }
}

// The decode-batch kernel's partials [ksplit][M][ntiles * 16] over the
// concatenated tiles of its matrices: the same slice-order sum, scattered to
// each matrix's output with its bias (columns past a matrix's rows skipped).
// Grid: 256-column blocks x rows, so no thread divides its index; the
// partials are read through a range-checked buffer resource with 32-bit
// offsets (the decode-batch kernel addresses them so too), slices past
// ksplit pointed at its end, where they read zeros without a branch.  KB:
// the slices loaded per batch, the split rounded up to 4, 8 or 16.
template <int KB>
__global__ __launch_bounds__(256) void splitk_reduce_mats_kernel(const float *__restrict__ part, int ksplit, int M,
                                                                 int ntiles, DecMats mats) {
  const int ncat = ntiles * 16;
  const int cc = (int)blockIdx.x * 256 + (int)threadIdx.x, row = (int)blockIdx.y, tile = cc >> 4;
  if (cc >= ncat) return;
  const int st1 = sarg(mats.tile0[1]), st2 = sarg(mats.tile0[2]), st3 = sarg(mats.tile0[3]);
  const int mn0 = sarg(mats.mat[0].n), mn1 = sarg(mats.mat[1].n), mn2 = sarg(mats.mat[2].n), mn3 = sarg(mats.mat[3].n);
  const int m = (int)(tile >= st1) + (int)(tile >= st2) + (int)(tile >= st3);
  const int t0 = m == 0 ? 0 : m == 1 ? st1 : m == 2 ? st2 : st3;
  const int nm = m == 0 ? mn0 : m == 1 ? mn1 : m == 2 ? mn2 : mn3;
  const int col = (tile - t0) * 16 + (cc & 15);
  if (col >= nm) return;
  // every slice's load in flight at once (one memory round trip for up to
  // 16 slices), then the sum in slice order from -0.0, as splitk_reduce_kernel
  // (the zeros past ksplit change no sum but an exact -0, which the bias
  // term below turns into +0 either way)
  const uint32_t slice = (uint32_t)M * (uint32_t)ncat, end = (uint32_t)ksplit * slice * 4u;
  const Rsrc rs = make_rsrc(part, end);
  const uint32_t i = (uint32_t)row * (uint32_t)ncat + (uint32_t)cc;
  float acc = -0.0f;
  for (int z0 = 0; z0 < ksplit; z0 += KB) {
    float v[KB];
#pragma unroll
    for (int d = 0; d < KB; ++d) {
      const uint32_t off = z0 + d < ksplit ? ((uint32_t)(z0 + d) * slice + i) * 4u : end;
      v[d] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
    }
#pragma unroll
    for (int d = 0; d < KB; ++d) acc += v[d];
  }
  float *const y0 = sarg(mats.mat[0].y), *const y1 = sarg(mats.mat[1].y), *const y2 = sarg(mats.mat[2].y),
              *const y3 = sarg(mats.mat[3].y);
  const float *const b0 = sarg(mats.mat[0].bias), *const b1 = sarg(mats.mat[1].bias),
              *const b2 = sarg(mats.mat[2].bias), *const b3 = sarg(mats.mat[3].bias);
  float *ym = m == 0 ? y0 : m == 1 ? y1 : m == 2 ? y2 : y3;
  const float *bm = m == 0 ? b0 : m == 1 ? b1 : m == 2 ? b2 : b3;
  ym[(size_t)row * nm + col] = acc + (bm ? bm[col] : 0.0f);
}

// The gate/up pair of a gated-SiLU MLP in one decode-batch launch (matrix 0
// gate, matrix 1 up, the same rows): each thread reduces one output of both,
// in slice order from -0.0 as splitk_reduce_mats_kernel does, and leaves the
// reference MLP's buffers (crates/kernels/src/mlp.rs:77-88, :233-238): up(x)
// in up's output and silu(gate(x)) * up(x) in gate's, with the standalone
// swiglu kernel's operations in its order (both files build with the same
// flags), one launch and one round trip fewer.  Grid, offsets and batches
// as splitk_reduce_mats_kernel.
template <int KB>
__global__ __launch_bounds__(256) void splitk_reduce_swiglu_kernel(const float *__restrict__ part, int ksplit, int M,
                                                                   int ntiles, DecMats mats) {
  const int n = sarg(mats.mat[0].n);
  const int col = (int)blockIdx.x * 256 + (int)threadIdx.x, row = (int)blockIdx.y;
  if (col >= n) return;
  const uint32_t ncat = (uint32_t)ntiles * 16u, slice = (uint32_t)M * ncat, end = (uint32_t)ksplit * slice * 4u;
  const Rsrc rs = make_rsrc(part, end);
  const uint32_t ig = (uint32_t)row * ncat + (uint32_t)col, iu = ig + (uint32_t)sarg(mats.tile0[1]) * 16u;
  float g = -0.0f, u = -0.0f;
  for (int z0 = 0; z0 < ksplit; z0 += KB) {
    float vg[KB], vu[KB];
#pragma unroll
    for (int d = 0; d < KB; ++d) {
      const bool in = z0 + d < ksplit;
      const uint32_t zo = (uint32_t)(z0 + d) * slice;
      vg[d] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, in ? (zo + ig) * 4u : end, 0, 0));
      vu[d] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, in ? (zo + iu) * 4u : end, 0, 0));
    }
#pragma unroll
    for (int d = 0; d < KB; ++d) g += vg[d], u += vu[d];  // zeros past the split: see splitk_reduce_mats_kernel
  }
  const float *const bg = sarg(mats.mat[0].bias), *const bu = sarg(mats.mat[1].bias);
  g = g + (bg ? bg[col] : 0.0f);
  u = u + (bu ? bu[col] : 0.0f);
  float *const yg = sarg(mats.mat[0].y), *const yu = sarg(mats.mat[1].y);
  yu[(size_t)row * n + col] = u;
  const float sig = 1.0f / (1.0f + expf(-g));
  yg[(size_t)row * n + col] = (g * sig) * u;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool gemm_supported(int type, int64_t M, int64_t K, int64_t N) {
  // 32-bit buffer offsets: activations (with a tile of padding rows) and weights
  const int64_t a_bytes = (M + 256) * K * 2;
  const int64_t sb_bytes = sb_bytes_of(type);
  const int64_t w_bytes = (N + kBN) * (K / 256) * sb_bytes + 1024;
  return (type == kQ4_K || type == kQ5_K || type == kQ6_K || type == kQ8_0) && K % 256 == 0 && N >= 1 && M >= 1 &&
         a_bytes < (int64_t)UINT32_MAX && w_bytes < (int64_t)UINT32_MAX;
}

GemmPlan gemm_plan(int type, int64_t M, int64_t N, int64_t K, bool x_is_bf16, int cu_count) {
  GemmPlan p{};
  p.kwaves = 1;
  // More than 32 rows: Q4_K, Q5_K and Q8_0 with bf16 activations take the
  // register-dequant kernels (okq_gemm_wide.hip, okq_gemm_pair.hip,
  // okq_gemm_q8.hip); the tiled kernel takes the rest with 128 x 128 tiles
  // (f32 activations need the second fp16 plane, which only fits the LDS
  // budget at 128 rows; Q6_K stages its larger raw windows in the 4-wave
  // tile's register budget), or 256 x 128 tiles for bf16 Q4_K shapes beyond
  // the wide kernel's 32-bit offsets.
  const int64_t nsb = K / 256;
  int64_t ks = 1;
  if (M <= kDecRows) {
    // decode batch: the streaming kernel.  K slices small enough for the
    // activations to fit the LDS budget (M rows of 1 or 2 planes of the slice plus
    // sums), and at least enough slices x column groups for every CU.
    p.bm = kDecRows;
    const int64_t per_sb = (int64_t)M * 256 * 2 * (x_is_bf16 ? 1 : 2) + (int64_t)M * 32;
    // slice bounds: the LDS budget and kDecStage pieces of 8 activations per
    // thread (M rows of 32 pieces per super-block)
    const int64_t max_sb = std::max<int64_t>(
        1, std::min<int64_t>((kDecLdsBytes - (int64_t)M * 16 * 2 * 2 - kDecRowExtra * 2 * 2) / per_sb,
                             (int64_t)kDecStage * kDecWaves * 64 / (M * 32)));
    const int64_t ntiles = (N + 15) / 16;
    const int64_t ks_lds = (nsb + max_sb - 1) / max_sb;
    // The whole K fits one workgroup's LDS, the rows one 16-row MFMA group,
    // and the tiles fill no more than one round of 16-wave workgroups: keep
    // K unsplit across workgroups (no
    // partials, no reduction launch) and let kw waves share each tile, each
    // taking every kw-th super-block; T = 16 / kw tiles per workgroup, with T
    // the smallest power of two that puts at most one workgroup on each CU.
    const int64_t per_wg = (ntiles + cu_count - 1) / cu_count;
    if (ks_lds == 1 && per_wg < kDecWaves && M <= 16) {
      int64_t T = 1;
      while (T < per_wg) T *= 2;
      while (kDecWaves / T > nsb) T *= 2;  // every wave needs at least one super-block
      p.kwaves = (int)(kDecWaves / T);
      p.groups = (int)((ntiles + T - 1) / T);
      p.ksplit = 1;
      p.off_lo = p.off_sums = p.off_rscale = p.off_part = 0;
      p.workspace = 0;
      return p;
    }
    // one workgroup (16 waves) per CU: column groups of 16 tiles, at most one
    // per CU (waves then take several tiles), and as many K slices as fit in
    // one round of workgroups (at least what the LDS budget needs)
    p.groups = (int)std::min<int64_t>((ntiles + kDecWaves - 1) / kDecWaves, cu_count);
    ks = std::min<int64_t>(nsb, std::max<int64_t>(ks_lds, cu_count / p.groups));
    // when the LDS split alone would need more than one round of workgroups,
    // fewer column groups (waves take more tiles) keep it to one round: each
    // CU then stages its activation slice once
    if (ks == ks_lds && (int64_t)p.groups * ks > cu_count && ks <= cu_count)
      p.groups = (int)std::max<int64_t>(1, cu_count / ks);
    // unsplit K writes the final outputs with the bias staged for at most
    // kDecMaxTiles tiles per wave; wider problems take the split path
    const int64_t mytiles = (ntiles + (int64_t)p.groups * kDecWaves - 1) / ((int64_t)p.groups * kDecWaves);
    if (ks == 1 && mytiles > kDecMaxTiles) ks = std::min<int64_t>(2, nsb);
    // a single super-block per row cannot be split: more column groups
    // (several rounds of workgroups) keep every wave within kDecMaxTiles
    if (ks == 1 && mytiles > kDecMaxTiles)
      p.groups = (int)((ntiles + (int64_t)kDecWaves * kDecMaxTiles - 1) / ((int64_t)kDecWaves * kDecMaxTiles));
  } else {
    // Q4_K, Q5_K and Q8_0 with bf16 activations: a kernel that dequantises
    // the weights in registers; everything else: the tiled kernel.  Split K
    // when the tiles alone leave CUs idle: enough slices for about one
    // workgroup per CU, at least two super-blocks per slice, at most 8.
    const bool reg_dequant = x_is_bf16 && gemm_wide_supported(type, M, K, N);
    // Q6_K with bf16 activations: gemm_wide_q6k_kernel (128 x 256 tiles, one
    // 8-wave workgroup per CU) while its (tile, K-slice) jobs fill at least
    // 3/4 of their rounds of CUs; otherwise the tiled kernel
    bool q6_wide = false;
    int64_t q6_ks = 1;
    if (x_is_bf16 && type == kQ6_K) {
      const int64_t cus = cu_count, t6 = gemm_q6_tiles(M, N);
      if (t6 * 4 < cus * 3) q6_ks = std::max<int64_t>(1, std::min<int64_t>({(cus + t6 - 1) / t6, nsb / 2, 8}));
      const int64_t jobs = t6 * q6_ks, rounds = (jobs + cus - 1) / cus;
      q6_wide = jobs * 4 >= rounds * cus * 3;
    }
    if (x_is_bf16 && type == kQ8_0) {
      // gemm_q8_kernel (bf16 activations straight from x: no pre-pass).  The
      // 8-wave 128 x 256 tiles (one workgroup per CU) while they fill at
      // least 3/4 of their rounds of CUs (M=2048 4096 x 4096: 1 round);
      // otherwise 4-wave 128 x 128 tiles, two workgroups per CU, K split in
      // 128-K stages while the tiles leave CUs idle: about one workgroup per
      // CU, at least four stages per slice, at most 8 slices (4096 x 4096, us
      // per call: M=512 37.9 at 2 slices vs 39.0 at 4, whose partials cost
      // more than the second workgroup per CU gains; M=128 22.7 at 8 slices)
      p.bm = 128;
      p.wide = 3;
      const int64_t cus = cu_count, t8 = gemm_q8_tiles(M, N, 8);
      if (t8 * 4 >= (t8 + cus - 1) / cus * cus * 3) {
        p.kwaves = 8;
      } else {
        p.kwaves = 4;
        const int64_t qtiles = gemm_q8_tiles(M, N, 4);
        ks = qtiles * 4 < cus * 3 ? std::max<int64_t>(1, std::min<int64_t>({cus / qtiles, K / 512, 8})) : 1;
      }
    } else if (q6_wide) {
      p.bm = 128;
      p.wide = 4;
      ks = q6_ks;
    } else {
      p.bm = reg_dequant ? 128 : ((type == kQ4_K || type == kQ5_K) && x_is_bf16 && M > 128) ? 256 : 128;
      const int64_t cus = cu_count;
      const int64_t tiles = reg_dequant ? gemm_wide_tiles(M, N) : ((M + p.bm - 1) / p.bm) * ((N + kBN - 1) / kBN);
      if (tiles * 4 < cus * 3) ks = std::min<int64_t>({(cus + tiles - 1) / tiles, nsb / 2, 8});
      if (reg_dequant) {
        // gemm_wide_q4k_kernel (128 x 256 tiles, one 8-wave workgroup per CU)
        // while its workgroups fill at least 3/4 of their rounds of CUs (C4,
        // us per call: M=512 gate 76.9 vs 86.7 for the other kernel, down 85.5
        // vs 91.2, q 40.0 vs 41.1; M=2048 gate 292 vs 296, down 268 vs 301);
        // otherwise gemm_pair_q4k_kernel (128 x 128 tiles, two 4-wave
        // workgroups per CU), whose finer tiles and slices occupy every CU
        // where the wide ones cannot (M=128 gate 39.5 vs 56.3, down 36.6 vs
        // 42.8, q 24.2 vs 26.3; M=512 v 25.3 vs 27.8), with as many slices as
        // fit one round of two workgroups per CU.
        const int64_t jobs = tiles * std::max<int64_t>(1, ks);
        const int64_t rounds = (jobs + cus - 1) / cus;
        if (jobs * 4 >= rounds * cus * 3) {
          p.wide = 1;
        } else {
          p.wide = 2;
          const int64_t ptiles = gemm_pair_tiles(M, N), slots = 2 * cus;
          ks = ptiles * 4 < slots * 3 ? std::max<int64_t>(1, std::min<int64_t>({slots / ptiles, nsb / 2, 8})) : 1;
        }
      }
    }
  }
  p.ksplit = (int)std::max<int64_t>(1, ks);
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  if (p.bm == kDecRows) {  // the decode-batch kernel needs only the split-K partials (whole 16-column tiles)
    p.off_lo = p.off_sums = p.off_rscale = p.off_part = 0;
    p.workspace = p.ksplit > 1 ? up((size_t)p.ksplit * M * ((N + 15) / 16 * 16) * sizeof(float)) : 0;
    return p;
  }
  if (p.wide == 3) {  // the Q8_0 bf16 kernel reads x itself: only the split-K partials
    p.off_lo = p.off_sums = p.off_rscale = p.off_part = 0;
    p.workspace = p.ksplit > 1 ? up((size_t)p.ksplit * M * N * sizeof(float)) : 0;
    return p;
  }
  const size_t plane = (size_t)M * (size_t)K * sizeof(_Float16);
  const size_t sums = (size_t)M * (size_t)(K / 32) * 2 * sizeof(_Float16);
  p.off_lo = up(plane);
  p.off_sums = p.off_lo + (x_is_bf16 ? 0 : up(plane));
  p.off_rscale = p.off_sums + up(sums);
  p.off_part = p.off_rscale + up((size_t)M * sizeof(float));
  p.workspace = p.off_part + (p.ksplit > 1 ? up((size_t)p.ksplit * M * N * sizeof(float)) : 0);
  return p;
}

// The decode-batch kernel (it converts the activations itself: no pre-pass)
// and, when K is split, the reduction of its partials (swiglu: the gate/up
// pair's reduction with the gated SiLU).  type2 != type: the
// first nt1 tiles (matrices) are of format `type`, the rest of type2 (Q4_K
// then Q6_K); the plan's column groups are shared out in proportion to the
// two formats' tiles, each format's group keeping at most the plan's tiles
// per wave.
static hipError_t launch_decode(int type, int type2, int nt1, const void *x, bool x_is_bf16, int64_t M, int64_t K,
                                const DecMats &mats, int ntiles, char *ws, const GemmPlan &plan, hipStream_t s,
                                bool swiglu) {
  const int m = (int)M, k = (int)K, ks = plan.ksplit;
  float *part = ks > 1 ? reinterpret_cast<float *>(ws + plan.off_part) : nullptr;
  const int nsb = (int)(K / 256), sl_base = nsb / ks, sl_rem = nsb % ks;  // slice z: sl_base + (z < sl_rem)
  const int nsbs_max = sl_base + (sl_rem > 0 ? 1 : 0);
  int kw_shift = 0;
  while ((1 << kw_shift) < plan.kwaves) ++kw_shift;
  const bool split_w = plan.kwaves > 1;
  const size_t lds = dec_tail_offset(m, 256 * nsbs_max + 8, nsbs_max, x_is_bf16 ? 1 : 2, split_w, M > 16 ? 2 : 1) +
                     ((size_t)kDecMaxTiles * 256 + (size_t)nsbs_max * kDecRows) * sizeof(float) + 16;
  if (lds > 160 * 1024 || (1 << kw_shift) != plan.kwaves || kDecWaves % plan.kwaves != 0 ||
      (split_w && (ks != 1 || M > 16)))
    return hipErrorInvalidValue;
  const bool mixed = type2 != type;
  if (mixed && (type != kQ4_K || type2 != kQ6_K || nt1 < 1 || nt1 >= ntiles)) return hipErrorInvalidValue;
  int g_split = plan.groups, groups = plan.groups;
  if (mixed) {
    auto share = [&](int64_t nt) { return (int)std::max<int64_t>(1, ((int64_t)plan.groups * nt + ntiles - 1) / ntiles); };
    g_split = share(nt1);
    groups = g_split + share(ntiles - nt1);
  }
  const dim3 grid((unsigned)groups, (unsigned)ks), block(kDecWaves * 64);
#define OKQ_DEC(F1_, F2_, LO_, RG_, W_)                                                                          \
  launch_timed(gemm_decode_kernel<F1_, F2_, LO_, RG_, W_>, grid, block, (unsigned)lds, s, x, mats, ntiles, m, k, \
               sl_base, sl_rem, kw_shift, part, g_split, nt1)
#define OKQ_DEC_RG(F1_, F2_, LO_)                 \
  if (M > 16) OKQ_DEC(F1_, F2_, LO_, 2, false);   \
  else if (split_w) OKQ_DEC(F1_, F2_, LO_, 1, true); \
  else OKQ_DEC(F1_, F2_, LO_, 1, false)
  // Q6_K items take d from their scale window when every tensor of the
  // launch has a size that is a multiple of 4 (Q4_K sizes always are)
  bool dw = true;
  for (int i = 0; i < kDecMats; ++i) dw = dw && mats.mat[i].w_bytes % 4u == 0;
  if (mixed) {
    if (dw) {
      if (x_is_bf16) OKQ_DEC_RG(DecQ4K, DecQ6KW, false);
      else OKQ_DEC_RG(DecQ4K, DecQ6KW, true);
    } else {
      if (x_is_bf16) OKQ_DEC_RG(DecQ4K, DecQ6K, false);
      else OKQ_DEC_RG(DecQ4K, DecQ6K, true);
    }
  } else if (type == kQ6_K) {
    if (dw) {
      if (x_is_bf16) OKQ_DEC_RG(DecQ6KW, DecQ6KW, false);
      else OKQ_DEC_RG(DecQ6KW, DecQ6KW, true);
    } else {
      if (x_is_bf16) OKQ_DEC_RG(DecQ6K, DecQ6K, false);
      else OKQ_DEC_RG(DecQ6K, DecQ6K, true);
    }
  } else if (type == kQ8_0) {
    if (x_is_bf16) OKQ_DEC_RG(DecQ80, DecQ80, false);
    else OKQ_DEC_RG(DecQ80, DecQ80, true);
  } else if (type == kQ5_K) {
    if (x_is_bf16) OKQ_DEC_RG(DecQ5K, DecQ5K, false);
    else OKQ_DEC_RG(DecQ5K, DecQ5K, true);
  } else {
    if (x_is_bf16) OKQ_DEC_RG(DecQ4K, DecQ4K, false);
    else OKQ_DEC_RG(DecQ4K, DecQ4K, true);
  }
#undef OKQ_DEC_RG
#undef OKQ_DEC
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || ks == 1) return e;
  if (swiglu) {
    const dim3 sgrid((unsigned)((mats.mat[0].n + 255) / 256), (unsigned)M);
    if (ks <= 4) hipLaunchKernelGGL(splitk_reduce_swiglu_kernel<4>, sgrid, dim3(256), 0, s, part, ks, m, ntiles, mats);
    else if (ks <= 8) hipLaunchKernelGGL(splitk_reduce_swiglu_kernel<8>, sgrid, dim3(256), 0, s, part, ks, m, ntiles, mats);
    else hipLaunchKernelGGL(splitk_reduce_swiglu_kernel<16>, sgrid, dim3(256), 0, s, part, ks, m, ntiles, mats);
    return hipGetLastError();
  }
  const dim3 rgrid((unsigned)((ntiles * 16 + 255) / 256), (unsigned)M);
  if (ks <= 4) hipLaunchKernelGGL(splitk_reduce_mats_kernel<4>, rgrid, dim3(256), 0, s, part, ks, m, ntiles, mats);
  else if (ks <= 8) hipLaunchKernelGGL(splitk_reduce_mats_kernel<8>, rgrid, dim3(256), 0, s, part, ks, m, ntiles, mats);
  else hipLaunchKernelGGL(splitk_reduce_mats_kernel<16>, rgrid, dim3(256), 0, s, part, ks, m, ntiles, mats);
  return hipGetLastError();
}

// A matrix's record for the decode-batch kernel (byte sizes within 32 bits:
// gemm_supported's limits).
static DecMat dec_mat(int type, int64_t K, const void *w, int64_t n, const float *bias, float *y, int tile0) {
  const int64_t sb_bytes = sb_bytes_of(type);
  DecMat d{};
  d.w = static_cast<const uint8_t *>(w);
  d.bias = bias;
  d.y = y;
  d.n = (int)n;
  d.tile0 = tile0;
  d.w_bytes = (uint32_t)(n * (K / 256) * sb_bytes);
  d.bias_bytes = bias ? (uint32_t)(n * 4) : 0u;
  return d;
}

hipError_t launch_gemm_decode_multi(int type, const void *x, bool x_is_bf16, int64_t M, int64_t K, int count,
                                    const void *const *w, const int64_t *N, const float *const *bias, float *const *y,
                                    void *workspace, const GemmPlan &plan, hipStream_t s, bool swiglu) {
  if ((type != kQ4_K && type != kQ5_K && type != kQ6_K && type != kQ8_0) || plan.bm != kDecRows || M > kDecRows || count < 1 ||
      count > kDecMats || (swiglu && (count != 2 || N[0] != N[1])))
    return hipErrorInvalidValue;
  DecMats mats{};
  int tiles = 0;
  for (int i = 0; i < kDecMats; ++i) {
    if (i < count) {
      mats.mat[i] = dec_mat(type, K, w[i], N[i], bias[i], y[i], tiles);
      mats.tile0[i] = tiles;
      tiles += (int)((N[i] + 15) / 16);
    } else {
      mats.tile0[i] = INT32_MAX;
    }
  }
  return launch_decode(type, type, tiles, x, x_is_bf16, M, K, mats, tiles, static_cast<char *>(workspace), plan, s,
                       swiglu);
}

hipError_t launch_gemm_decode_mixed(const void *x, bool x_is_bf16, int64_t M, int64_t K, int count, const int *types,
                                    const void *const *w, const int64_t *N, const float *const *bias, float *const *y,
                                    void *workspace, const GemmPlan &plan, hipStream_t s) {
  if (plan.bm != kDecRows || M > kDecRows || count < 2 || count > kDecMats) return hipErrorInvalidValue;
  DecMats mats{};
  int tiles = 0, nt1 = 0;
  // the Q4_K matrices first, then the Q6_K ones, at least one of each
  if (types[0] != kQ4_K || types[count - 1] != kQ6_K) return hipErrorInvalidValue;
  for (int i = 1; i < count; ++i)
    if ((types[i] != kQ4_K && types[i] != kQ6_K) || (types[i - 1] == kQ6_K && types[i] != kQ6_K))
      return hipErrorInvalidValue;
  for (int i = 0; i < kDecMats; ++i) {
    if (i < count) {
      mats.mat[i] = dec_mat(types[i], K, w[i], N[i], bias[i], y[i], tiles);
      mats.tile0[i] = tiles;
      tiles += (int)((N[i] + 15) / 16);
      if (types[i] == kQ4_K) nt1 = tiles;
    } else {
      mats.tile0[i] = INT32_MAX;
    }
  }
  return launch_decode(kQ4_K, kQ6_K, nt1, x, x_is_bf16, M, K, mats, tiles, static_cast<char *>(workspace), plan, s,
                       false);
}

// The tiled kernel over the pre-pass's planes (every format; f32 or bf16).
static hipError_t launch_gemm_tiled(int type, bool x_is_bf16, _Float16 *xhi, _Float16 *xlo, h2 *xsum, float *rscale,
                                    const uint8_t *W, const float *bias, float *y, int64_t M, int64_t N, int64_t K,
                                    const GemmPlan &plan, float *part, hipStream_t s) {
  const int m = (int)M, n = (int)N, k = (int)K, ks = plan.ksplit;
  const int tiles_n = (int)((N + kBN - 1) / kBN);
  const int tiles_m = (int)((M + plan.bm - 1) / plan.bm);
  const int tiles = tiles_m * tiles_n;
  const int per_xcd = (tiles * ks + 7) / 8;
  const dim3 grid((unsigned)(per_xcd * 8)), block((unsigned)(plan.bm * 2));
#define OKQ_GEMM(BM_, LO_, FMT_)                                                                                   \
  launch_timed(gemm_kq_kernel<BM_, LO_, FMT_>, grid, block, 0u, s, xhi, xlo, xsum, rscale, W, bias, y, m, n, k,     \
               tiles_m, tiles, ks, part)
  if (type == kQ6_K) {
    if (x_is_bf16) OKQ_GEMM(128, false, kQ6_K);
    else OKQ_GEMM(128, true, kQ6_K);
  } else if (type == kQ8_0) {
    if (x_is_bf16) OKQ_GEMM(128, false, kQ8_0);
    else OKQ_GEMM(128, true, kQ8_0);
  } else if (type == kQ5_K) {
    if (plan.bm == 256) OKQ_GEMM(256, false, kQ5_K);
    else if (x_is_bf16) OKQ_GEMM(128, false, kQ5_K);
    else OKQ_GEMM(128, true, kQ5_K);
  } else if (plan.bm == 256) {
    OKQ_GEMM(256, false, kQ4_K);
  } else if (x_is_bf16) {
    OKQ_GEMM(128, false, kQ4_K);
  } else {
    OKQ_GEMM(128, true, kQ4_K);
  }
#undef OKQ_GEMM
  return hipGetLastError();
}


hipError_t launch_gemm(int type, const void *x, bool x_is_bf16, int64_t M, int64_t K, const void *w, int64_t N,
                       const float *bias, float *y, void *workspace, const GemmPlan &plan, hipStream_t s) {
  if (type != kQ4_K && type != kQ5_K && type != kQ6_K && type != kQ8_0) return hipErrorInvalidValue;
  if (type != kQ4_K && type != kQ5_K && plan.bm != 128 && plan.bm != kDecRows) return hipErrorInvalidValue;
  char *ws = static_cast<char *>(workspace);
  const uint8_t *W = static_cast<const uint8_t *>(w);
  const int m = (int)M, n = (int)N, ks = plan.ksplit;
  if (plan.bm == kDecRows) {
    if (M > kDecRows) return hipErrorInvalidValue;
    DecMats mats{};
    mats.mat[0] = dec_mat(type, K, W, N, bias, y, 0);
    for (int i = 1; i < kDecMats; ++i) mats.tile0[i] = INT32_MAX;
    return launch_decode(type, type, (int)((N + 15) / 16), x, x_is_bf16, M, K, mats, (int)((N + 15) / 16), ws, plan, s,
                         false);
  }
  float *part = plan.ksplit > 1 ? reinterpret_cast<float *>(ws + plan.off_part) : nullptr;
  const dim3 rgrid((unsigned)((N + 255) / 256), (unsigned)std::min<int64_t>(M, 65535));
  if (ks > 1 && (int64_t)ks * M * N * 4 > (int64_t)UINT32_MAX) return hipErrorInvalidValue;  // excluded by gemm_plan
  // the split-K reduction of the partials (rscale: the pre-pass's row scales, or none)
  auto reduce = [&](const float *rscale) {
    constexpr int RR = kReduceRows;
    if (N % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0 && (M + RR - 1) / RR <= 65535) {
      const dim3 g4((unsigned)((N + 1023) / 1024), (unsigned)((M + RR - 1) / RR));
      if (ks <= 2) hipLaunchKernelGGL((splitk_reduce4_kernel<2, RR>), g4, dim3(256), 0, s, part, ks, m, n, rscale, bias, y);
      else if (ks <= 4) hipLaunchKernelGGL((splitk_reduce4_kernel<4, RR>), g4, dim3(256), 0, s, part, ks, m, n, rscale, bias, y);
      else hipLaunchKernelGGL((splitk_reduce4_kernel<8, RR>), g4, dim3(256), 0, s, part, ks, m, n, rscale, bias, y);
      return hipGetLastError();
    }
    if (ks <= 2) hipLaunchKernelGGL(splitk_reduce_kernel<2>, rgrid, dim3(256), 0, s, part, ks, m, n, rscale, bias, y);
    else if (ks <= 4) hipLaunchKernelGGL(splitk_reduce_kernel<4>, rgrid, dim3(256), 0, s, part, ks, m, n, rscale, bias, y);
    else hipLaunchKernelGGL(splitk_reduce_kernel<8>, rgrid, dim3(256), 0, s, part, ks, m, n, rscale, bias, y);
    return hipGetLastError();
  };
  if (plan.wide == 3) {
    if (!x_is_bf16 || type != kQ8_0) return hipErrorInvalidValue;
    hipError_t e = launch_gemm_q8(x, W, bias, y, M, N, K, ks, plan.kwaves, part, s);
    return e != hipSuccess || ks == 1 ? e : reduce(nullptr);
  }
  _Float16 *xhi = reinterpret_cast<_Float16 *>(ws);
  _Float16 *xlo = x_is_bf16 ? nullptr : reinterpret_cast<_Float16 *>(ws + plan.off_lo);
  h2 *xsum = reinterpret_cast<h2 *>(ws + plan.off_sums);
  float *rscale = reinterpret_cast<float *>(ws + plan.off_rscale);
  // chunks of 8 activations per thread: 2 (K <= 4096), 4, 8 held in registers, longer rows read twice
  const int64_t per_thread = (K / 8 + 255) / 256;
  const PrepIeee ieee{W, bias, y, (size_t)(K / 256) * (size_t)sb_bytes_of(type), type, (int)N};
#define OKQ_PREP(F32_, CH_)                                                                                       \
  hipLaunchKernelGGL((gemm_prep_kernel<F32_, CH_>), dim3((unsigned)M), dim3(256), 0, s, x, (int)M, (int)K, xhi, xlo, \
                     xsum, rscale, ieee)
#define OKQ_PREP_CH(F32_)                     \
  if (per_thread <= 2) OKQ_PREP(F32_, 2);     \
  else if (per_thread <= 4) OKQ_PREP(F32_, 4); \
  else if (per_thread <= 8) OKQ_PREP(F32_, 8); \
  else OKQ_PREP(F32_, 0)
  if (x_is_bf16) {
    OKQ_PREP_CH(false);
  } else {
    OKQ_PREP_CH(true);
  }
#undef OKQ_PREP_CH
#undef OKQ_PREP
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (plan.wide == 4) {
    e = launch_gemm_q6(xhi, rscale, W, bias, y, M, N, K, ks, part, s);
  } else if (plan.wide == 2) {
    e = launch_gemm_pair(type, xhi, xsum, rscale, W, bias, y, M, N, K, ks, part, s);
  } else if (plan.wide) {
    e = launch_gemm_wide(type, xhi, xsum, rscale, W, bias, y, M, N, K, ks, part, s);
  } else {
    e = launch_gemm_tiled(type, x_is_bf16, xhi, xlo, xsum, rscale, W, bias, y, M, N, K, plan, part, s);
  }
  return e != hipSuccess || ks == 1 ? e : reduce(rscale);
}

}  // namespace okq
