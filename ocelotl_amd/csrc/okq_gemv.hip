// okq_gemv.hip -- fused dequant-GEMV for decode (one activation row).
//
// Design (gfx950, wave64):
//   * A wavefront owns whole output rows.  Its 64 lanes split a row into
//     "units" of 64 weights that live inside whole GGUF blocks (every format
//     has K/64 units per row):
//       Q4_K unit = (super-block, 64-weight chunk c) : 16 B header + 32 B qs
//       Q6_K unit = (super-block, half h, 16-run u2) : 3 x 16 B of ql/qh + scales + d
//       Q8_0 unit = a pair of 34-B blocks             : 68 B, dword aligned
//     Lane l handles units l, l+64, ... (P per lane), so it always touches the
//     same columns of x.
//   * x is quantised once per workgroup, cooperatively, into LDS: each run of
//     32 (Q4_K, Q8_0) or 16 (Q6_K) activations gets a power-of-two scale, is
//     rounded to int16 and split into hi/lo int8 dwords, with the run's exact
//     f32 sum alongside.  The weights' 4/6/8-bit integers contract with them
//     through v_dot4_i32_i8; the partial sums are exact integers and the block
//     scales are applied in f32.
//   * A row of U = K/64 units is split over a team of T = ceil(U/64) waves,
//     so every lane owns exactly one unit and keeps its activations in
//     registers for all rows.  A workgroup holds G teams (G*T <= 16 waves) and
//     walks batches of G*R rows; each wave issues the next batch's loads before
//     computing the current one (register double buffer).  The first batch's
//     loads are issued before the x prologue so their latency overlaps it.
//   * Weights are read with buffer loads against one descriptor spanning the
//     tensor: 32-bit offsets (row offset + lane constant), immediate field
//     offsets, and the hardware range check as a backstop.  2-byte-aligned
//     Q6_K/Q8_0 blocks are read as dword-aligned windows and re-aligned with
//     v_alignbyte_b32; no read leaves the weight tensor.
//   * Row sums are reduced across the wave with DPP + readlane, then across
//     the team's waves through LDS, both in a fixed order (deterministic).
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

// Buffer descriptor over [base, base + bytes), bytes < 2^32 (gfx9 dword 3).
__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// Dword-aligned byte offsets into the descriptor's range.
__device__ __forceinline__ u32x4a4 ld4(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
__device__ __forceinline__ u32x2a4 ld2(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }
__device__ __forceinline__ uint32_t ld1(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
__device__ __forceinline__ uint32_t ld16(Rsrc r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// Quantised activations of one unit (160 bytes, LDS and registers):
//   hi/lo[16]: int8 limbs of 64 activations, byte order = weight byte order
//   s[4]     : power-of-two scale of each run (2 runs of 32 or 4 runs of 16)
//   t[4]     : exact f32 sum of each run (for min/offset terms)
struct XRec {
  uint32_t hi[16];
  uint32_t lo[16];
  float s[4];
  float t[4];
};
static_assert(sizeof(XRec) == 160, "XRec layout");

// Quantise the run of NW*4 floats at xp; write limbs to hi/lo (LDS).
template <int NW>
__device__ __forceinline__ void quantize_run(const float *__restrict__ xp, uint32_t *hi, uint32_t *lo, float &sx,
                                             float &sum) {
  float v[4 * NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const float4 t = *reinterpret_cast<const float4 *>(xp + 4 * i);
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
  const int e = x_exp(amax);
  sx = ldexpf(1.0f, e);
  sum = s;
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

// 16 bytes starting at byte offset a (2-byte aligned, a & 3 == r) as four
// dwords; reads [a - r, a - r + 16) and [a + 12 + r, a + 16 + r), both inside
// [a - 2, a + 18).
struct Win16 {
  u32x4a4 v;
  uint32_t e;
};
__device__ __forceinline__ Win16 ldwin16(Rsrc rs, uint32_t a, uint32_t r) { return {ld4(rs, a - r), ld1(rs, a + 12 + r)}; }
__device__ __forceinline__ void realign16(const Win16 &w, uint32_t r, uint32_t o[4]) {
  o[0] = realign(w.v.y, w.v.x, r);
  o[1] = realign(w.v.z, w.v.y, r);
  o[2] = realign(w.v.w, w.v.z, r);
  o[3] = realign(w.e, w.v.w, r);
}

// ---------------------------------------------------------------------------
// Q4_K
// ---------------------------------------------------------------------------
struct FQ4K {
  static constexpr int kRun = 32;
  static __host__ __device__ size_t row_bytes(int K) { return (size_t)(K / 256) * kQ4KBytes; }
  struct Regs {
    u32x4a4 hd, qa, qb;
  };
  static constexpr int kRows = 2;  // rows per batch (register budget)
  // lane constant: byte offset of the unit's block within a row
  __device__ static uint32_t unit_off(int u) { return (uint32_t)(u >> 2) * kQ4KBytes; }
  __device__ static void load(Regs &r, Rsrc rs, uint32_t blk, uint32_t lane) {
    const uint32_t c = lane & 3;
    r.hd = ld4(rs, blk);
    r.qa = ld4(rs, blk + 16 + 32 * c);
    r.qb = ld4(rs, blk + 32 + 32 * c);
  }
  // run i = [32i, 32i+32): unit i/2, half i%2
  __device__ static void prep(const float *x, int run, XRec *xr) {
    XRec &rec = xr[run >> 1];
    const int h = run & 1;
    quantize_run<8>(x + 32 * run, rec.hi + 8 * h, rec.lo + 8 * h, rec.s[h], rec.t[h]);
  }
  __device__ static float compute(const Regs &r, const XRec &x, uint32_t lane) {
    const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
    int ah = 0, al = 0, bh = 0, bl = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const uint32_t lo4 = q[w] & 0x0F0F0F0Fu;
      const uint32_t hi4 = (q[w] >> 4) & 0x0F0F0F0Fu;
      ah = sdot4(lo4, x.hi[w], ah);
      al = sdot4(lo4, x.lo[w], al);
      bh = sdot4(hi4, x.hi[8 + w], bh);
      bl = sdot4(hi4, x.lo[8 + w], bl);
    }
    // 6-bit scale/min of sub-blocks 2c and 2c+1 without divergence: for
    // c < 2 both fields are 6-bit slices of bytes 0-7, for c >= 2 a 4-bit
    // slice of bytes 8-11 plus two high bits from bytes 0-7.
    const uint32_t c = lane & 3;
    const bool lowj = c < 2;
    const uint32_t width = lowj ? 6u : 4u;
    const uint32_t himask = lowj ? 0u : 0x30u;
    const uint32_t srcs = lowj ? r.hd.y : r.hd.w;
    const uint32_t srcm = lowj ? r.hd.z : r.hd.w;
    const uint32_t j0 = (2 * c) & 3, j1 = (2 * c + 1) & 3;
    const uint32_t mo = lowj ? 0u : 4u;
    const uint32_t scA =
        __builtin_amdgcn_ubfe(srcs, 8 * j0, width) | ((__builtin_amdgcn_ubfe(r.hd.y, 8 * j0 + 6, 2) << 4) & himask);
    const uint32_t scB =
        __builtin_amdgcn_ubfe(srcs, 8 * j1, width) | ((__builtin_amdgcn_ubfe(r.hd.y, 8 * j1 + 6, 2) << 4) & himask);
    const uint32_t mA =
        __builtin_amdgcn_ubfe(srcm, 8 * j0 + mo, width) | ((__builtin_amdgcn_ubfe(r.hd.z, 8 * j0 + 6, 2) << 4) & himask);
    const uint32_t mB =
        __builtin_amdgcn_ubfe(srcm, 8 * j1 + mo, width) | ((__builtin_amdgcn_ubfe(r.hd.z, 8 * j1 + 6, 2) << 4) & himask);
    const float d = f16_bits_hw(r.hd.x & 0xffffu);
    const float dmin = f16_bits_hw(r.hd.x >> 16);
    const float fa = (float)(ah * 256 + al);
    const float fb = (float)(bh * 256 + bl);
    float acc = (d * (float)scA) * (x.s[0] * fa) - (dmin * (float)mA) * x.t[0];
    acc += (d * (float)scB) * (x.s[1] * fb) - (dmin * (float)mB) * x.t[1];
    return acc;
  }
};

// ---------------------------------------------------------------------------
// Q6_K
// ---------------------------------------------------------------------------
struct FQ6K {
  static constexpr int kRun = 16;
  static __host__ __device__ size_t row_bytes(int K) { return (size_t)(K / 256) * kQ6KBytes; }
  struct Regs {
    Win16 L, Lh, H;
    u32x2a4 sv;
    uint32_t se;
    uint32_t d;
    uint32_t r;
  };
  static constexpr int kRows = 1;
  __device__ static uint32_t unit_off(int u) { return (uint32_t)(u >> 2) * kQ6KBytes; }
  __device__ static void load(Regs &g, Rsrc rs, uint32_t B, uint32_t lane) {
    const uint32_t r = B & 3u;  // the tensor base is dword aligned
    const uint32_t h = (lane >> 1) & 1u, u2 = lane & 1u;
    g.r = r;
    g.L = ldwin16(rs, B + 64 * h + 16 * u2, r);
    g.Lh = ldwin16(rs, B + 64 * h + 32 + 16 * u2, r);
    g.H = ldwin16(rs, B + 128 + 32 * h + 16 * u2, r);
    const uint32_t S = B + 192 + 8 * h;  // 8 scale bytes: [S - r, S - r + 8) and [S + 4 + r, S + 8 + r)
    g.sv = ld2(rs, S - r);
    g.se = ld1(rs, S + 4 + r);
    g.d = ld16(rs, B + 208);
  }
  // run j = [16j, 16j+16): super-block j/16; within it 16*(j%16) = 128h + 32qq + 16u2
  __device__ static void prep(const float *x, int run, XRec *xr) {
    const int sb = run >> 4, rr = run & 15;
    const int h = rr >> 3, qq = (rr & 7) >> 1, u2 = rr & 1;
    XRec &rec = xr[4 * sb + 2 * h + u2];
    quantize_run<4>(x + 16 * run, rec.hi + 4 * qq, rec.lo + 4 * qq, rec.s[qq], rec.t[qq]);
  }
  __device__ static float compute(const Regs &g, const XRec &x, uint32_t lane) {
    uint32_t L[4], Lh[4], H[4];
    realign16(g.L, g.r, L);
    realign16(g.Lh, g.r, Lh);
    realign16(g.H, g.r, H);
    const uint32_t S0 = realign(g.sv.y, g.sv.x, g.r);
    const uint32_t S1 = realign(g.se, g.sv.y, g.r);
    int ah[4] = {0, 0, 0, 0}, al[4] = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t q1 = (L[w] & 0x0F0F0F0Fu) | ((H[w] << 4) & 0x30303030u);
      const uint32_t q2 = (Lh[w] & 0x0F0F0F0Fu) | ((H[w] << 2) & 0x30303030u);
      const uint32_t q3 = ((L[w] >> 4) & 0x0F0F0F0Fu) | (H[w] & 0x30303030u);
      const uint32_t q4 = ((Lh[w] >> 4) & 0x0F0F0F0Fu) | ((H[w] >> 2) & 0x30303030u);
      ah[0] = sdot4(q1, x.hi[w], ah[0]);
      al[0] = sdot4(q1, x.lo[w], al[0]);
      ah[1] = sdot4(q2, x.hi[4 + w], ah[1]);
      al[1] = sdot4(q2, x.lo[4 + w], al[1]);
      ah[2] = sdot4(q3, x.hi[8 + w], ah[2]);
      al[2] = sdot4(q3, x.lo[8 + w], al[2]);
      ah[3] = sdot4(q4, x.hi[12 + w], ah[3]);
      al[3] = sdot4(q4, x.lo[12 + w], al[3]);
    }
    const uint32_t u2 = lane & 1u;
    const int sc[4] = {(int)__builtin_amdgcn_sbfe((int)S0, 8 * u2, 8u), (int)__builtin_amdgcn_sbfe((int)S0, 8 * u2 + 16, 8u),
                       (int)__builtin_amdgcn_sbfe((int)S1, 8 * u2, 8u), (int)__builtin_amdgcn_sbfe((int)S1, 8 * u2 + 16, 8u)};
    const float d = f16_bits_hw(g.d);
    float acc = 0.0f;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const float t = x.s[qq] * (float)(ah[qq] * 256 + al[qq]) - 32.0f * x.t[qq];
      acc += (d * (float)sc[qq]) * t;
    }
    return acc;
  }
};

// ---------------------------------------------------------------------------
// Q8_0 (pairs of 34-byte blocks; needs an even number of blocks per row)
// ---------------------------------------------------------------------------
struct FQ80 {
  static constexpr int kRun = 32;
  static __host__ __device__ size_t row_bytes(int K) { return (size_t)(K / 32) * kQ8Bytes; }
  struct Regs {
    u32x4a4 v0, v1, v2, v3;
    uint32_t v4;
  };
  static constexpr int kRows = 1;
  __device__ static uint32_t unit_off(int u) { return (uint32_t)u * (2 * kQ8Bytes); }
  __device__ static void load(Regs &r, Rsrc rs, uint32_t pr, uint32_t) {
    r.v0 = ld4(rs, pr);
    r.v1 = ld4(rs, pr + 16);
    r.v2 = ld4(rs, pr + 32);
    r.v3 = ld4(rs, pr + 48);
    r.v4 = ld1(rs, pr + 64);
  }
  __device__ static void prep(const float *x, int run, XRec *xr) {
    XRec &rec = xr[run >> 1];
    const int h = run & 1;
    quantize_run<8>(x + 32 * run, rec.hi + 8 * h, rec.lo + 8 * h, rec.s[h], rec.t[h]);
  }
  __device__ static float compute(const Regs &r, const XRec &x, uint32_t) {
    const uint32_t w[17] = {r.v0.x, r.v0.y, r.v0.z, r.v0.w, r.v1.x, r.v1.y, r.v1.z, r.v1.w, r.v2.x,
                            r.v2.y, r.v2.z, r.v2.w, r.v3.x, r.v3.y, r.v3.z, r.v3.w, r.v4};
    int a0h = 0, a0l = 0, a1h = 0, a1l = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t q0 = realign(w[k + 1], w[k], 2u);  // block 0 quants: bytes 2..33
      const uint32_t q1 = w[9 + k];                       // block 1 quants: bytes 36..67
      a0h = sdot4(q0, x.hi[k], a0h);
      a0l = sdot4(q0, x.lo[k], a0l);
      a1h = sdot4(q1, x.hi[8 + k], a1h);
      a1l = sdot4(q1, x.lo[8 + k], a1l);
    }
    const float d0 = f16_bits_hw(w[0] & 0xffffu);
    const float d1 = f16_bits_hw(w[8] >> 16);
    return d0 * (x.s[0] * (float)(a0h * 256 + a0l)) + d1 * (x.s[1] * (float)(a1h * 256 + a1l));
  }
};

// ---------------------------------------------------------------------------
// the streaming kernel
// ---------------------------------------------------------------------------
template <class F>
__global__ __launch_bounds__(1024) void gemv_kernel(const uint8_t *__restrict__ W, uint32_t w_bytes,
                                                    const float *__restrict__ x, const float *__restrict__ bias,
                                                    float *__restrict__ y, int N, int K, int T) {
  constexpr int R = F::kRows;
  extern __shared__ __align__(16) unsigned char smem[];
  const int U = K >> 6;
  XRec *xr = reinterpret_cast<XRec *>(smem);
  const uint32_t lane = threadIdx.x & 63;
  const int wave = (int)(threadIdx.x >> 6);
  const int G = (int)(blockDim.x >> 6) / T;  // teams per workgroup
  const int g = wave / T, w = wave % T;
  float *part = reinterpret_cast<float *>(smem + (size_t)U * sizeof(XRec));  // [2][G][R][T]
  const int u = w * 64 + (int)lane;
  const bool active = u < U;
  const uint32_t rb = (uint32_t)F::row_bytes(K);
  const uint32_t uoff = active ? F::unit_off(u) : 0u;
  const Rsrc rs = make_rsrc(W, w_bytes);
  const int rows_per_batch = G * R;

  typename F::Regs A[R], B[R];
  int batch = (int)blockIdx.x;
  const int row0 = batch * rows_per_batch + g * R;
  if (active) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (row0 + r < N) F::load(A[r], rs, (uint32_t)(row0 + r) * rb + uoff, lane);
  }

  // x prologue: one run per thread, cooperatively, into LDS
  const int nruns = K / F::kRun;
  for (int i = (int)threadIdx.x; i < nruns; i += (int)blockDim.x) F::prep(x, i, xr);
  __syncthreads();
  XRec xreg;
  if (active) xreg = xr[u];

  int par = 0;
  while (batch * rows_per_batch < N) {
    const int nbatch = batch + (int)gridDim.x;
    const int nrow0 = nbatch * rows_per_batch + g * R;
    const int row = batch * rows_per_batch + g * R;
    if (active && nbatch * rows_per_batch < N) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (nrow0 + r < N) F::load(B[r], rs, (uint32_t)(nrow0 + r) * rb + uoff, lane);
    }
    float sum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc = 0.0f;
      if (active && row + r < N) acc = F::compute(A[r], xreg, lane);
      sum[r] = wave_sum(acc);
    }
    if (T == 1) {
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (row + r < N) y[row + r] = sum[r] + (bias ? bias[row + r] : 0.0f);
      }
    } else {
      float *pp = part + (size_t)par * G * R * T;
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) pp[(g * R + r) * T + w] = sum[r];
      }
      __syncthreads();
      if (w == 0 && (int)lane < R && row + (int)lane < N) {
        float s = 0.0f;
        for (int t = 0; t < T; ++t) s += pp[(g * R + (int)lane) * T + t];
        y[row + lane] = s + (bias ? bias[row + lane] : 0.0f);
      }
      par ^= 1;  // the next batch writes the other half; two barriers separate reuse
    }
#pragma unroll
    for (int r = 0; r < R; ++r) A[r] = B[r];
    batch = nbatch;
  }
}

// ---------------------------------------------------------------------------
// General fallback (any block-aligned K, 2-byte-aligned blocks): one wave per
// row, lanes stride over elements with byte loads and fp32 FMA.  Used for
// rows longer than 16 waves of units (K > 65536), tensors of 4 GiB or more,
// and Q8_0 rows that are not dword aligned (an odd number of blocks per row).
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
hipError_t launch_gemv(int type, const float *x, int64_t K, const void *w, int64_t N, const float *bias, float *y,
                       int cu_count, hipStream_t s) {
  const uint8_t *W = static_cast<const uint8_t *>(w);
  const uintptr_t wa = reinterpret_cast<uintptr_t>(W);
  const int U = (int)(K / 64);
  const int T = (U + 63) / 64;  // waves per row team
  const size_t wbytes_total =
      (size_t)N * (size_t)(type == kQ8_0 ? (K / 32) * kQ8Bytes : (K / 256) * (type == kQ4_K ? kQ4KBytes : kQ6KBytes));
  bool fast = (K % 64 == 0) && T <= 16 && wbytes_total < 0xFFFFFFFFull;
  if (type == kQ4_K) fast = fast && (wa & 15u) == 0;
  else if (type == kQ6_K) fast = fast && (wa & 3u) == 0;
  else if (type == kQ8_0) fast = fast && (wa & 3u) == 0 && ((K / 32) % 2 == 0);
  else return hipErrorInvalidValue;
  if (fast) {
    const int R = type == kQ4_K ? FQ4K::kRows : 1;
    // teams per workgroup: cover the rows with about one workgroup per CU
    const int64_t max_g = 16 / T;
    int64_t G = (N + (int64_t)cu_count * R - 1) / ((int64_t)cu_count * R);
    if (G < 1) G = 1;
    if (G > max_g) G = max_g;
    const int64_t rows_per_batch = G * R;
    int64_t blocks = (N + rows_per_batch - 1) / rows_per_batch;
    if (blocks > cu_count) blocks = cu_count;
    const dim3 grid((unsigned)blocks), block((unsigned)(64 * T * G));
    const size_t lds = (size_t)U * sizeof(XRec) + (T > 1 ? sizeof(float) * 2 * G * R * T : 0);
    const uint32_t wb = (uint32_t)wbytes_total;
    const int n = (int)N, k = (int)K;
    if (type == kQ4_K) launch_timed(gemv_kernel<FQ4K>, grid, block, (unsigned)lds, s, W, wb, x, bias, y, n, k, T);
    else if (type == kQ6_K) launch_timed(gemv_kernel<FQ6K>, grid, block, (unsigned)lds, s, W, wb, x, bias, y, n, k, T);
    else launch_timed(gemv_kernel<FQ80>, grid, block, (unsigned)lds, s, W, wb, x, bias, y, n, k, T);
    return hipGetLastError();
  }
  int64_t blocks = (N + 3) / 4;
  if (blocks > (int64_t)cu_count * 4) blocks = (int64_t)cu_count * 4;
  if (blocks < 1) blocks = 1;
  const size_t row_bytes =
      (size_t)(type == kQ8_0 ? (K / 32) * kQ8Bytes : (K / 256) * (type == kQ4_K ? kQ4KBytes : kQ6KBytes));
  launch_timed(gemv_generic_kernel, dim3((unsigned)blocks), dim3(256), 0u, s, type, W, x, bias, y, (int)N, (int)K,
               row_bytes);
  return hipGetLastError();
}

}  // namespace okq
