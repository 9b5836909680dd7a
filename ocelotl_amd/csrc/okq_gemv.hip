// okq_gemv.hip -- fused dequant-GEMV for decode (one activation row).
//
// Design (gfx950, wave64):
//   * A wavefront owns whole output rows.  Its 64 lanes split a row into
//     "units" of 64 weights that live inside whole GGUF blocks (every format
//     has K/64 units per row):
//       Q4_K unit = (super-block, 64-weight chunk c) : 16 B header + 32 B qs
//       Q6_K unit = (super-block, half h, 16-run u2) : 3 x 16 B of ql/qh + scales + d
//       Q8_0 unit = a pair of 34-B blocks             : 68 B, dword aligned
//     A lane always handles the same unit position, so it always touches the
//     same columns of x.
//   * x is quantised once per workgroup, cooperatively, into LDS: each run of
//     32 (Q4_K, Q8_0) or 16 (Q6_K) activations gets a power-of-two scale, is
//     rounded to a 24-bit integer and split into three int8 limbs, with the
//     run's f32 sum alongside (groups of 8 or 4 lanes, one float4 each, share
//     the run's max and sum through DPP).  The weights' 4/6/8-bit integers
//     contract with them through v_dot4_i32_i8; the partial sums are exact
//     integers and the block scales are applied in f32.
//   * Activations holding an infinity or a NaN (some run sum is not finite;
//     every workgroup sees the same x, so all take the same branch) are
//     contracted in plain f32 instead, element by element with the weights
//     dequantised exactly, so outputs carry the reference's IEEE infinities
//     and NaNs; rows of finite activations in the same launch keep the
//     integer path's bits.
//   * A row of U = K/64 units is split over a team of T = ceil(U/64) waves,
//     so every lane owns exactly one unit and keeps its activations in
//     registers for all rows.  A workgroup holds G teams (G*T <= 16 waves).
//   * Ordering is what makes it fast (measured with per-wave timestamps):
//     vector loads complete in issue order per CU, so every wave first issues
//     its x loads, a bare barrier queues all of them ahead of any weight load,
//     and only then do the weight loads start.  Rows are swept step-major
//     across the chip (one contiguous window of rows per step keeps the HBM
//     channels evenly loaded); each wave keeps a ring of D rows in flight and
//     computes a row as soon as it arrives.  The SIMD arbiters favour older
//     waves (a workgroup's youngest waves finished ~2.7 us after its oldest
//     on the gate/up shape), so launches with more than a few rows per wave
//     hand out all but each wave's first D rows from a workgroup counter in
//     LDS, in the same step-major order.  Every load is unconditional:
//     rows past the end address past the tensor and read zeros, because a
//     branch around a load makes the compiler wait for all outstanding loads.
//   * Weights are read with buffer loads against one descriptor spanning the
//     tensor: 32-bit offsets (row offset + lane constant), immediate field
//     offsets, and the hardware range check as a backstop.  2-byte-aligned
//     Q6_K/Q8_0 blocks are read as dword-aligned windows and re-aligned with
//     v_alignbyte_b32; no read leaves the weight tensor.
//   * Row sums are reduced across the wave with DPP + readlane, then (T > 1)
//     across the team's waves through LDS once per chunk of steps, both in a
//     fixed order (deterministic).  The file is compiled without FMA
//     contraction and every FMA is written out, so a row's result does not
//     depend on which instantiation (rows per launch, matrices per launch)
//     computed it.
#include "okq_device.h"
#include "okq_internal.h"

#include <algorithm>
#include <type_traits>

namespace okq {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3a4 __attribute__((ext_vector_type(3)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

// Buffer descriptor over [base, base + bytes), bytes < 2^32 (gfx9 dword 3).
__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// Dword-aligned byte offsets into the descriptor's range.
__device__ __forceinline__ u32x4a4 ld4(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
__device__ __forceinline__ u32x2a4 ld2(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }
__device__ __forceinline__ u32x3a4 ld3(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0); }
__device__ __forceinline__ uint32_t ld1(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
__device__ __forceinline__ uint32_t ld16(Rsrc r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// Quantised activations of one unit (224 bytes, LDS and registers):
//   hi/mi/lo[16]: int8 limbs of 64 activations, byte order = weight byte order
//   s[4]        : power-of-two scale of each run (2 runs of 32 or 4 runs of 16)
//   t[4]        : f32 sum of each run (for min/offset terms); a run holding an
//                 infinity or a NaN has a non-finite sum, which is how the
//                 kernel finds activations that need the IEEE path
struct XRec {
  uint32_t hi[16];
  uint32_t mi[16];
  uint32_t lo[16];
  float s[4];
  float t[4];
};
static_assert(sizeof(XRec) == 224, "XRec layout");
// The low limbs are read from LDS where they are used (three-limb launches
// only), so a lane's registers hold the hi/mi limbs, scales and sums.
typedef __attribute__((address_space(3))) const uint32_t LdsU32;

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
  static constexpr int kType = kQ4_K;
  // element e < 64 of unit u is k = 64 u + e (low nibbles of the chunk's 32
  // bytes, then the high nibbles)
  __device__ static int kidx(int u, int e) { return 64 * u + e; }
  static __host__ __device__ size_t row_bytes(int K) { return (size_t)(K / 256) * kQ4KBytes; }
  struct Regs {
    u32x4a4 hd, qa, qb;
  };
  static constexpr int kMaxDepth = 2;  // rows in flight per wave
  // lane constant: byte offset of the unit's block within a row
  __device__ static uint32_t unit_off(int u) { return (uint32_t)(u >> 2) * kQ4KBytes; }
  __device__ static void load(Regs &r, Rsrc rs, uint32_t blk, uint32_t lane) {
    const uint32_t c = lane & 3;
    r.hd = ld4(rs, blk);
    r.qa = ld4(rs, blk + 16 + 32 * c);
    r.qb = ld4(rs, blk + 32 + 32 * c);
  }
  // run i = [32i, 32i+32): unit i/2, half i%2
  __device__ static void xslot(int run, int &rec, int &word, int &slot) {
    rec = run >> 1;
    word = 8 * (run & 1);
    slot = run & 1;
  }
  __device__ static float compute(const Regs &r, const XRec &x, const LdsU32 *xlo, bool lo3, uint32_t lane) {
    const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
    int ah = 0, am = 0, al = 0, bh = 0, bm = 0, bl = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const uint32_t lo4 = q[w] & 0x0F0F0F0Fu;
      const uint32_t hi4 = (q[w] >> 4) & 0x0F0F0F0Fu;
      ah = sdot4(lo4, x.hi[w], ah);
      am = sdot4(lo4, x.mi[w], am);
      bh = sdot4(hi4, x.hi[8 + w], bh);
      bm = sdot4(hi4, x.mi[8 + w], bm);
    }
    if (lo3) {  // wave-uniform
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        al = sdot4(q[w] & 0x0F0F0F0Fu, xlo[w], al);
        bl = sdot4((q[w] >> 4) & 0x0F0F0F0Fu, xlo[8 + w], bl);
      }
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
    const float pa = x.s[0] * limb_sum(ah, am, al);  // the power-of-two scale is exact
    const float pb = x.s[1] * limb_sum(bh, bm, bl);
    const float a = fmaf(d * (float)scA, pa, -((dmin * (float)mA) * x.t[0]));
    const float b = fmaf(d * (float)scB, pb, -((dmin * (float)mB) * x.t[1]));
    return a + b;
  }
};

// ---------------------------------------------------------------------------
// Q5_K: Q4_K with a fifth bit per weight.  Unit = (super-block, 64-weight
// chunk c): the 16-byte header, the 32 qh bytes (bit 2c of qh[l] tops the
// low nibble of qs byte l of the chunk, bit 2c + 1 the high one) and the
// chunk's 32 qs bytes.  The four lanes of a super-block read the same qh
// bytes in one instruction.
// ---------------------------------------------------------------------------
struct FQ5K {
  static constexpr int kRun = 32;
  static constexpr int kType = kQ5_K;
  __device__ static int kidx(int u, int e) { return 64 * u + e; }
  static __host__ __device__ size_t row_bytes(int K) { return (size_t)(K / 256) * kQ5KBytes; }
  struct Regs {
    u32x4a4 hd, ha, hb, qa, qb;
  };
  static constexpr int kMaxDepth = 2;
  __device__ static uint32_t unit_off(int u) { return (uint32_t)(u >> 2) * kQ5KBytes; }
  __device__ static void load(Regs &r, Rsrc rs, uint32_t blk, uint32_t lane) {
    const uint32_t c = lane & 3;
    r.hd = ld4(rs, blk);
    r.ha = ld4(rs, blk + 16);
    r.hb = ld4(rs, blk + 32);
    r.qa = ld4(rs, blk + 48 + 32 * c);
    r.qb = ld4(rs, blk + 64 + 32 * c);
  }
  __device__ static void xslot(int run, int &rec, int &word, int &slot) { FQ4K::xslot(run, rec, word, slot); }
  __device__ static float compute(const Regs &r, const XRec &x, const LdsU32 *xlo, bool lo3, uint32_t lane) {
    const uint32_t c = lane & 3;
    const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
    const uint32_t h[8] = {r.ha.x, r.ha.y, r.ha.z, r.ha.w, r.hb.x, r.hb.y, r.hb.z, r.hb.w};
    uint32_t lo5[8], hi5[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const uint32_t hs = h[w] >> (2 * c);
      lo5[w] = (q[w] & 0x0F0F0F0Fu) | ((hs << 4) & 0x10101010u);
      hi5[w] = ((q[w] >> 4) & 0x0F0F0F0Fu) | ((hs << 3) & 0x10101010u);
    }
    int ah = 0, am = 0, al = 0, bh = 0, bm = 0, bl = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      ah = sdot4(lo5[w], x.hi[w], ah);
      am = sdot4(lo5[w], x.mi[w], am);
      bh = sdot4(hi5[w], x.hi[8 + w], bh);
      bm = sdot4(hi5[w], x.mi[8 + w], bm);
    }
    if (lo3) {  // wave-uniform
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        al = sdot4(lo5[w], xlo[w], al);
        bl = sdot4(hi5[w], xlo[8 + w], bl);
      }
    }
    // the scale/min fields are Q4_K's (see FQ4K::compute)
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
    const float pa = x.s[0] * limb_sum(ah, am, al);
    const float pb = x.s[1] * limb_sum(bh, bm, bl);
    const float a = fmaf(d * (float)scA, pa, -((dmin * (float)mA) * x.t[0]));
    const float b = fmaf(d * (float)scB, pb, -((dmin * (float)mB) * x.t[1]));
    return a + b;
  }
};

// ---------------------------------------------------------------------------
// Q6_K
// ---------------------------------------------------------------------------
struct FQ6K {
  static constexpr int kRun = 16;
  static constexpr int kType = kQ6_K;
  // unit u = (super-block u / 4, half h = (u / 2) & 1, 16-run u2 = u & 1):
  // element e < 64 is k = 256 sb + 128 h + 32 (e / 16) + 16 u2 + e % 16
  __device__ static int kidx(int u, int e) {
    return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 32 * (e >> 4) + 16 * (u & 1) + (e & 15);
  }
  static __host__ __device__ size_t row_bytes(int K) { return (size_t)(K / 256) * kQ6KBytes; }
  struct Regs {
    u32x4a4 qa, qb;  // a 36-byte window of this lane's 32 ql bytes [64 h + 32 u2, + 32)
    uint32_t qe;
    Win16 H;
    u32x4a4 sw;  // the half's scales (and, h = 1, d)
    uint32_t r;
  };
  static constexpr int kMaxDepth = 1;  // measured: deeper rings slow the long Q6_K streams
  __device__ static uint32_t unit_off(int u) { return (uint32_t)(u >> 2) * kQ6KBytes; }
  __device__ static void load(Regs &g, Rsrc rs, uint32_t B, uint32_t lane) {
    const uint32_t r = B & 3u;  // the tensor base is dword aligned
    const uint32_t h = (lane >> 1) & 1u, u2 = lane & 1u;
    g.r = r;
    // the half's 64 ql bytes are shared out by the lane pair (u2 = 0, 1):
    // each loads 32 contiguous bytes, and compute() trades the 16-byte
    // pieces each needs with its partner lane
    const uint32_t a = B + 64 * h + 32 * u2;
    g.qa = ld4(rs, a - r);
    g.qb = ld4(rs, a - r + 16);
    g.qe = ld1(rs, a - r + 32);
    g.H = ldwin16(rs, B + 128 + 32 * h + 16 * u2, r);
    // one 16-byte window: h = 0 the half's 8 scale bytes [S, S + 8) inside
    // the block ([S - 4, S + 12) or [S - 2, S + 14)); h = 1 its scales and
    // d, [B + 196, B + 212) (r = 0: 2 bytes into the next block) or
    // [B + 194, B + 210) (r = 2).  The tensor's last block starts 2 bytes
    // off a dword (its size is a multiple of 4: checked by the launcher), so
    // no window leaves the tensor.
    const uint32_t S = B + 192 + 8 * h;
    g.sw = ld4(rs, S - 4 + r - ((h & (r >> 1)) << 2));
  }
  // run j = [16j, 16j+16): super-block j/16; within it 16*(j%16) = 128h + 32qq + 16u2
  __device__ static void xslot(int run, int &rec, int &word, int &slot) {
    const int sb = run >> 4, rr = run & 15;
    const int h = rr >> 3, qq = (rr & 7) >> 1, u2 = rr & 1;
    rec = 4 * sb + 2 * h + u2;
    word = 4 * qq;
    slot = qq;
  }
  __device__ static float compute(const Regs &g, const XRec &x, const LdsU32 *xlo, bool lo3, uint32_t lane) {
    // this lane's ql pieces 2 u2 and 2 u2 + 1 (16 bytes each) of its half;
    // it needs pieces u2 (L) and u2 + 2 (Lh): lane u2 = 0 keeps piece 0 and
    // takes piece 2 from its partner (lane ^ 1), lane u2 = 1 keeps piece 3
    // and takes piece 1 (DPP quad_perm 1,0,3,2 swaps the pair's values)
    const uint32_t w9[9] = {g.qa.x, g.qa.y, g.qa.z, g.qa.w, g.qb.x, g.qb.y, g.qb.z, g.qb.w, g.qe};
    uint32_t Mq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) Mq[i] = realign(w9[i + 1], w9[i], g.r);
    const bool odd = (lane & 1u) != 0u;
    uint32_t L[4], Lh[4], H[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t send = odd ? Mq[i] : Mq[4 + i];
      const uint32_t recv = dpp_row_u<0xB1>(send);
      L[i] = odd ? recv : Mq[i];
      Lh[i] = odd ? Mq[4 + i] : recv;
    }
    realign16(g.H, g.r, H);
    // scales at window byte 4 - r (h = 0) or 4 + r (h = 1); d at 12 + r
    // (h = 1), taken by the h = 0 lanes from their h = 1 partner (lane ^ 2)
    const uint32_t hh = (lane >> 1) & 1u;
    const bool hi1 = hh != 0u || g.r == 0u;  // the scales start in dword 1
    const uint32_t S0 = hi1 ? realign(g.sw.z, g.sw.y, g.r) : realign(g.sw.y, g.sw.x, g.r);
    const uint32_t S1 = hi1 ? realign(g.sw.w, g.sw.z, g.r) : realign(g.sw.z, g.sw.y, g.r);
    const uint32_t dh = (g.sw.w >> (8u * g.r)) & 0xffffu;
    const uint32_t dq = dpp_row_u<0x4E>(dh);  // quad_perm 2,3,0,1
    const uint32_t dbits = hh ? dh : dq;
    int ah[4] = {0, 0, 0, 0}, am[4] = {0, 0, 0, 0}, al[4] = {0, 0, 0, 0};
    uint32_t qv[4][4];  // [w][quarter]
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      qv[w][0] = (L[w] & 0x0F0F0F0Fu) | ((H[w] << 4) & 0x30303030u);
      qv[w][1] = (Lh[w] & 0x0F0F0F0Fu) | ((H[w] << 2) & 0x30303030u);
      qv[w][2] = ((L[w] >> 4) & 0x0F0F0F0Fu) | (H[w] & 0x30303030u);
      qv[w][3] = ((Lh[w] >> 4) & 0x0F0F0F0Fu) | ((H[w] >> 2) & 0x30303030u);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        ah[qq] = sdot4(qv[w][qq], x.hi[4 * qq + w], ah[qq]);
        am[qq] = sdot4(qv[w][qq], x.mi[4 * qq + w], am[qq]);
      }
    }
    if (lo3) {  // wave-uniform
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) al[qq] = sdot4(qv[w][qq], xlo[4 * qq + w], al[qq]);
    }
    const uint32_t u2 = lane & 1u;
    const int sc[4] = {(int)__builtin_amdgcn_sbfe((int)S0, 8 * u2, 8u), (int)__builtin_amdgcn_sbfe((int)S0, 8 * u2 + 16, 8u),
                       (int)__builtin_amdgcn_sbfe((int)S1, 8 * u2, 8u), (int)__builtin_amdgcn_sbfe((int)S1, 8 * u2 + 16, 8u)};
    const float d = f16_bits_hw(dbits);
    float acc = 0.0f;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const float t = x.s[qq] * limb_sum(ah[qq], am[qq], al[qq]) - 32.0f * x.t[qq];  // both products exact
      acc = fmaf(d * (float)sc[qq], t, acc);
    }
    return acc;
  }
};

// ---------------------------------------------------------------------------
// Q8_0 (pairs of 34-byte blocks; needs an even number of blocks per row)
// ---------------------------------------------------------------------------
struct FQ80 {
  static constexpr int kRun = 32;
  static constexpr int kType = kQ8_0;
  // unit u = blocks 2u and 2u + 1: k = 64 u + e
  __device__ static int kidx(int u, int e) { return 64 * u + e; }
  static __host__ __device__ size_t row_bytes(int K) { return (size_t)(K / 32) * kQ8Bytes; }
  struct Regs {
    u32x4a4 v0, v1, v2, v3;
    uint32_t v4;
  };
  static constexpr int kMaxDepth = 2;
  __device__ static uint32_t unit_off(int u) { return (uint32_t)u * (2 * kQ8Bytes); }
  __device__ static void load(Regs &r, Rsrc rs, uint32_t pr, uint32_t) {
    r.v0 = ld4(rs, pr);
    r.v1 = ld4(rs, pr + 16);
    r.v2 = ld4(rs, pr + 32);
    r.v3 = ld4(rs, pr + 48);
    r.v4 = ld1(rs, pr + 64);
  }
  __device__ static void xslot(int run, int &rec, int &word, int &slot) {
    rec = run >> 1;
    word = 8 * (run & 1);
    slot = run & 1;
  }
  __device__ static float compute(const Regs &r, const XRec &x, const LdsU32 *xlo, bool lo3, uint32_t) {
    const uint32_t w[17] = {r.v0.x, r.v0.y, r.v0.z, r.v0.w, r.v1.x, r.v1.y, r.v1.z, r.v1.w, r.v2.x,
                            r.v2.y, r.v2.z, r.v2.w, r.v3.x, r.v3.y, r.v3.z, r.v3.w, r.v4};
    int a0h = 0, a0m = 0, a0l = 0, a1h = 0, a1m = 0, a1l = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t q0 = realign(w[k + 1], w[k], 2u);  // block 0 quants: bytes 2..33
      const uint32_t q1 = w[9 + k];                       // block 1 quants: bytes 36..67
      a0h = sdot4(q0, x.hi[k], a0h);
      a0m = sdot4(q0, x.mi[k], a0m);
      a1h = sdot4(q1, x.hi[8 + k], a1h);
      a1m = sdot4(q1, x.mi[8 + k], a1m);
    }
    if (lo3) {  // wave-uniform
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        a0l = sdot4(realign(w[k + 1], w[k], 2u), xlo[k], a0l);
        a1l = sdot4(w[9 + k], xlo[8 + k], a1l);
      }
    }
    const float d0 = f16_bits_hw(w[0] & 0xffffu);
    const float d1 = f16_bits_hw(w[8] >> 16);
    return fmaf(d1, x.s[1] * limb_sum(a1h, a1m, a1l), d0 * (x.s[0] * limb_sum(a0h, a0m, a0l)));
  }
};

// ---------------------------------------------------------------------------
// activation prologue: lanes in groups of kRun/4 each hold one float4 of a
// run; the group shares the run's max|x| and sum through DPP (fixed order),
// then each lane writes one dword of each limb of the run's XRec.
// ---------------------------------------------------------------------------

// Returns the run's status: bit 0 when the run is wide (its largest |x|
// exceeds 8 times its mean |x|, so the launch contracts all three limbs),
// bit 1 when the run holds an infinity or a NaN (its sum is not finite).
template <class F>
__device__ __forceinline__ unsigned quant_group(u32x4a4 raw, int f, int nf, XRec *xr) {
  constexpr int GL = F::kRun / 4;  // lanes per run: 8 (runs of 32) or 4 (runs of 16)
  const float v0 = as_f32(raw.x), v1 = as_f32(raw.y), v2 = as_f32(raw.z), v3 = as_f32(raw.w);
  // The lanes' max|x| meet as bit patterns: for |x| the unsigned order is
  // the float order, and an unsigned max takes its DPP operand in the same
  // instruction, where a float max first quiets it (v_max_f32 x, x).  A NaN
  // then wins where the float max would drop it; such a run has a NaN sum,
  // so its activation row takes the f32 path and its record goes unused.
  auto umax = [](uint32_t p, uint32_t q) { return p > q ? p : q; };
  uint32_t ab = as_u32(fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3))));
  float t = (v0 + v1) + (v2 + v3);
  float m = (fabsf(v0) + fabsf(v1)) + (fabsf(v2) + fabsf(v3));
  ab = umax(ab, dpp_row_u<0xB1>(ab));  // quad_perm 1,0,3,2
  t += dpp_row_f<0xB1>(t);
  m += dpp_row_f<0xB1>(m);
  ab = umax(ab, dpp_row_u<0x4E>(ab));  // quad_perm 2,3,0,1
  t += dpp_row_f<0x4E>(t);
  m += dpp_row_f<0x4E>(m);
  if (GL == 8) {
    ab = umax(ab, dpp_row_u<0x141>(ab));  // row_half_mirror: lane i <-> 7 - i within 8
    t += dpp_row_f<0x141>(t);
    m += dpp_row_f<0x141>(m);
  }
  // Pinned here, with every lane on: otherwise the compiler sinks the last
  // step's add and max into the branch below and keeps its DPP moves apart
  // (a DPP operand must be read with all lanes on).
  asm volatile("" : : "v"(ab), "v"(t), "v"(m));
  const float a = as_f32(ab);
  // max <= 8 * mean: a <= m * 8 / kRun (m is the run's sum of |x|)
  const unsigned wide = (a <= m * (8.0f / (float)F::kRun)) ? 0u : 1u;
  const unsigned status = f < nf ? (__builtin_isfinite(t) ? wide : 2u) : 0u;
  if (f < nf) {
    const int e = x_exp(a);
    uint32_t hi, mi, lo;
    limbs4(x_digits(v0, e), x_digits(v1, e), x_digits(v2, e), x_digits(v3, e), hi, mi, lo);
    const int run = f / GL, i = f % GL;
    int rec, word, slot;
    F::xslot(run, rec, word, slot);
    xr[rec].hi[word + i] = hi;
    xr[rec].mi[word + i] = mi;
    xr[rec].lo[word + i] = lo;
    if (i == 0) {
      xr[rec].s[slot] = ldexpf(1.0f, e);
      xr[rec].t[slot] = t;
    }
  }
  return status;
}

// ---------------------------------------------------------------------------
// the streaming kernel
// ---------------------------------------------------------------------------
// The matrices of a multi-matrix launch, matrix 0 included: its blocks
// (bytes: the tensor's size, within 32 bits), bias and output, its first row
// among the launch's concatenated rows and its row count (the output's row
// stride).  Rows [start[i], start[i+1]) belong to matrix i + 1; start[i] =
// INT_MAX and an empty record for unused entries.
struct GemvMat {
  const uint8_t *w;
  const float *bias;
  float *y;
  uint32_t bytes;
  int first, rows, pad;
};
struct GemvMore {
  GemvMat mat[kGemvMaxProblems];
  int start[kGemvMaxProblems - 1];
};

constexpr int kMaxXV = 4;        // float4s of x per thread, one-row launches (K <= 4 * 4 * 1024)
constexpr int kMaxXVRows = 8;    // per thread and row, multi-row launches (K <= 8 * 4 * 512)
constexpr int kPartChunk = 32;   // steps whose team partial sums wait in LDS
constexpr int kMaxRowsPerLaunch = 4;
constexpr int kDynSteps = 4;     // dynamic rows above this many steps per wave (one wave per row)
constexpr size_t kLdsBytes = 160 * 1024;  // LDS per workgroup on gfx950

// One activation row keeps one XRec per lane in registers and 16 waves fit a
// CU; R rows keep R of them (their hi/mi limbs, scales and sums: 160 VGPRs
// for four; the low limbs are read from LDS), so multi-row launches are
// limited to 8 waves (two per SIMD).
template <int R>
constexpr int gemv_max_threads() {
  return R == 1 ? 1024 : 512;
}

// Rows are swept step-major across the chip: at step s, team g of workgroup
// b (B workgroups of G teams) takes row (s * B + b) * G + g, so the whole grid
// reads one contiguous window per step and HBM channels stay evenly loaded;
// the launch picks G so that the steps divide the rows as evenly as
// possible.  Each wave keeps the next D rows' loads in flight in a ring of
// register sets and computes a row as soon as it has arrived.
//
// One launch may serve several weight matrices of one format and in_features
// that share the activation row (q/k/v, gate/up): their rows are numbered
// consecutively and every row finds its matrix, bias and output through
// wave-uniform scalar selects.
//
// R activation rows (x [nrows, K], nrows <= R; y_i [nrows, N_i]) share one
// pass over the weights: every lane holds its unit's XRec of each row and
// contracts each weight unit it loads with all of them, so a batch of up to
// four decode rows streams the weights once.
//
// kPro transforms x before it is quantised (the decode neighbours of the
// projections, computed by every workgroup from the same inputs in the same
// order, so all workgroups agree): kProRms is the RMSNorm of x with weight
// P.a (crates/kernels/src/rmsnorm.rs:73-128), kProSwiGLU is silu(x) * P.a with
// x = gate and P.a = up (crates/kernels/src/mlp.rs:77-88, :233-238).
//
// kDyn (one wave per row, T == 1, and more than kDynSteps steps): each wave's
// first D rows are static, the rest are handed out in the workgroup's
// step-major order by an LDS counter, so the waves that the SIMD arbiters
// favour take more rows and a workgroup's waves finish together.  Results
// are the same bits as the static order's (every row is one wave's work).
template <class F, int D, int XV, bool kMulti, int kPro, int R, bool kDyn>
__global__ __launch_bounds__(gemv_max_threads<R>()) void gemv_kernel(
    const uint8_t *__restrict__ W, uint32_t w_bytes, const float *__restrict__ x, const float *__restrict__ bias,
    float *__restrict__ y, int N, int K, int T, int G, GemvMore M, GemvPro P, int nrows) {
  static_assert(kPro == kProNone || R == 1, "the neighbour prologues take one activation row");
  // kDyn launches have T == 1 (one wave per row), checked by the launcher
  __shared__ unsigned next_row;  // kDyn: the workgroup's next row index
  __shared__ unsigned qflags[16];  // per wave: the run status bits of its lanes
  // G teams of T waves stream rows; with T == 1 the workgroup may hold extra
  // waves (g >= G) that only help quantise x.
  extern __shared__ __align__(16) unsigned char smem[];
  const int U = K >> 6;
  XRec *xr = reinterpret_cast<XRec *>(smem);  // [R][U]
  const int tid = (int)threadIdx.x, nt = (int)blockDim.x;
  const uint32_t lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: rows live in SGPRs
  const int g = wave / T, w = wave % T;
  float *part = reinterpret_cast<float *>(smem + (size_t)R * U * sizeof(XRec));  // [kChunk][G][T][R] (T > 1)
  const int u = w * 64 + (int)lane;
  const bool active = u < U && g < G;
  const uint32_t rb = (uint32_t)F::row_bytes(K);
  const uint32_t uoff = active ? F::unit_off(u) : 0u;
  const uint32_t idle_mask = active ? 0u : 0xFFFFFFFFu;  // kDyn
  const int window = (int)gridDim.x * G;         // rows per step
  const int steps = (N + window - 1) / window;  // grid-uniform
  const int end = N;
  float inv_rms = 0.0f;  // kProRms: 1 / rms of the row (the IEEE path reapplies it)
  auto row_of = [&](int step) { return step * window + (int)blockIdx.x * G + g; };
  // Matrix selection: single-matrix launches (kMulti = false) never touch M;
  // in multi-matrix launches a row finds its matrix from the three row
  // boundaries and reads that matrix's record with scalar loads at a
  // wave-uniform index.  (Selecting each field from four candidates instead
  // compiled into chains of scalar compares and branches -- ~170 scalar
  // instructions per row, with every wave of the CU sharing one scalar unit;
  // the records halve that and took q+k+v from 7.07 to 6.72 us.)
  const int st1 = kMulti ? M.start[0] : INT32_MAX, st2 = kMulti ? M.start[1] : INT32_MAX;
  const int st3 = kMulti ? M.start[2] : INT32_MAX;
  auto rec = [&](int p) -> GemvMat {
    if constexpr (kMulti) return M.mat[__builtin_amdgcn_readfirstlane(p)];
    else return GemvMat{W, bias, y, w_bytes, 0, N, 0};
  };
  // the matrix of a row (rows past the end map to the last one)
  auto prob = [&](int row) {
    return kMulti ? (int)(row >= st1) + (int)(row >= st2) + (int)(row >= st3) : 0;
  };
  auto first_row = [&](int p) { return rec(p).first; };
  auto rsrc = [&](int p) { const GemvMat m = rec(p); return make_rsrc(m.w, m.bytes); };
  auto bytes_of = [&](int p) { return rec(p).bytes; };
  auto bias_of = [&](int p) { return rec(p).bias; };
  auto y_of = [&](int p) { return rec(p).y; };
  // rows of matrix p (the row stride of its output)
  auto rows_of = [&](int p) { return rec(p).rows; };
  // Byte offset of this lane's unit in `row`; rows past the end (and idle
  // lanes) point at the end of their tensor, where buffer loads return zeros
  // without touching memory, so every load is unconditional.
  auto wload = [&](typename F::Regs &Rg, int row) {
    const int p = prob(row);
    uint32_t off;
    if constexpr (kDyn) {  // no branch on the lane: idle lanes select the end arithmetically
      const uint32_t endb = bytes_of(p);
      const uint32_t in = row < end ? (uint32_t)(row - first_row(p)) * rb + uoff : endb;
      off = in ^ ((in ^ endb) & idle_mask);
    } else {
      off = (active && row < end) ? (uint32_t)(row - first_row(p)) * rb + uoff : bytes_of(p);
    }
    F::load(Rg, rsrc(p), off, lane);
  };
  // bias values are wave-uniform scalar loads, outside the vector-memory
  // queue that the weight waits count (the dynamic loop reads them through
  // the constant address space: the bias is read-only for the launch, and
  // otherwise the compiler cannot prove it and falls back to vector loads)
  auto bload = [&](int row) -> float {
    typedef __attribute__((address_space(4))) const float ConstF;
    const int p = prob(row);
    const float *b = bias_of(p);
    if constexpr (kDyn) return (b != nullptr && row < end) ? ((ConstF *)b)[row - first_row(p)] : 0.0f;
    return (b != nullptr && row < end) ? b[row - first_row(p)] : 0.0f;
  };
  auto store = [&](int row, int r, float v) {
    const int p = prob(row);
    y_of(p)[(size_t)r * rows_of(p) + (row - first_row(p))] = v;
  };
  auto wbase_of = [&](int p) { return rec(p).w; };
  // The output of (row, activation row r) from lane 0 of a wave: a
  // range-checked buffer store whose other lanes (and rows that store
  // nothing) address past the end, where the hardware drops them, so no
  // branch on the lane surrounds it.
  auto store_l0 = [&](int row, int r, float v, bool ok) {
    const GemvMat m = rec(prob(row));
    const uint32_t yb = (uint32_t)nrows * (uint32_t)m.rows * 4u;
    const uint32_t off = lane == 0 && ok ? ((uint32_t)r * (uint32_t)m.rows + (uint32_t)(row - m.first)) * 4u : yb;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), make_rsrc(m.y, yb), off, 0, 0);
  };
  // The IEEE path, taken by the whole launch when some activation row holds
  // an infinity or a NaN (bit r of `slow`).  Team g's rows are shared out
  // step by step among its T waves, and each wave computes whole rows, 64
  // units at a time in the team's unit order.  Rows of a flagged activation
  // row are contracted in f32 with every weight dequantised exactly (the
  // reference's products, so its infinities and NaNs); the other rows repeat
  // the integer path's computation and summation order, bit for bit.
  auto ieee_rows = [&](unsigned slow_rows, unsigned wide_rows) {
    auto xval = [&](int r, int k) -> float {
      const float v = x[(size_t)r * K + k];
      if constexpr (kPro == kProRms) return v * inv_rms * P.a[k];
      if constexpr (kPro == kProSwiGLU) {
        const float sig = 1.0f / (1.0f + expf(-v));
        return (v * sig) * P.a[k];
      }
      return v;
    };
    for (int st = w; st < steps; st += T) {
      const int row = row_of(st);
      if (row >= end) break;
      const int p = prob(row);
      const uint32_t roff = (uint32_t)(row - first_row(p)) * rb;
      const uint8_t *rowp = wbase_of(p) + roff;
      const float bv = bload(row);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (r >= nrows) break;
        float tot = 0.0f;
        for (int q = 0; q < T; ++q) {
          const int uq = 64 * q + (int)lane;
          float acc = 0.0f;
          if ((slow_rows >> r) & 1u) {
            if (uq < U) {
              for (int e = 0; e < 64; ++e) {
                const int k = F::kidx(uq, e);
                acc = acc + xval(r, k) * deq_elem(F::kType, rowp, (uint32_t)k);
              }
            }
          } else {
            typename F::Regs Rg;
            F::load(Rg, rsrc(p), uq < U ? roff + F::unit_off(uq) : bytes_of(p), lane);
            if (uq < U)
              acc = F::compute(Rg, xr[r * U + uq], (const LdsU32 *)xr[r * U + uq].lo, (wide_rows >> r) & 1u, lane);
          }
          const float sum = wave_sum(acc);
          tot = T == 1 ? sum : tot + sum;
        }
        if (lane == 0) store(row, r, tot + bv);
      }
    }
  };

  // 1. activations first, XV float4s per thread (launch: XV * threads >= K/4;
  //    loads past the end of x return zeros without a memory access).  The
  //    CU serves vector loads in issue order, so the bare barrier below puts
  //    every wave's x loads ahead of all weight loads: x arrives after one
  //    cache round trip instead of behind the first rows of weights.
  const int nf = K >> 2;
  u32x4a4 xv[R][XV];
  u32x4a4 av[kPro != kProNone ? XV : 1];
#pragma unroll
  for (int r = 0; r < R; ++r) {  // rows r >= nrows get an empty range: zeros
    const Rsrc rx = make_rsrc(x + (size_t)r * K, r < nrows ? (uint32_t)K * 4u : 0u);
#pragma unroll
    for (int i = 0; i < XV; ++i) xv[r][i] = ld4(rx, 16u * (uint32_t)min(tid + i * nt, nf));
  }
  if constexpr (kPro != kProNone) {
    const Rsrc ra = make_rsrc(P.a, (uint32_t)K * 4u);
#pragma unroll
    for (int i = 0; i < XV; ++i) av[i] = ld4(ra, 16u * (uint32_t)min(tid + i * nt, nf));
  }
  __builtin_amdgcn_s_barrier();

  // 2. the first row of weights; the rest of the ring once the activations
  //    are quantised.  With all 16 waves' full rings in flight the CU's
  //    vector-memory queue is full and a wave that still has loads to issue
  //    stalls, holding up the quantisation barrier (measured against the
  //    whole ring early: gate+up 15.5 -> 14.9 us, down 10.5 -> 9.9 us; the
  //    whole ring late: C2 step +2%).  (The loop form matters: written as a
  //    single statement, the one-row launches compiled to code 0.2-0.6 us
  //    slower.)
  typename F::Regs S[D];
  float bs[D];
#pragma unroll
  for (int j = 0; j < 1; ++j) {
    wload(S[j], row_of(j));
    bs[j] = bload(row_of(j));
  }

  // 3. (optional neighbour transform, then) quantise x into LDS while the
  //    weights stream in.  Values past the end of x are zeros and stay zeros.
  if constexpr (kPro == kProRms) {
    // sum of squares: per thread, per wave (DPP), then the waves' partials in
    // wave order, so every workgroup gets the same value
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const float a0 = as_f32(xv[0][i].x), a1 = as_f32(xv[0][i].y), a2 = as_f32(xv[0][i].z), a3 = as_f32(xv[0][i].w);
      ss += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
    }
    ss = wave_sum(ss);
    float *red = part + (T > 1 ? kPartChunk * G * T : 0);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int q = 0; q < (nt >> 6); ++q) tot += red[q];
    const float inv = 1.0f / sqrtf(tot / (float)K + P.eps);  // rms = sqrt(mean + eps), then 1 / rms
    inv_rms = inv;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      xv[0][i].x = as_u32(as_f32(xv[0][i].x) * inv * as_f32(av[i].x));
      xv[0][i].y = as_u32(as_f32(xv[0][i].y) * inv * as_f32(av[i].y));
      xv[0][i].z = as_u32(as_f32(xv[0][i].z) * inv * as_f32(av[i].z));
      xv[0][i].w = as_u32(as_f32(xv[0][i].w) * inv * as_f32(av[i].w));
    }
  } else if constexpr (kPro == kProSwiGLU) {
    auto gate = [](uint32_t gb, uint32_t ub) {
      const float gv = as_f32(gb);
      const float sig = 1.0f / (1.0f + expf(-gv));
      return as_u32((gv * sig) * as_f32(ub));
    };
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      xv[0][i].x = gate(xv[0][i].x, av[i].x);
      xv[0][i].y = gate(xv[0][i].y, av[i].y);
      xv[0][i].z = gate(xv[0][i].z, av[i].z);
      xv[0][i].w = gate(xv[0][i].w, av[i].w);
    }
  }
  // 4. stream the rows, contracting two or all three limbs of each
  //    activation row (the low limb only for rows with a wide run: a
  //    wave-uniform branch inside the contraction)
  auto stream_rows = [&](unsigned wide_rows) {
    XRec xreg[R];
    const LdsU32 *xlo[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      xreg[r] = active ? xr[r * U + u] : XRec{};
      xlo[r] = (const LdsU32 *)xr[r * U + (active ? u : 0)].lo;
    }

    // Teams of several waves (T > 1) park each row's per-wave sums in LDS and
    // reduce them kChunk steps at a time, one barrier per chunk.
    constexpr int kChunk = kPartChunk;
    auto flush = [&](int step_end) {  // rows of steps [step_end - n, step_end), n = ((step_end - 1) % kChunk) + 1
      __syncthreads();
      const int first = (step_end - 1) / kChunk * kChunk;
      const int n = (step_end - first) * R;  // (step, activation row) pairs
      if (w == 0) {
        for (int l = (int)lane; l < n; l += 64) {
          const int st = first + l / R, r = l % R;
          const int row = row_of(st);
          if (row < end && r < nrows) {
            const float *pp = part + ((size_t)(st % kChunk) * G + g) * T * R + r;
            float t = 0.0f;
            for (int q = 0; q < T; ++q) t += pp[q * R];
            const int p = prob(row);
            const float *b = bias_of(p);
            store(row, r, t + (b != nullptr ? b[row - first_row(p)] : 0.0f));
          }
        }
      }
      __syncthreads();  // the slots are rewritten by the next chunk
    };
    auto finish = [&](const typename F::Regs &Q, float b, int step) {
      const int row = row_of(step);
      // idle lanes and rows past the end hold zero activations or read zero
      // weights, so the compute needs no branch around it
      float acc[R];
  #pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = F::compute(Q, xreg[r], xlo[r], (wide_rows >> r) & 1u, lane);  // the weight unpack is shared
      float sum[R];
  #pragma unroll
      for (int r = 0; r < R; ++r) sum[r] = wave_sum(acc[r]);
      if (T == 1) {
  #pragma unroll
        for (int r = 0; r < R; ++r) store_l0(row, r, sum[r] + b, row < end && r < nrows);
      } else {
        if (lane == 0) {
  #pragma unroll
          for (int r = 0; r < R; ++r) part[((size_t)(step % kChunk) * G + g) * T * R + w * R + r] = sum[r];
        }
        if ((step + 1) % kChunk == 0) flush(step + 1);
      }
    };

    if constexpr (kDyn) {
      // Ring slot j holds row ring_row[j]; a wave's rows increase in slot
      // order.  Idle lanes read zeros and hold zero activations, so the compute
      // needs no branch on the lane (a divergent branch here, like an exit
      // between slots, makes the compiler wait for every load in flight).  The
      // loop runs while all D slots hold rows (the last slot has the largest);
      // the drain consumes the rest without loads.
      int ring_row[D];
  #pragma unroll
      for (int j = 0; j < D; ++j) ring_row[j] = row_of(j);
      auto consume = [&](int j) {
        const int row = ring_row[j];
        float acc[R];
  #pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = F::compute(S[j], xreg[r], xlo[r], (wide_rows >> r) & 1u, lane);
        float sum[R];
  #pragma unroll
        for (int r = 0; r < R; ++r) sum[r] = wave_sum(acc[r]);
        // lane 0 alone stores here: a store by every lane (the others
        // dropped past the end) made the one-row ring of the Q6_K head 8%
        // slower
        if (lane == 0 && row < end) {
  #pragma unroll
          for (int r = 0; r < R; ++r)
            if (r < nrows) store(row, r, sum[r] + bs[j]);
        }
      };
      const int nb = (int)gridDim.x, bi = (int)blockIdx.x;
      while (ring_row[D - 1] < end) {
  #pragma unroll
        for (int j = 0; j < D; ++j) {
          unsigned c = 0;
          if (lane == 0) {
            // LDS add with return, written out so that the compiler sees no
            // atomic (one makes it drop the scalar bias loads); the wait is
            // part of the statement because the compiler cannot track it
            const uint32_t addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned *)&next_row;
            asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)" : "=v"(c) : "v"(addr), "v"(1u));
          }
          consume(j);
          c = (unsigned)__builtin_amdgcn_readfirstlane((int)c);  // the c-th row of the workgroup, step-major
          const int cs = (int)(c / (unsigned)G);
          const int nrow = (cs * nb + bi) * G + (int)(c - (unsigned)cs * (unsigned)G);
          ring_row[j] = nrow;
          wload(S[j], nrow);
          bs[j] = bload(nrow);
        }
      }
  #pragma unroll
      for (int j = 0; j < D; ++j)
        if (ring_row[j] < end) consume(j);
      return;
    }

    // 4. stream: consume ring slot j, then refill it D steps ahead.  The loads
    //    stay unconditional (control flow around loads makes the compiler wait
    //    for all of them); the last pass may fetch up to D - 1 rows past the
    //    range, which read zeros.  The final D rows are drained without loads.
    int s0 = 0;
    for (; s0 + D < steps; s0 += D) {
  #pragma unroll
      for (int j = 0; j < D; ++j) {
        finish(S[j], bs[j], s0 + j);
        wload(S[j], row_of(s0 + j + D));
        bs[j] = bload(row_of(s0 + j + D));
      }
    }
  #pragma unroll
    for (int j = 0; j < D; ++j)
      if (s0 + j < steps) finish(S[j], bs[j], s0 + j);
    if (T > 1 && steps % kChunk != 0) flush(steps);
  };

  // Run status (quant_group): bit 2r = some run of activation row r is wide,
  // bit 2r + 1 = some run of row r is not finite.  Each wave ORs its lanes'
  // bits into its own LDS slot (every slot is written, so none needs
  // clearing); after the barrier every wave ORs all slots, so the decision is
  // the same in every wave of every workgroup (all quantised the same x).
  unsigned qst = 0u;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < XV; ++i) qst |= quant_group<F>(xv[r][i], tid + i * nt, nf, xr + r * U) << (2 * r);
  unsigned wst = 0u;
#pragma unroll
  for (int b = 0; b < 2 * R; ++b)
    if (__ballot((qst >> b) & 1u) != 0ull) wst |= 1u << b;
  if (lane == 0) qflags[wave] = wst;
  if (kDyn && tid == 0) next_row = (unsigned)(D * G);
  __syncthreads();
  if (g >= G) return;  // helper wave (T == 1: no barriers follow)
  {
#pragma unroll
    for (int j = 1; j < D; ++j) {
      wload(S[j], row_of(j));
      bs[j] = bload(row_of(j));
    }
  }
  unsigned st_all = 0u;
  for (int q = 0; q < (nt >> 6); ++q) st_all |= qflags[q];
  st_all = (unsigned)__builtin_amdgcn_readfirstlane((int)st_all);
  unsigned slow = 0u, wide = 0u;  // activation rows holding an infinity or a NaN; a wide run
#pragma unroll
  for (int r = 0; r < R; ++r) {
    slow |= ((st_all >> (2 * r + 1)) & 1u) << r;
    wide |= ((st_all >> (2 * r)) & 1u) << r;
  }
  // Every run narrow (max|x| <= 8 mean|x|): two limbs, the 16-bit
  // quantisation, keep each activation within 2^-12 of its run's mean
  // magnitude; a wide run (an outlier channel) makes the launch contract all
  // three limbs, 2^-23 of the run maximum.
  if (slow != 0u) {
    ieee_rows(slow, wide);
    return;
  }
  stream_rows(wide);
}

// ---------------------------------------------------------------------------
// General fallback (any block-aligned K, 2-byte-aligned blocks): one wave per
// row, lanes stride over elements with byte loads and fp32 FMA.  Used for
// rows longer than 16 waves of units (K > 65536), tensors of 4 GiB or more,
// and Q8_0 rows that are not dword aligned (an odd number of blocks per row).
// ---------------------------------------------------------------------------
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
    for (int k = lane; k < K; k += 64) acc = fmaf(x[k], deq_elem(type, base, (uint32_t)k), acc);  // explicit FMA
    const float s = wave_sum(acc);
    if (lane == 0) y[row] = s + (bias ? bias[row] : 0.0f);
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
// The matrices of one launch: matrix 0 in the kernel arguments, the rest in M.
struct GemvLaunch {
  const uint8_t *w;
  uint32_t bytes;
  const float *bias;
  float *y;
  int rows;  // total over all matrices
  bool multi;
  GemvMore M;
  GemvPro P;
  int nrows;  // activation rows of this launch (<= R)
  bool dyn;   // dynamic rows (T == 1 and more than kDynSteps steps)
};

// One instantiation: the dynamic-row kernel where the launch asks for it and
// its shape is one the dynamic kernels are built for (one wave per row means
// K <= 4096, so at most two float4s of x per thread, and the full ring).
template <class F, int D, int XV, bool kMulti, int kPro, int R>
void launch_kernel(dim3 grid, dim3 block, size_t lds, hipStream_t s, const GemvLaunch &L, const float *x, int k,
                   int T, int G) {
  if constexpr (XV <= 2 && D == F::kMaxDepth) {
    if (L.dyn && T == 1) {
      launch_timed(gemv_kernel<F, D, XV, kMulti, kPro, R, true>, grid, block, (unsigned)lds, s, L.w, L.bytes, x,
                   L.bias, L.y, L.rows, k, T, G, L.M, L.P, L.nrows);
      return;
    }
  }
  launch_timed(gemv_kernel<F, D, XV, kMulti, kPro, R, false>, grid, block, (unsigned)lds, s, L.w, L.bytes, x, L.bias,
               L.y, L.rows, k, T, G, L.M, L.P, L.nrows);
}

template <class F, int D, int XV, bool kMulti, int R>
void launch_pro(dim3 grid, dim3 block, size_t lds, hipStream_t s, const GemvLaunch &L, const float *x, int k, int T,
                int G) {
  if constexpr (R == 1) {
    if (L.P.kind == kProRms) return launch_kernel<F, D, XV, kMulti, kProRms, 1>(grid, block, lds, s, L, x, k, T, G);
    if (L.P.kind == kProSwiGLU)
      return launch_kernel<F, D, XV, kMulti, kProSwiGLU, 1>(grid, block, lds, s, L, x, k, T, G);
  }
  launch_kernel<F, D, XV, kMulti, kProNone, R>(grid, block, lds, s, L, x, k, T, G);
}

template <class F, int D, int XV, int R>
void launch_multi(dim3 grid, dim3 block, size_t lds, hipStream_t s, const GemvLaunch &L, const float *x, int k, int T,
                  int G) {
  if (L.multi) launch_pro<F, D, XV, true, R>(grid, block, lds, s, L, x, k, T, G);
  else launch_pro<F, D, XV, false, R>(grid, block, lds, s, L, x, k, T, G);
}

// Ring depth: the format's maximum when every wave has that many rows to
// stream and more than two, else 1 (a deeper ring than the row count would
// only issue loads past the range; at two rows per wave the one-row ring
// measured faster: C2 q+k+v 6.60 -> 6.23 us).  Multi-row launches always use
// the maximum.
template <class F, int XV, int R>
void launch_depth(int64_t steps, dim3 grid, dim3 block, size_t lds, hipStream_t s, const GemvLaunch &L,
                  const float *x, int k, int T, int G) {
  if constexpr (R > 1) {
    launch_multi<F, F::kMaxDepth, XV, R>(grid, block, lds, s, L, x, k, T, G);
  } else {
    if (steps >= F::kMaxDepth && steps > 2) launch_multi<F, F::kMaxDepth, XV, 1>(grid, block, lds, s, L, x, k, T, G);
    else launch_multi<F, 1, XV, 1>(grid, block, lds, s, L, x, k, T, G);
  }
}

template <class F, int R>
void launch_xv(int xv, int64_t steps, dim3 grid, dim3 block, size_t lds, hipStream_t s, const GemvLaunch &L,
               const float *x, int k, int T, int G) {
  if (xv <= 1) launch_depth<F, 1, R>(steps, grid, block, lds, s, L, x, k, T, G);
  else if (xv == 2) launch_depth<F, 2, R>(steps, grid, block, lds, s, L, x, k, T, G);
  else if (xv <= 4) launch_depth<F, 4, R>(steps, grid, block, lds, s, L, x, k, T, G);
  else if constexpr (R > 1) launch_depth<F, 8, R>(steps, grid, block, lds, s, L, x, k, T, G);
}

template <class F>
void launch_rows(int R, int xv, int64_t steps, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                 const GemvLaunch &L, const float *x, int k, int T, int G) {
  if (R == 1) launch_xv<F, 1>(xv, steps, grid, block, lds, s, L, x, k, T, G);
  else if (R == 2) launch_xv<F, 2>(xv, steps, grid, block, lds, s, L, x, k, T, G);
  else launch_xv<F, 4>(xv, steps, grid, block, lds, s, L, x, k, T, G);
}

namespace {

size_t row_bytes_of(int type, int64_t K) {
  return (size_t)(type == kQ8_0 ? (K / 32) * kQ8Bytes
                                : (K / 256) * (type == kQ4_K ? kQ4KBytes : type == kQ5_K ? kQ5KBytes : kQ6KBytes));
}

// Conditions of the streaming kernel for one matrix: aligned base, a 32-bit
// tensor size, and K within the x prologue's reach.
bool fast_ok(int type, int64_t K, const void *w, int64_t N) {
  const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
  const size_t bytes = (size_t)N * row_bytes_of(type, K);
  bool fast = (K % 64 == 0) && K <= 4 * kMaxXV * 1024 && bytes < 0xFFFFFFFFull;
  if (type == kQ4_K || type == kQ5_K) fast = fast && (wa & 15u) == 0;
  else if (type == kQ6_K) fast = fast && (wa & 3u) == 0 && bytes % 4 == 0;  // the last block 2 bytes off a dword
  else fast = fast && (wa & 3u) == 0 && ((K / 32) % 2 == 0);
  return fast;
}

hipError_t launch_generic(int type, const float *x, int64_t K, const void *w, int64_t N, const float *bias, float *y,
                          int cu_count, hipStream_t s) {
  int64_t blocks = (N + 3) / 4;
  if (blocks > (int64_t)cu_count * 4) blocks = (int64_t)cu_count * 4;
  if (blocks < 1) blocks = 1;
  launch_timed(gemv_generic_kernel, dim3((unsigned)blocks), dim3(256), 0u, s, type, static_cast<const uint8_t *>(w),
               x, bias, y, (int)N, (int)K, row_bytes_of(type, K));
  return hipGetLastError();
}

// One streaming launch over the concatenated rows of P (all matrices pass
// fast_ok) for R activation rows (P.nrows of them real).
hipError_t launch_stream(int type, const float *x, int64_t K, const GemvLaunch &P, int R, int cu_count,
                         hipStream_t s) {
  const int64_t N = P.rows;
  const int U = (int)(K / 64);
  const int T = (U + 63) / 64;  // waves per row team
  const int max_threads = R == 1 ? gemv_max_threads<1>() : gemv_max_threads<4>();
  const int max_xv = R == 1 ? kMaxXV : kMaxXVRows;
  // one workgroup per CU (fewer for short tensors); steps = rows per team at
  // the largest team count, then the fewest teams that still finish in that
  // many steps (so the last window is as full as possible)
  int64_t blocks = std::min<int64_t>(cu_count, N);
  const int64_t max_g = std::max(1, max_threads / 64 / T);
  const int64_t steps0 = (N + blocks * max_g - 1) / (blocks * max_g);
  int64_t G = std::max<int64_t>(1, std::min<int64_t>(max_g, (N + blocks * steps0 - 1) / (blocks * steps0)));
  // Every thread quantises at most max_xv float4s of each x row: with T == 1
  // extra helper waves cover x, with teams (T > 1) extra teams do (teams
  // without rows stream nothing; K <= 16384 keeps this within the limit).
  const int64_t x_threads = (K / 4 + max_xv - 1) / max_xv;
  if (T > 1) G = std::max<int64_t>(G, (x_threads + 64 * T - 1) / (64 * T));
  blocks = std::min<int64_t>(blocks, (N + G * steps0 - 1) / (G * steps0));
  int64_t threads = 64 * T * G;
  if (T == 1) threads = std::min<int64_t>(max_threads, std::max(threads, (x_threads + 63) / 64 * 64));
  const int xv = (int)((K / 4 + threads - 1) / threads);
  if (xv > max_xv || threads > max_threads) return hipErrorInvalidConfiguration;  // excluded by fast_ok's K bound
  const dim3 grid((unsigned)blocks), block((unsigned)threads);
  const size_t lds = (size_t)R * U * sizeof(XRec) + (T > 1 ? sizeof(float) * kPartChunk * G * T * R : 0) +
                     (P.P.kind == kProRms ? sizeof(float) * 16 : 0);
  const int k = (int)K, gg = (int)G;
  GemvLaunch L = P;
  const int64_t steps = (N + blocks * G - 1) / (blocks * G);  // the kernel's own count
  L.dyn = T == 1 && steps > kDynSteps;
  if (type == kQ4_K) launch_rows<FQ4K>(R, xv, steps0, grid, block, lds, s, L, x, k, T, gg);
  else if (type == kQ5_K) launch_rows<FQ5K>(R, xv, steps0, grid, block, lds, s, L, x, k, T, gg);
  else if (type == kQ6_K) launch_rows<FQ6K>(R, xv, steps0, grid, block, lds, s, L, x, k, T, gg);
  else launch_rows<FQ80>(R, xv, steps0, grid, block, lds, s, L, x, k, T, gg);
  return hipGetLastError();
}

}  // namespace

bool gemv_streams(int type, int64_t K, const void *w, int64_t N) { return fast_ok(type, K, w, N); }

hipError_t launch_gemv_multi(int type, const float *x, int64_t K, int64_t rows, int count, const void *const *w,
                             const int64_t *N, const float *const *bias, float *const *y, int cu_count,
                             hipStream_t s, const GemvPro &pro) {
  if (type != kQ4_K && type != kQ5_K && type != kQ6_K && type != kQ8_0) return hipErrorInvalidValue;
  if (count < 1 || count > kGemvMaxProblems) return hipErrorInvalidValue;
  if (pro.kind != kProNone && rows != 1) return hipErrorNotSupported;  // prologues run one row at a time
  GemvLaunch P{};
  P.P = pro;
  int64_t total = 0;
  bool fast = true;
  for (int i = 0; i < count; ++i) {
    fast = fast && fast_ok(type, K, w[i], N[i]);
    total += N[i];
  }
  fast = fast && total < (int64_t)INT32_MAX;
  if (!fast && pro.kind != kProNone) return hipErrorNotSupported;  // callers check gemv_streams first
  if (!fast) {  // matrix by matrix, each on its own best path
    for (int i = 0; i < count; ++i) {
      if (N[i] == 0) continue;
      hipError_t e = hipSuccess;
      if (fast_ok(type, K, w[i], N[i])) {
        e = launch_gemv_multi(type, x, K, rows, 1, &w[i], &N[i], &bias[i], &y[i], cu_count, s, pro);
      } else {
        for (int64_t r = 0; r < rows && e == hipSuccess; ++r)
          e = launch_generic(type, x + r * K, K, w[i], N[i], bias[i], y[i] + r * N[i], cu_count, s);
      }
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  P.w = static_cast<const uint8_t *>(w[0]);
  P.bytes = (uint32_t)((size_t)N[0] * row_bytes_of(type, K));
  P.bias = bias[0];
  P.multi = count > 1;
  int64_t start = 0;
  for (int i = 0; i < kGemvMaxProblems; ++i) {
    GemvMat &m = P.M.mat[i];
    if (i < count) {
      m.w = static_cast<const uint8_t *>(w[i]);
      m.bytes = (uint32_t)((size_t)N[i] * row_bytes_of(type, K));
      m.bias = bias[i];
      m.first = (int)start;
      m.rows = (int)N[i];
      if (i > 0) P.M.start[i - 1] = (int)start;
      start += N[i];
    } else {
      m = GemvMat{nullptr, nullptr, nullptr, 0u, INT32_MAX, 0, 0};
      P.M.start[i - 1] = INT32_MAX;
    }
  }
  P.rows = (int)total;
  if (total == 0) return hipSuccess;
  // up to kMaxRowsPerLaunch activation rows per pass over the weights, as
  // many as the LDS holds: R rows of XRecs plus the teams' partial sums
  // (<= 8 waves x kPartChunk x R floats) within 160 KiB
  const int64_t U = K / 64;
  int per_launch = kMaxRowsPerLaunch;
  while (per_launch > 1 && (size_t)per_launch * (U * sizeof(XRec) + sizeof(float) * kPartChunk * 8) + 64 > kLdsBytes)
    per_launch /= 2;
  for (int64_t r0 = 0; r0 < rows; r0 += per_launch) {
    const int nr = (int)std::min<int64_t>(per_launch, rows - r0);
    P.nrows = nr;
    P.y = y[0] + r0 * N[0];
    for (int i = 0; i < count; ++i) P.M.mat[i].y = y[i] + r0 * N[i];
    const int R = nr == 1 ? 1 : nr == 2 ? 2 : 4;
    hipError_t e = launch_stream(type, x + r0 * K, K, P, R, cu_count, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_gemv(int type, const float *x, int64_t K, const void *w, int64_t N, const float *bias, float *y,
                       int cu_count, hipStream_t s) {
  return launch_gemv_multi(type, x, K, 1, 1, &w, &N, &bias, &y, cu_count, s, GemvPro{});
}

}  // namespace okq
