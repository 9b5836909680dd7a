// okq_gemm_pair.hip -- Q4_K (and Q5_K) prefill dequant-GEMM, weights
// dequantised in registers, two 4-wave workgroups per CU:
// Y[M,N] = X[M,K] W[N,K]^T (+bias).
//
// Operands and numerics are those of gemm_wide_q4k_kernel (okq_gemm_wide.hip):
// A = the pre-pass's row-scaled fp16 activations, B = sc * q exact in fp16,
// every product exact, f32 accumulation; d applied per super-block in f32;
// the min term  -sum dmin m_j xsum_j  contracted by MFMAs straight into the
// output accumulator from exact (hi, lo) fp16 planes of dmin * m and of the
// per-32 sums.
//
// What differs is the unit of synchronisation.  A workgroup is four waves,
// one per SIMD, on a 128 x 128 tile (wave w: columns 32w .. 32w+31, all 128
// rows, four 32x32x16 MFMA blocks per B fragment), and a stage is half a
// super-block (128 K), so its double-buffered activation stages (2 x 34 KB)
// let two workgroups share a CU.  The two waves of a SIMD then belong to
// different workgroups: a barrier holds only the four waves of its own tile,
// and while they wait the other workgroup's wave keeps the SIMD's MFMA pipe
// fed (with one 8-wave workgroup per CU, every super-block's barrier left the
// SIMD with the slower wave of its pair alone).
//
//   * Stage (super-block sb, half h), MFMA step s (0..7), lane group g:
//     k = 256 sb + 128 h + 64 g + 8 s + [0, 8), the nibble plane s / 4 of qs
//     bytes 8 (s & 3) .. of 64-element chunk 2h + g.  A lane reads the 32 qs
//     bytes of its chunk per stage (two 16-byte loads, one stage ahead, in
//     the register set of the stage's parity) and the 16-byte header per
//     super-block (one super-block ahead, two register sets).
//   * Activations: 128 rows x 256 bytes per stage, 16-byte chunk c of row r
//     at chunk c ^ (r & 15) (conflict-free fragment reads), copied by
//     buffer-to-LDS loads one stage ahead; the stage's per-32 sums
//     (4 (hi, lo) pairs per row) ride along.
//   * Min term: one MFMA per row block per stage: lane group g holds
//     (xh, xl, xh, xl) of its two sub-blocks against (-ph, -ph, -pl, -pl).
//   * acc += d * accs after the second half of every super-block.
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef __attribute__((address_space(3))) void *LdsPtr;

constexpr int kPM = 128;  // tile rows
constexpr int kPN = 128;  // tile columns (4 waves x 32)

__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Activation stages: two buffers of [128 rows][128 halves] (swizzled 16-byte
// chunks) and [128 rows][4 (hi, lo) per-32 sums]; distinct objects, so that
// the fragment reads of one do not wait for the loads into the other.
__shared__ __attribute__((aligned(16))) _Float16 pA0[kPM * 128];
__shared__ __attribute__((aligned(16))) _Float16 pA1[kPM * 128];
__shared__ __attribute__((aligned(16))) _Float16 pX0[kPM * 8];
__shared__ __attribute__((aligned(16))) _Float16 pX1[kPM * 8];
// the tile's row scales for the epilogue
__shared__ __attribute__((aligned(16))) float pR[kPM];

// 0x6400 | q is the fp16 1024 + q; (1024 + q) * sc - 1024 * sc = sc * q is one
// fused fp16 FMA with an exact integer result (<= 945).
__device__ __forceinline__ h2 nib_pair(uint32_t spread, h2 sc2, h2 off2) {
  return __builtin_elementwise_fma(__builtin_bit_cast(h2, spread), sc2, off2);
}

}  // namespace

// The kernel body for Q4_K (kQ5 = false) and Q5_K (kQ5: the fifth bit of
// every weight from the block's qh bytes, as in okq_gemm_wide.hip).
template <bool kQ5>
__device__ __forceinline__ void pair_body(const _Float16 *__restrict__ xhi, const h2 *__restrict__ xsum,
                                          const float *__restrict__ rscale, const uint8_t *__restrict__ W,
                                          const float *__restrict__ bias, float *__restrict__ Y, int M, int N, int K,
                                          int tiles_m, int tiles, int ksplit, float *__restrict__ part) {
  constexpr uint32_t kSB = kQ5 ? kQ5KBytes : kQ4KBytes;  // bytes per super-block
  // XCD-aware order: workgroup b runs on XCD b % 8; each XCD takes a
  // contiguous range of (slice, tile) jobs, and consecutive jobs are the
  // M-tiles of one N-tile (they share its weights in that XCD's L2).
  const int b = (int)blockIdx.x;
  const int jobs = tiles * ksplit;
  const int per_xcd = (jobs + 7) / 8;
  const int job = (b % 8) * per_xcd + b / 8;
  if (job >= jobs) return;
  const int z = job / tiles, tile = job % tiles;
  const int m0 = (tile % tiles_m) * kPM;
  const int n0 = (tile / tiles_m) * kPN;

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, cl = lane & 31;
  const int nsb_all = K >> 8;
  const int sb0 = (int)((int64_t)z * nsb_all / ksplit);
  const int nst = 2 * ((int)((int64_t)(z + 1) * nsb_all / ksplit) - sb0);  // stages (half super-blocks)
  const uint32_t row_bytes = (uint32_t)nsb_all * kSB;
  const uint32_t K2 = (uint32_t)K * 2u;

  const Rsrc rs_x = make_rsrc(xhi, (uint32_t)((size_t)M * K * 2));
  const Rsrc rs_s = make_rsrc(xsum, (uint32_t)((size_t)M * (K / 32) * 4));
  const Rsrc rs_w = make_rsrc(W, (uint32_t)((size_t)N * row_bytes));

  // Activation copy of stage st (super-block sb0 + st / 2, half st & 1):
  // wave w moves rows 32w .. 32w+31, four rows (1 KB) per instruction; lane
  // L of instruction t writes chunk L & 15 of row 32w + 4t + L/16, which
  // holds the row's logical chunk (L & 15) ^ (row & 15).  The sums (2 KB):
  // one instruction per wave, lane L of wave w takes the 16 bytes of row
  // 64 (w & 1) + L (waves 2-3 repeat waves 0-1 -- the same bytes to the same
  // place -- so every wave issues the same nine loads per stage).
  uint32_t a_off[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    a_off[t] = (uint32_t)(m0 + 32 * wave + (lane >> 4)) * K2 +
               16u * ((uint32_t)(lane & 15) ^ (uint32_t)(4 * t + (lane >> 4)));
  const uint32_t s_off = (uint32_t)(m0 + 64 * (wave & 1) + lane) * (uint32_t)(K / 32) * 4u;
  auto copy_piece = [&](int t, int st, _Float16 *bufA) {
    const uint32_t kb = (uint32_t)(sb0 * 256 + st * 128);  // first K of the stage
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, (LdsPtr)(bufA + (32 * wave + 4 * t) * 128), 16, a_off[t & 3],
                                             (int)((uint32_t)t * 4u * K2 + kb * 2u), 0, 0);
  };
  auto copy_sums = [&](int st, _Float16 *bufX) {
    const uint32_t kb = (uint32_t)(sb0 * 256 + st * 128);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_s, (LdsPtr)(bufX + 64 * (wave & 1) * 8), 16, s_off,
                                             (int)(kb / 8u), 0, 0);
  };

  // This lane's weight column n0 + 32w + cl (columns past N read past the
  // tensor: zeros): the 16-byte header of each super-block and, per stage,
  // the 32 qs bytes of chunk 2h + g.
  const uint32_t w_hd = (uint32_t)(n0 + 32 * wave + cl) * row_bytes;
  const uint32_t w_q = w_hd + (kQ5 ? 48u : 16u) + 32u * (uint32_t)g;
  auto ldw = [&](uint32_t voff, int sb) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs_w, voff, (int)((uint32_t)sb * kSB), 0);
  };
  // Q5_K: the 32 qh bytes of a super-block (hr0, hr1: loaded with its header,
  // one super-block ahead) and, for the current one, the 4 bits lane group g
  // uses of each -- bits 2g, 2g + 1 (half 0: chunk g) and 4 + 2g, 5 + 2g
  // (half 1: chunk 2 + g) -- packed as field bit 2h + plane, with bytes
  // 8j .. 8j + 3 in the low nibbles of hc[j] and 8j + 4 .. 8j + 7 in the high
  u32x4 hr0 = {}, hr1 = {};
  uint32_t hc[4] = {0u, 0u, 0u, 0u};
  auto compact_qh = [&]() {
    const uint32_t sh = 2u * (uint32_t)g;
    const uint32_t r[8] = {hr0.x, hr0.y, hr0.z, hr0.w, hr1.x, hr1.y, hr1.z, hr1.w};
    auto field = [&](uint32_t x) { return ((x >> sh) & 0x03030303u) | ((x >> (sh + 2u)) & 0x0C0C0C0Cu); };
#pragma unroll
    for (int j = 0; j < 4; ++j) hc[j] = field(r[2 * j]) | (field(r[2 * j + 1]) << 4);
  };
  auto ldq = [&](int st, u32x4 &q0, u32x4 &q1) {
    const int sb = sb0 + (st >> 1);
    const uint32_t o = w_q + 64u * (uint32_t)(st & 1);
    q0 = ldw(o, sb);
    q1 = ldw(o + 16u, sb);
  };
  u32x4 qe0, qe1, qo0, qo1, hdA, hdB;

  f16x acc[4], accs[4];
  const f16x zero = {};
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = zero;

  // A fragment of row block i at MFMA step s: row 32 i + cl, logical chunk
  // 8 g + s, stored at chunk (8 g + s) ^ (cl & 15)
  int a_lane = cl * 256 + 128 * (g ^ ((cl >> 3) & 1)), a_x = cl & 7;
  asm volatile("" : "+v"(a_lane), "+v"(a_x));
  auto a_addr = [&](int s) { return a_lane + 16 * (s ^ a_x); };
  auto a_at = [&](const _Float16 *bufA, int addr, int i) {
    return *reinterpret_cast<const h8 *>(reinterpret_cast<const char *>(bufA) + addr + 8192 * i);
  };

  // (sc, off) of sub-block j: low nibble planes take (sc, -1024 sc) on
  // 0x6400 | q = 1024 + q; high planes, masked in place (0x6400 | 16 q =
  // 1024 + 16 q), take (sc / 16, -64 sc): the fused product 64 sc + sc q is
  // exact and so is the result sc q.
  auto scales = [&](const u32x4 &hd, uint32_t j, bool high, h2 &sc2, h2 &off2) {
    uint32_t sc, mv;
    q4k_scale_min_sel(j, hd.y, hd.z, hd.w, sc, mv);
    const float f = (float)sc;
    const _Float16 sh = (_Float16)(high ? f * 0.0625f : f), oh = (_Float16)(high ? -64.0f * f : -1024.0f * f);
    sc2 = h2{sh, sh};
    off2 = h2{oh, oh};
  };
  // Q5_K's fifth bit (field bit 2h + s / 4 of byte l): bit 4 of the byte
  // on low planes (1024 + q5), the exponent byte 0x64 | h on high planes
  // (1024 + 256 h + 16 q4 = 1024 + 16 q5), so the scale pairs stay Q4_K's
  auto dequant = [&](int s, int h, const u32x4 &q0, const u32x4 &q1, h2 sc2, h2 off2) {
    const u32x4 qq = ((s & 3) >> 1) ? q1 : q0;
    const uint32_t d0 = (s & 1) ? qq.z : qq.x, d1 = (s & 1) ? qq.w : qq.y;
    const bool hi = (s >> 2) != 0;
    const uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    uint32_t n0v = d0 & mask, n1v = d1 & mask;
    uint32_t e0 = 0x64646464u, e1 = 0x64646464u;
    uint32_t s00 = 0x04010400u, s01 = 0x04030402u;
    if constexpr (kQ5) {
      const uint32_t b = 2u * (uint32_t)h + (uint32_t)(s >> 2);
      const uint32_t c = hc[s & 3];
      const uint32_t h0 = (c >> b) & 0x01010101u, h1 = (c >> (b + 4u)) & 0x01010101u;
      if (hi) {
        e0 |= h0;
        e1 |= h1;
        s00 = 0x05010400u;
        s01 = 0x07030602u;
      } else {
        n0v |= h0 << 4;
        n1v |= h1 << 4;
      }
    }
    const h2 p0 = nib_pair(__builtin_amdgcn_perm(e0, n0v, s00), sc2, off2);
    const h2 p1 = nib_pair(__builtin_amdgcn_perm(e0, n0v, s01), sc2, off2);
    const h2 p2 = nib_pair(__builtin_amdgcn_perm(e1, n1v, s00), sc2, off2);
    const h2 p3 = nib_pair(__builtin_amdgcn_perm(e1, n1v, s01), sc2, off2);
    return h8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  };

  // One stage (half h of a super-block with header hd, qs in (q0, q1)) from
  // (bufA, bufX): 8 MFMA steps of 4 MFMAs (accs restarts at the first half),
  // the min term of its four sub-blocks into acc, and after the second half
  // acc += d * accs.  Step s's MFMAs issue while the A fragments and the B
  // fragment of step s + 1 are read and dequantised, and steps 0-3 copy stage
  // st_next's activations into (nbufA, nbufX), two copy instructions per step
  // (all at once, the waves' copies queue at the vector memory unit and hold
  // back every wave's MFMAs at the start of the stage).
  auto contract = [&](const _Float16 *bufA, const _Float16 *bufX, const u32x4 &hd, const u32x4 &q0,
                      const u32x4 &q1, const int h, int st_next, _Float16 *nbufA, _Float16 *nbufX) {
    h8 a[4], an[4], bv;
    h2 sc2, off2;
    const uint32_t j0 = 4u * (uint32_t)h + 2u * (uint32_t)g;  // sub-block of the low nibble plane
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = a_at(bufA, a_addr(0), i);
    scales(hd, j0, false, sc2, off2);
    bv = dequant(0, h, q0, q1, sc2, off2);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s < 7) {
        const int ad = a_addr(s + 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) an[i] = a_at(bufA, ad, i);
      }
      if (s < 4) {
        copy_piece(2 * s, st_next, nbufA);
        copy_piece(2 * s + 1, st_next, nbufA);
        if (s == 3) copy_sums(st_next, nbufX);
      }
      // the next step's fragment reads issue ahead of this step's MFMAs (the
      // scheduler would otherwise sink them to their use)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        accs[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bv, (h == 0 && s == 0) ? zero : accs[i], 0, 0, 0);
      if (s < 7) {
        if (s + 1 == 4) scales(hd, j0 + 1u, true, sc2, off2);
        bv = dequant(s + 1, h, q0, q1, sc2, off2);
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = an[i];
      }
    }
    // min term of sub-blocks j0, j0 + 1: A = (xh, xl, xh, xl) of each,
    // B = (-ph, -ph, -pl, -pl) of each
    h8 xa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x2 p = *reinterpret_cast<const u32x2 *>(bufX + (32 * i + cl) * 8 + 4 * g);
      xa[i] = __builtin_bit_cast(h8, u32x4{p.x, p.x, p.y, p.y});
    }
    const float dmin = f16_bits_hw(hd.x >> 16);
    h8 mb;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      uint32_t sc, mv;
      q4k_scale_min_sel(j0 + (uint32_t)u, hd.y, hd.z, hd.w, sc, mv);
      const float prod = dmin * (float)mv;  // exact (<= 17 significant bits)
      const _Float16 ph = (_Float16)prod;
      const _Float16 pl = (_Float16)(prod - (float)ph);  // exact remainder
      mb[4 * u] = -ph;
      mb[4 * u + 1] = -ph;
      mb[4 * u + 2] = -pl;
      mb[4 * u + 3] = -pl;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[i], mb, acc[i], 0, 0, 0);
    if (h == 1) {
      const float dv = f16_bits_hw(hd.x & 0xffffu);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = __builtin_fmaf(dv, accs[i][e], acc[i][e]);
    }
  };

  // Pipeline, a period of four stages (buffers alternate per stage, qs
  // register sets per stage, header sets per super-block): stage st reads
  // buffer st & 1 while stage st + 1's qs go into the other register set (a
  // super-block's first stage also loads the next super-block's header) and
  // its activations into the other buffer.  Every stage issues the same loads
  // (past the last stage they reload it: idle buffer, dead registers), so the
  // compiler's load counts stay exact on every path; the qs and header loads
  // issue first, so the wait for every load before the stage's one barrier
  // waits for the copy, whose last piece left at step 3.
  const int last = nst - 1;
  auto cl_st = [&](int st) { return st < last ? st : last; };
  auto hd_sb = [&](int st) { return sb0 + (cl_st(st) >> 1); };
#pragma unroll
  for (int t = 0; t < 8; ++t) copy_piece(t, 0, pA0);
  copy_sums(0, pX0);
  if (tid < kPM) pR[tid] = m0 + tid < M ? rscale[m0 + tid] : 0.0f;
  hdA = ldw(w_hd, sb0);
  ldq(0, qe0, qe1);
  if constexpr (kQ5) {
    hr0 = ldw(w_hd + 16u, sb0);
    hr1 = ldw(w_hd + 32u, sb0);
  }
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  __syncthreads();
  // Q5_K: at a super-block's first stage its qh bits are packed, then the raw
  // registers take the next super-block's (with its header)
  auto next_qh = [&](int sb) {
    if constexpr (kQ5) {
      compact_qh();
      hr0 = ldw(w_hd + 16u, sb);
      hr1 = ldw(w_hd + 32u, sb);
    }
  };
  constexpr int kWaitAll = 0x0070;  // vmcnt(0) expcnt(7) lgkmcnt(0), gfx9 encoding
  for (int st = 0;; st += 4) {
    // stage st: first half of a super-block (header hdA), buffer 0, qs qe
    ldq(cl_st(st + 1), qo0, qo1);
    hdB = ldw(w_hd, hd_sb(st + 2));
    next_qh(hd_sb(st + 2));
    __builtin_amdgcn_sched_barrier(0);  // the prefetch issues first
    contract(pA0, pX0, hdA, qe0, qe1, 0, cl_st(st + 1), pA1, pX1);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    __builtin_amdgcn_s_barrier();
    // stage st + 1: second half (hdA), buffer 1, qs qo
    ldq(cl_st(st + 2), qe0, qe1);
    __builtin_amdgcn_sched_barrier(0);
    contract(pA1, pX1, hdA, qo0, qo1, 1, cl_st(st + 2), pA0, pX0);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    __builtin_amdgcn_s_barrier();
    if (st + 2 >= nst) break;
    // stage st + 2: first half of the next super-block (hdB), buffer 0, qs qe
    ldq(cl_st(st + 3), qo0, qo1);
    hdA = ldw(w_hd, hd_sb(st + 4));
    next_qh(hd_sb(st + 4));
    __builtin_amdgcn_sched_barrier(0);
    contract(pA0, pX0, hdB, qe0, qe1, 0, cl_st(st + 3), pA1, pX1);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    __builtin_amdgcn_s_barrier();
    // stage st + 3: second half (hdB), buffer 1, qs qo
    ldq(cl_st(st + 4), qe0, qe1);
    __builtin_amdgcn_sched_barrier(0);
    contract(pA1, pX1, hdB, qo0, qo1, 1, cl_st(st + 4), pA0, pX0);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    __builtin_amdgcn_s_barrier();
    if (st + 4 >= nst) break;
  }
  // The last stage's copy into the idle buffer and its reloads must land
  // before the workgroup's LDS is released.  The empty asm reads the
  // prefetched registers on the way out, so that the loads a stage issues
  // for the next one are live on both sides of the exit tests: the compiler
  // cannot sink them to just before their first use, where each would wait
  // out its latency.
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::"v"(hdA), "v"(hdB), "v"(qe0), "v"(qe1), "v"(qo0), "v"(qo1));
  if constexpr (kQ5) asm volatile("" ::"v"(hr0), "v"(hr1));

  // epilogue: lane (cl, g) holds rows 8 (e / 4) + 4 g + e % 4 of column cl
  // of each 32 x 32 block; split K stores the raw partial sums, otherwise the
  // row scale (from LDS) and the bias are applied.  A whole tile stores
  // without per-value row tests.
  const int col = n0 + 32 * wave + cl;
  const int rows = M - m0 < kPM ? M - m0 : kPM;
  // rows whose scale is NaN (computed by the pre-pass), tested by every lane
  // of the wave before any lane leaves for a column past N
  const bool flagged =
      __builtin_amdgcn_ballot_w64(__builtin_isnan(pR[lane]) || __builtin_isnan(pR[64 + lane])) != 0;
  if (col < N) {
    if (ksplit > 1) {
      float *dst = part + ((size_t)z * M + m0) * N + col;
      auto store = [&](bool guard) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
            if (!guard || r < rows) dst[(size_t)r * N] = acc[i][e];
          }
      };
      if (rows == kPM) {
        store(false);
      } else {
        store(true);
      }
    } else {
      const float bv = bias ? bias[col] : 0.0f;
      float *dst = Y + (size_t)m0 * N + col;
      // skip: rows whose scale is NaN hold an infinity or a NaN; the pre-pass
      // wrote their IEEE outputs (a wave-uniform test over the tile's scales,
      // so whole tiles keep the branch-free stores)
      auto store = [&](bool guard, bool skip) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r0 = 32 * i + 8 * j + 4 * g;
            const float4 rs = *reinterpret_cast<const float4 *>(pR + r0);
            const float rv[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if ((!guard || r0 + q < rows) && (!skip || !__builtin_isnan(rv[q])))
                dst[(size_t)(r0 + q) * N] = acc[i][4 * j + q] * rv[q] + bv;
          }
      };
      if (flagged) {
        store(true, true);
      } else if (rows == kPM) {
        store(false, false);
      } else {
        store(true, false);
      }
    }
  }
}

__global__ __launch_bounds__(256, 2) void gemm_pair_q4k_kernel(const _Float16 *__restrict__ xhi,
                                                               const h2 *__restrict__ xsum,
                                                               const float *__restrict__ rscale,
                                                               const uint8_t *__restrict__ W,
                                                               const float *__restrict__ bias, float *__restrict__ Y,
                                                               int M, int N, int K, int tiles_m, int tiles,
                                                               int ksplit, float *__restrict__ part) {
  pair_body<false>(xhi, xsum, rscale, W, bias, Y, M, N, K, tiles_m, tiles, ksplit, part);
}

__global__ __launch_bounds__(256, 2) void gemm_pair_q5k_kernel(const _Float16 *__restrict__ xhi,
                                                               const h2 *__restrict__ xsum,
                                                               const float *__restrict__ rscale,
                                                               const uint8_t *__restrict__ W,
                                                               const float *__restrict__ bias, float *__restrict__ Y,
                                                               int M, int N, int K, int tiles_m, int tiles,
                                                               int ksplit, float *__restrict__ part) {
  pair_body<true>(xhi, xsum, rscale, W, bias, Y, M, N, K, tiles_m, tiles, ksplit, part);
}

int gemm_pair_tiles(int64_t M, int64_t N) { return (int)(((M + kPM - 1) / kPM) * ((N + kPN - 1) / kPN)); }

hipError_t launch_gemm_pair(int type, const _Float16 *xhi, const void *xsum, const float *rscale, const void *w,
                            const float *bias, float *y, int64_t M, int64_t N, int64_t K, int ksplit, float *part,
                            hipStream_t s) {
  const int tiles_m = (int)((M + kPM - 1) / kPM);
  const int tiles = gemm_pair_tiles(M, N);
  const int per_xcd = (tiles * ksplit + 7) / 8;
  launch_timed(type == kQ5_K ? gemm_pair_q5k_kernel : gemm_pair_q4k_kernel, dim3((unsigned)(per_xcd * 8)), dim3(256),
               0u, s, xhi, static_cast<const h2 *>(xsum), rscale, static_cast<const uint8_t *>(w), bias, y, (int)M,
               (int)N, (int)K, tiles_m, tiles, ksplit, part);
  return hipGetLastError();
}

}  // namespace okq
