// okq_gemm_wide.hip -- Q4_K (and Q5_K) prefill dequant-GEMM with weights
// dequantised straight into MFMA registers: Y[M,N] = X[M,K] W[N,K]^T (+bias).
// Q5_K is the same contraction with the fifth bit of every weight taken from
// the block's 32 qh bytes (sc * q5 <= 1953 stays an exact fp16 integer).
//
// Operands and numerics are those of gemm_kq_kernel (okq_gemm.hip): A = the
// pre-pass's row-scaled fp16 activations, B = sc * q exact in fp16, every
// product exact, f32 accumulation; d is applied per super-block in f32.  The
// min term  -sum_sb dmin_sb sum_j m_j xsum_j  is contracted by MFMAs straight
// into the output accumulator: dmin * m (an fp16 times a 6-bit integer, at
// most 17 significant bits whose lowest is >= 2^-24) is the exact sum of two
// fp16 planes hi = fp16(dmin * m) and lo = fp16(dmin * m - hi), each
// multiplied by the per-32 sums (hi, lo) of the pre-pass.
//
// Layout / schedule (gfx950, one 8-wave workgroup per CU, two waves per SIMD):
//   * Workgroup tile 128 rows x 256 columns; wave w owns columns 32w .. 32w+31
//     of it for all 128 rows (four MFMA 32x32x16 blocks).  Each weight column
//     belongs to exactly one wave, which loads its GGUF blocks and dequantises
//     them into B fragments in registers: the weights never pass through LDS
//     and no two waves dequantise the same block (one weight serves 128 rows,
//     ~2.5 VALU instructions per MFMA).
//   * Only the activations are shared: one super-block (256 K) of the 128 rows
//     per stage, 64 KB of fp16 plus 4 KB of per-32 sums, copied into LDS by
//     buffer-to-LDS loads (no registers) one stage ahead into the other of two
//     buffers.  The 16-byte chunk c of row r sits at chunk c ^ (r & 15), so
//     the fragment reads of 16 consecutive rows hit distinct banks.
//   * K order inside a super-block: MFMA step s (0..15) and lane group
//     g = lane / 32 cover k = 128 g + 8 s + [0, 8), i.e. nibble plane (s/4)&1
//     of qs bytes 8 (s&3) .. of chunk 2g + s/8; a lane group reads its own
//     64 qs bytes of each block (plus the 16-byte header).
//   * Each step reads the next step's A fragments, issues its four MFMAs as
//     one cluster and then dequantises the next step's B fragment, so the two
//     waves of a SIMD overlap one's MFMAs with the other's VALU work.  Both
//     accumulator sets (per super-block and total, 64 values each) live in
//     VGPRs (built with -amdgpu-mfma-vgpr-form), so the per-super-block f32
//     scaling is plain FMAs.  One barrier per super-block.
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef __attribute__((address_space(3))) void *LdsPtr;

constexpr int kWM = 128;  // tile rows
constexpr int kWN = 256;  // tile columns (8 waves x 32)

__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload4(Rsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }

// Activation stages: two buffers of [128 rows][256 halves] (swizzled 16-byte
// chunks) and [128 rows][8 (hi, lo) per-32 sums].  Distinct objects, so that
// the fragment reads of one buffer do not wait for the loads into the other.
__shared__ __attribute__((aligned(16))) _Float16 wA0[kWM * 256];
__shared__ __attribute__((aligned(16))) _Float16 wA1[kWM * 256];
__shared__ __attribute__((aligned(16))) _Float16 wX0[kWM * 16];
__shared__ __attribute__((aligned(16))) _Float16 wX1[kWM * 16];
// The tile's row scales, read by the epilogue (four consecutive rows per
// 16-byte read) instead of one dependent global load per output value.
__shared__ __attribute__((aligned(16))) float wR[kWM];

// 0x6400 | q is the fp16 1024 + q; (1024 + q) * sc - 1024 * sc = sc * q is one
// fused fp16 FMA with an exact integer result (<= 945).
__device__ __forceinline__ h2 nib_pair(uint32_t spread, h2 sc2, h2 off2) {
  return __builtin_elementwise_fma(__builtin_bit_cast(h2, spread), sc2, off2);
}

}  // namespace

// The kernel body for Q4_K (kQ5 = false) and Q5_K (kQ5: the same with the
// fifth bit of every weight from the block's 32 qh bytes; see dequant below).
template <bool kQ5>
__device__ __forceinline__ void wide_body(const _Float16 *__restrict__ xhi, const h2 *__restrict__ xsum,
                                          const float *__restrict__ rscale, const uint8_t *__restrict__ W,
                                          const float *__restrict__ bias, float *__restrict__ Y, int M, int N, int K,
                                          int tiles_m, int tiles, int ksplit, float *__restrict__ part) {
  constexpr uint32_t kSB = kQ5 ? kQ5KBytes : kQ4KBytes;  // bytes per super-block
  // XCD-aware order: workgroup b runs on XCD b % 8; each XCD takes a
  // contiguous range of (slice, tile) jobs.  Tiles go in groups of up to 8
  // M-tiles: consecutive jobs walk a group's M-tiles (they share an N-tile's
  // weights in that XCD's L2), then its N-tiles, so an XCD's activation
  // tiles also stay few (M=2048 gate: 8 x 14 tiles per XCD rather than
  // 16 x 7, kernel 289.7 -> 281.7 us).
  const int b = (int)blockIdx.x;
  const int jobs = tiles * ksplit;
  const int per_xcd = (jobs + 7) / 8;
  const int job = (b % 8) * per_xcd + b / 8;
  if (job >= jobs) return;
  const int z = job / tiles, tile = job % tiles;
  const int tiles_n = tiles / tiles_m;
  const int grp = tile / (8 * tiles_n), rg = tile % (8 * tiles_n);
  const int gm = tiles_m - 8 * grp < 8 ? tiles_m - 8 * grp : 8;
  const int m0 = (8 * grp + rg % gm) * kWM;
  const int n0 = (rg / gm) * kWN;

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, cl = lane & 31;
  const int nsb_all = K >> 8;
  const int sb0 = (int)((int64_t)z * nsb_all / ksplit);
  const int nsb = (int)((int64_t)(z + 1) * nsb_all / ksplit) - sb0;
  const uint32_t row_bytes = (uint32_t)nsb_all * kSB;
  const uint32_t K32 = (uint32_t)K;

  const Rsrc rs_x = make_rsrc(xhi, (uint32_t)((size_t)M * K * 2));
  const Rsrc rs_s = make_rsrc(xsum, (uint32_t)((size_t)M * (K / 32) * 4));
  const Rsrc rs_w = make_rsrc(W, (uint32_t)((size_t)N * row_bytes));

  // Activation copy of super-block sb into (bufA, bufX): wave w moves rows
  // 16w .. 16w+15, two rows (1 KB, contiguous in LDS and in memory) per
  // instruction; lane L of instruction t writes chunk L & 31 of row
  // 16w + 2t + L/32, which holds the row's logical 16-byte chunk
  // (L & 31) ^ (row & 15), so that the fragment reads of 16 consecutive rows
  // hit distinct banks.  The sums (4 KB): one instruction per wave, lane L
  // of wave w takes half L & 1 (four (hi, lo) pairs) of row 32 (w & 3) + L/2.
  uint32_t a_off[8];
#pragma unroll
  for (int t = 0; t < 8; ++t)
    a_off[t] = (uint32_t)(m0 + 16 * wave + (lane >> 5)) * K32 * 2u +
               16u * ((uint32_t)cl ^ ((uint32_t)(2 * t + (lane >> 5)) & 15u));
  // (Waves 4-7 repeat the sums of waves 0-3 -- the same bytes to the same
  // place -- so that every wave issues the same nine loads per stage and the
  // compiler's vector-load counts stay exact on every path.)
  const uint32_t s_off = ((uint32_t)(m0 + 32 * (wave & 3) + (lane >> 1)) * (K32 / 32u) + 4u * (uint32_t)(lane & 1)) * 4u;
  auto copy_piece = [&](int t, int sb, _Float16 *bufA) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, (LdsPtr)(bufA + (16 * wave + 2 * t) * 256), 16, a_off[t],
                                             (int)((uint32_t)t * 4u * K32 + (uint32_t)sb * 512u), 0, 0);
  };
  auto copy_sums = [&](int sb, _Float16 *bufX) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_s, (LdsPtr)(bufX + 32 * (wave & 3) * 16), 16, s_off,
                                             (int)((uint32_t)sb * 32u), 0, 0);
  };

  // This lane's weight column n0 + 32w + cl: the 16-byte header of each
  // super-block and the 64 qs bytes of lane group g (columns past N read past
  // the tensor: zeros).  q[t] holds qs bytes 64g + 16t ..; q[0..1] are last
  // used at MFMA step 7 and q[2..3] at step 15, so each pair is reloaded for
  // the next super-block right after its last use (half a super-block
  // ahead); the header is double buffered in two register sets that the two
  // halves of the main loop use alternately (no copy between them).
  const uint32_t w_hd = (uint32_t)(n0 + 32 * wave + cl) * row_bytes;
  const uint32_t w_q = w_hd + (kQ5 ? 48u : 16u) + 64u * (uint32_t)g;
  auto ldw = [&](uint32_t voff, int sb) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs_w, voff, (int)((uint32_t)sb * kSB), 0);
  };
  u32x4 q[4], hdA, hdB;
  // Q5_K: the 32 qh bytes of the super-block (hr0, hr1: loaded one
  // super-block ahead) and, for the one being contracted, the 4 bits lane
  // group g uses of each (bits 4g .. 4g + 3: chunks 2g and 2g + 1, both
  // nibble planes), packed as hc[j] = those of bytes 8j .. 8j + 3 in the low
  // nibbles and of bytes 8j + 4 .. 8j + 7 in the high ones
  u32x4 hr0 = {}, hr1 = {};
  uint32_t hc[4] = {0u, 0u, 0u, 0u};
  auto compact_qh = [&]() {
    const uint32_t sh = 4u * (uint32_t)g;
    const uint32_t r[8] = {hr0.x, hr0.y, hr0.z, hr0.w, hr1.x, hr1.y, hr1.z, hr1.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      hc[j] = ((r[2 * j] >> sh) & 0x0F0F0F0Fu) | (((r[2 * j + 1] >> sh) & 0x0F0F0F0Fu) << 4);
  };

  f16x acc[4], accs[4];
  const f16x zero = {};
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = zero;

  // A fragment of row block i at MFMA step s: row 32 i + cl, logical chunk
  // 16 g + s, stored at chunk 16 g + (s ^ (cl & 15)); one address register
  // per step (the lane's part is opaque, so the compiler keeps one XOR per
  // step instead of a register per step), the row blocks at constant offsets
  int a_lane = cl * 512 + 256 * g, a_x = cl & 15;
  asm volatile("" : "+v"(a_lane), "+v"(a_x));
  auto a_addr = [&](int s) { return a_lane + 16 * (s ^ a_x); };
  auto a_at = [&](const _Float16 *bufA, int addr, int i) {
    return *reinterpret_cast<const h8 *>(reinterpret_cast<const char *>(bufA) + addr + 16384 * i);
  };

  // (sc, off) of sub-block 4g + u: low nibble planes (u even) take
  // (sc, -1024 sc) on 0x6400 | q = 1024 + q; high planes (u odd) take the
  // byte masked in place, 0x6400 | 16 q = 1024 + 16 q, with (sc / 16, -64 sc):
  // the fused product 64 sc + sc q is exact and so is the result sc q.
  auto scales = [&](const u32x4 &hd, int u, h2 &sc2, h2 &off2) {
    uint32_t sc, mv;
    q4k_scale_min_sel(4u * (uint32_t)g + (uint32_t)u, hd.y, hd.z, hd.w, sc, mv);
    const float f = (float)sc;
    const _Float16 sh = (_Float16)((u & 1) ? f * 0.0625f : f), oh = (_Float16)((u & 1) ? -64.0f * f : -1024.0f * f);
    sc2 = h2{sh, sh};
    off2 = h2{oh, oh};
  };
  // Q5_K adds the fifth bit (bit b = 2 (s / 8) + (s / 4) % 2 of the lane
  // group's field of byte l): on low planes as bit 4 of the byte (1024 + q5),
  // on high planes, where the byte holds 16 q4, as 256 -- the exponent byte
  // 0x64 | h, i.e. 1024 + 256 h + 16 q4 = 1024 + 16 q5 -- so (sc, -1024 sc)
  // and (sc / 16, -64 sc) give sc * q5 (<= 1953) exactly as for Q4_K.
  auto dequant = [&](int s, h2 sc2, h2 off2) {
    const u32x4 qq = q[(s >> 3) * 2 + ((s & 3) >> 1)];
    const uint32_t d0 = (s & 1) ? qq.z : qq.x, d1 = (s & 1) ? qq.w : qq.y;
    const bool hi = ((s >> 2) & 1) != 0;
    const uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    uint32_t n0v = d0 & mask, n1v = d1 & mask;
    uint32_t e0 = 0x64646464u, e1 = 0x64646464u;
    uint32_t s00 = 0x04010400u, s01 = 0x04030402u;
    if constexpr (kQ5) {
      const uint32_t b = 2u * (uint32_t)(s >> 3) + (uint32_t)((s >> 2) & 1);
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

  // One super-block from (bufA, bufX) with header hd: 16 MFMA steps of 4
  // MFMAs, then the min term into acc and acc += d * accs.  Step s's MFMAs
  // issue while the A fragments and the B fragment of step s + 1 are read and
  // dequantised.  Super-block sb_next is prefetched meanwhile
  // (unconditionally: the last super-block reloads itself, so every path
  // issues the same loads): its activations into (nbufA, nbufX), one copy
  // instruction per step over steps 0-8 -- issued all at once, the eight
  // waves' 72 copy instructions queue at the vector memory unit and hold
  // every wave's MFMAs back at the start of each super-block --, its qs
  // bytes as their registers free up.
  auto contract = [&](const _Float16 *bufA, const _Float16 *bufX, const u32x4 &hd, int sb_next, _Float16 *nbufA,
                      _Float16 *nbufX) {
    h8 a[4], an[4], bv;
    h2 sc2, off2;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = a_at(bufA, a_addr(0), i);
    scales(hd, 0, sc2, off2);
    bv = dequant(0, sc2, off2);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      // per step: the next step's A fragments are read first (they land
      // while this step's MFMAs run), then this step's MFMAs as one cluster
      // at raised priority (the other wave of the SIMD dequantises
      // meanwhile: ping-pong), then the next step's B fragment
      if (s < 15) {
        const int ad = a_addr(s + 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) an[i] = a_at(bufA, ad, i);
      }
      if (s < 8) copy_piece(s, sb_next, nbufA);
      if (s == 8) {  // the sums, then q[0..1] (last used at step 7)
        copy_sums(sb_next, nbufX);
        q[0] = ldw(w_q, sb_next);
        q[1] = ldw(w_q + 16u, sb_next);
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        accs[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bv, s == 0 ? zero : accs[i], 0, 0, 0);
      __builtin_amdgcn_s_setprio(0);
      if (s < 15) {
        if (((s + 1) & 3) == 0) scales(hd, (s + 1) >> 2, sc2, off2);
        bv = dequant(s + 1, sc2, off2);
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = an[i];
      }
    }
    // q[2..3] last used at step 15
    q[2] = ldw(w_q + 32u, sb_next);
    q[3] = ldw(w_q + 48u, sb_next);
    // min term: lane group g holds the (hi, lo) sums of sub-blocks 4g .. 4g+3
    // of its row, B the matching -dmin * m planes (each value twice)
    h8 xa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xa[i] = *reinterpret_cast<const h8 *>(bufX + (32 * i + cl) * 16 + 8 * g);
    const float dmin = f16_bits_hw(hd.x >> 16), dv = f16_bits_hw(hd.x & 0xffffu);
    h8 mh, ml;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t sc, mv;
      q4k_scale_min_sel(4u * (uint32_t)g + (uint32_t)u, hd.y, hd.z, hd.w, sc, mv);
      const float prod = dmin * (float)mv;  // exact (<= 17 significant bits)
      const _Float16 ph = (_Float16)prod;
      const _Float16 pl = (_Float16)(prod - (float)ph);  // exact remainder
      mh[2 * u] = -ph;
      mh[2 * u + 1] = -ph;
      ml[2 * u] = -pl;
      ml[2 * u + 1] = -pl;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[i], mh, acc[i], 0, 0, 0);
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[i], ml, acc[i], 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][e] = __builtin_fmaf(dv, accs[i][e], acc[i][e]);
    }
  };

  // Pipeline: super-block i reads activation buffer i & 1 and header set
  // (hdA, hdB)[i & 1] while the next super-block's header (first) and
  // activations (steps 0-8) go into the other set and buffer, ahead of the
  // qs reloads, so waiting for all but the last four vector loads -- the
  // reloads -- at the end of i waits for the copy and the header; one barrier
  // per super-block.  Every stage issues the same loads (the last one reloads
  // its own super-block into the idle buffer), so no path leaves the compiler
  // an inexact load count and no wait covers the reloads in flight.
  const int last = nsb - 1;
  auto nxt = [&](int i) { return sb0 + (i + 1 < last ? i + 1 : last); };
#pragma unroll
  for (int t = 0; t < 8; ++t) copy_piece(t, sb0, wA0);
  copy_sums(sb0, wX0);
  if (tid < kWM) wR[tid] = m0 + tid < M ? rscale[m0 + tid] : 0.0f;
  hdA = ldw(w_hd, sb0);
#pragma unroll
  for (int t = 0; t < 4; ++t) q[t] = ldw(w_q + 16u * t, sb0);
  if constexpr (kQ5) {
    hr0 = ldw(w_hd + 16u, sb0);
    hr1 = ldw(w_hd + 32u, sb0);
  }
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  __syncthreads();
  constexpr int kWaitCopy = 0x0074;  // vmcnt(4) expcnt(7) lgkmcnt(0), gfx9 encoding
  // Q5_K: the current super-block's qh bits are packed before its contraction,
  // then the raw registers take the next super-block's (ahead of the qs
  // reloads, so the wait before each barrier covers them)
  auto next_qh = [&](int sb) {
    if constexpr (kQ5) {
      compact_qh();
      hr0 = ldw(w_hd + 16u, sb);
      hr1 = ldw(w_hd + 32u, sb);
    }
  };
  for (int i = 0;; i += 2) {
    hdB = ldw(w_hd, nxt(i));
    next_qh(nxt(i));
    contract(wA0, wX0, hdA, nxt(i), wA1, wX1);
    __builtin_amdgcn_s_waitcnt(kWaitCopy);
    __builtin_amdgcn_s_barrier();
    if (i + 1 >= nsb) break;
    hdA = ldw(w_hd, nxt(i + 1));
    next_qh(nxt(i + 1));
    contract(wA1, wX1, hdB, nxt(i + 1), wA0, wX0);
    __builtin_amdgcn_s_waitcnt(kWaitCopy);
    __builtin_amdgcn_s_barrier();
    if (i + 2 >= nsb) break;
  }
  // The last stage's copy into the idle buffer and its reloads must land
  // before the workgroup's LDS is released.  The empty asm reads the
  // prefetched registers on the way out, so that the loads a stage issues
  // for the next one are live on both sides of the exit test between the
  // two halves of the loop: the compiler cannot sink them past the test to
  // just before their first use, where each would wait out its latency.
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::"v"(hdA), "v"(hdB), "v"(q[0]), "v"(q[1]), "v"(q[2]), "v"(q[3]));
  if constexpr (kQ5) asm volatile("" ::"v"(hr0), "v"(hr1));

  // epilogue: lane (cl, g) holds rows 8 (e / 4) + 4 g + e % 4 of column cl
  // of each 32 x 32 block; split K stores the raw partial sums, otherwise the
  // row scale (from LDS) and the bias are applied
  // A whole tile stores without per-value row tests: branches there would
  // leave loads pending at every join and cost a wait per store.
  const int col = n0 + 32 * wave + cl;
  const int rows = M - m0 < kWM ? M - m0 : kWM;
  // rows whose scale is NaN (computed by the pre-pass), tested by every lane
  // of the wave before any lane leaves for a column past N
  const bool flagged =
      __builtin_amdgcn_ballot_w64(__builtin_isnan(wR[lane]) || __builtin_isnan(wR[64 + lane])) != 0;
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
      if (rows == kWM) {
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
            const float4 rs = *reinterpret_cast<const float4 *>(wR + r0);
            const float rv[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if ((!guard || r0 + q < rows) && (!skip || !__builtin_isnan(rv[q])))
                dst[(size_t)(r0 + q) * N] = acc[i][4 * j + q] * rv[q] + bv;
          }
      };
      if (flagged) {
        store(true, true);
      } else if (rows == kWM) {
        store(false, false);
      } else {
        store(true, false);
      }
    }
  }
}

__global__ __launch_bounds__(512) void gemm_wide_q4k_kernel(const _Float16 *__restrict__ xhi,
                                                            const h2 *__restrict__ xsum,
                                                            const float *__restrict__ rscale,
                                                            const uint8_t *__restrict__ W,
                                                            const float *__restrict__ bias, float *__restrict__ Y,
                                                            int M, int N, int K, int tiles_m, int tiles, int ksplit,
                                                            float *__restrict__ part) {
  wide_body<false>(xhi, xsum, rscale, W, bias, Y, M, N, K, tiles_m, tiles, ksplit, part);
}

__global__ __launch_bounds__(512) void gemm_wide_q5k_kernel(const _Float16 *__restrict__ xhi,
                                                            const h2 *__restrict__ xsum,
                                                            const float *__restrict__ rscale,
                                                            const uint8_t *__restrict__ W,
                                                            const float *__restrict__ bias, float *__restrict__ Y,
                                                            int M, int N, int K, int tiles_m, int tiles, int ksplit,
                                                            float *__restrict__ part) {
  wide_body<true>(xhi, xsum, rscale, W, bias, Y, M, N, K, tiles_m, tiles, ksplit, part);
}

bool gemm_wide_supported(int type, int64_t M, int64_t K, int64_t N) {
  const int64_t a_bytes = (M + kWM) * K * 2;
  const int64_t w_bytes = (N + kWN) * (K / 256) * (type == kQ5_K ? kQ5KBytes : kQ4KBytes) + 1024;
  return (type == kQ4_K || type == kQ5_K) && K % 256 == 0 && M >= 1 && N >= 1 && a_bytes < (int64_t)UINT32_MAX &&
         w_bytes < (int64_t)UINT32_MAX;
}

int gemm_wide_tiles(int64_t M, int64_t N) { return (int)(((M + kWM - 1) / kWM) * ((N + kWN - 1) / kWN)); }

hipError_t launch_gemm_wide(int type, const _Float16 *xhi, const void *xsum, const float *rscale, const void *w,
                            const float *bias, float *y, int64_t M, int64_t N, int64_t K, int ksplit, float *part,
                            hipStream_t s) {
  const int tiles_m = (int)((M + kWM - 1) / kWM);
  const int tiles = gemm_wide_tiles(M, N);
  const int per_xcd = (tiles * ksplit + 7) / 8;
  launch_timed(type == kQ5_K ? gemm_wide_q5k_kernel : gemm_wide_q4k_kernel, dim3((unsigned)(per_xcd * 8)), dim3(512),
               0u, s, xhi, static_cast<const h2 *>(xsum), rscale, static_cast<const uint8_t *>(w), bias, y, (int)M,
               (int)N, (int)K, tiles_m, tiles, ksplit, part);
  return hipGetLastError();
}

}  // namespace okq
