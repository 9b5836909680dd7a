// okq_gemm_q6.hip -- Q6_K prefill dequant-GEMM with the weights dequantised
// in registers: Y[M,N] = X[M,K] W[N,K]^T (+bias), bf16 activations through
// the pre-pass's row-scaled fp16 plane (as the Q4_K kernels).
//
// Numerics.  A Q6_K weight is d * sc * (q - 32) with sc an int8 per 16
// weights and q six bits; sc * (q - 32) (|.| <= 4096) is not exact in fp16,
// so it enters as two exact planes that the MFMAs add into the same
// accumulator: with sc = 16 sh + sl (sh = sc >> 4 in [-8, 7], sl = sc & 15),
//   B_hi = 16 sh (q - 32)   (a multiple of 16 with at most 10 significant bits)
//   B_lo = sl (q - 32)      (|.| <= 480)
// Both come from one fp16 encoding of q, 0x6400 | 16 q = 1024 + 16 q, by one
// packed fp16 FMA each whose exact result is representable:
//   (1024 + 16 q) * sh      - 1536 sh = 16 sh (q - 32)
//   (1024 + 16 q) * sl / 16 -   96 sl =    sl (q - 32)
// Every product inside the MFMAs is exact; d is applied per super-block in f32
// (acc += d * accs).  No min term.
//
// Layout, as okq_gemm_wide.hip: one 8-wave workgroup per CU on a 128 x 256
// tile, wave w owning columns 32w .. 32w+31 for all 128 rows (four 32x32x16
// MFMA blocks per B fragment, two B fragments -- the planes -- per step);
// one super-block (256 K) of the 128 rows' activations per stage,
// double-buffered in LDS by buffer-to-LDS copies with the 16-byte chunk c of
// row r at chunk c ^ (r & 15).
//
//   * K order: MFMA step s (0..15), lane group g = lane / 32 covers
//     k = 128 g + 8 s + [0, 8): half g of the super-block, quarter t = s / 4
//     (elements l + 32 t), l = 8 (s & 3) + [0, 8) -- low nibbles of ql[l]
//     (t = 0), of ql[l + 32] (t = 1), high nibbles of the same (t = 2, 3),
//     bits 2t, 2t+1 of qh[l], scale sc[l / 16 + 2 t] of the half.
//   * Weights: a lane loads its half's 64 ql bytes, 32 qh bytes, 8 scales
//     (dword windows: super-blocks are 210 bytes, so a window starts 0 or 2
//     bytes before its data, realigned with v_alignbyte) and d (a 2-byte
//     load: a dword window could end past a tensor whose size is only
//     2-byte aligned), one super-block ahead.
//   * Dequant: per 8 weights, the nibbles placed at bits 4..7 of a byte and
//     the two high bits in the exponent byte 0x64 | h (v_perm_b32 pairs
//     them into 1024 + 16 q), then one packed FMA per pair and plane.
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef __attribute__((address_space(3))) void *LdsPtr;

constexpr int kWM = 128;  // tile rows
constexpr int kWN = 256;  // tile columns (8 waves x 32)

__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Activation stages: two buffers of [128 rows][256 halves] (swizzled 16-byte
// chunks); distinct objects, so that the fragment reads of one do not wait
// for the copy into the other.
__shared__ __attribute__((aligned(16))) _Float16 q6A0[kWM * 256];
__shared__ __attribute__((aligned(16))) _Float16 q6A1[kWM * 256];
// the tile's row scales for the epilogue
__shared__ __attribute__((aligned(16))) float q6R[kWM];

// A lane's share of a super-block as loaded (dword windows starting r = 0
// or 2 bytes before the data) and as the steps use it.
struct Q6Raw {
  u32x4 l0, l1, l2, l3;  // ql window: 17 dwords
  uint32_t l4;
  u32x4 h0, h1;  // qh window: 9 dwords
  uint32_t h2;
  u32x3 s;        // scales window: 3 dwords
  uint32_t d;     // f16 d (2-byte load)
  uint32_t r;     // bytes between the window starts and the data
};
struct Q6Cur {
  uint32_t L[16];  // the half's 64 ql bytes
  uint32_t H[8];   // its 32 qh bytes
  uint32_t S[2];   // its 8 scales
  float d;
};

}  // namespace

__global__ __launch_bounds__(512) void gemm_wide_q6k_kernel(const _Float16 *__restrict__ xhi,
                                                            const float *__restrict__ rscale,
                                                            const uint8_t *__restrict__ W,
                                                            const float *__restrict__ bias, float *__restrict__ Y,
                                                            int M, int N, int K, int tiles_m, int tiles, int ksplit,
                                                            float *__restrict__ part) {
  // XCD-aware order (workgroup b runs on XCD b % 8, each XCD takes a
  // contiguous range of jobs), tiles in groups of up to 8 M-tiles as in
  // okq_gemm_wide.hip.
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
  const uint32_t row_bytes = (uint32_t)nsb_all * kQ6KBytes;
  const uint32_t K32 = (uint32_t)K;

  const Rsrc rs_x = make_rsrc(xhi, (uint32_t)((size_t)M * K * 2));
  const Rsrc rs_w = make_rsrc(W, (uint32_t)((size_t)N * row_bytes));

  // Activation copy of super-block sb into bufA: wave w moves rows
  // 16w .. 16w+15, two rows (1 KB) per instruction; lane L of instruction t
  // writes chunk L & 31 of row 16w + 2t + L/32, which holds the row's logical
  // 16-byte chunk (L & 31) ^ (row & 15).
  // (the lane's offset is recomputed per copy: two VALU instructions
  // instead of eight registers held through the loop)
  const uint32_t a_row = (uint32_t)(m0 + 16 * wave + (lane >> 5)) * K32 * 2u;
  auto copy_piece = [&](int t, int sb, _Float16 *bufA) {
    const uint32_t off = a_row + 16u * ((uint32_t)cl ^ ((uint32_t)(2 * t + (lane >> 5)) & 15u));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, (LdsPtr)(bufA + (16 * wave + 2 * t) * 256), 16, off,
                                             (int)((uint32_t)t * 4u * K32 + (uint32_t)sb * 512u), 0, 0);
  };

  // This lane's weight column n0 + 32w + cl (columns past N read past the
  // tensor: zeros), half g of each super-block.
  const uint32_t w_col = (uint32_t)(n0 + 32 * wave + cl) * row_bytes;
  auto ldw = [&](int sb, Q6Raw &R) {
    const uint32_t base = w_col + (uint32_t)sb * kQ6KBytes;
    const uint32_t r = base & 3u;
    const uint32_t a = base - r;
    const uint32_t gq = 64u * (uint32_t)g, gh = 128u + 32u * (uint32_t)g, gs = 192u + 8u * (uint32_t)g;
    R.r = r;
    R.l0 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, a + gq, 0, 0);
    R.l1 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, a + gq + 16u, 0, 0);
    R.l2 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, a + gq + 32u, 0, 0);
    R.l3 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, a + gq + 48u, 0, 0);
    R.l4 = __builtin_amdgcn_raw_buffer_load_b32(rs_w, a + gq + 64u, 0, 0);
    R.h0 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, a + gh, 0, 0);
    R.h1 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, a + gh + 16u, 0, 0);
    R.h2 = __builtin_amdgcn_raw_buffer_load_b32(rs_w, a + gh + 32u, 0, 0);
    R.s = __builtin_amdgcn_raw_buffer_load_b96(rs_w, a + gs, 0, 0);
    R.d = __builtin_amdgcn_raw_buffer_load_b16(rs_w, base + 208u, 0, 0);
  };
  auto realign_all = [&](const Q6Raw &R, Q6Cur &C) {
    const uint32_t l[17] = {R.l0.x, R.l0.y, R.l0.z, R.l0.w, R.l1.x, R.l1.y, R.l1.z, R.l1.w, R.l2.x,
                            R.l2.y, R.l2.z, R.l2.w, R.l3.x, R.l3.y, R.l3.z, R.l3.w, R.l4};
    const uint32_t h[9] = {R.h0.x, R.h0.y, R.h0.z, R.h0.w, R.h1.x, R.h1.y, R.h1.z, R.h1.w, R.h2};
#pragma unroll
    for (int i = 0; i < 16; ++i) C.L[i] = realign(l[i + 1], l[i], R.r);
#pragma unroll
    for (int i = 0; i < 8; ++i) C.H[i] = realign(h[i + 1], h[i], R.r);
    C.S[0] = realign(R.s.y, R.s.x, R.r);
    C.S[1] = realign(R.s.z, R.s.y, R.r);
    C.d = f16_bits_hw(R.d & 0xffffu);
  };

  f16x acc[4], accs[4];
  const f16x zero = {};
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = zero;

  // A fragment of row block i at MFMA step s: row 32 i + cl, logical chunk
  // 16 g + s, stored at chunk 16 g + (s ^ (cl & 15)); one address register per
  // step, the row blocks at constant offsets
  int a_lane = cl * 512 + 256 * g, a_x = cl & 15;
  asm volatile("" : "+v"(a_lane), "+v"(a_x));
  auto a_addr = [&](int s) { return a_lane + 16 * (s ^ a_x); };
  auto a_at = [&](const _Float16 *bufA, int addr, int i) {
    return *reinterpret_cast<const h8 *>(reinterpret_cast<const char *>(bufA) + addr + 16384 * i);
  };

  // The two planes' (scale, offset) pairs of scale byte j of the half
  auto scales = [&](const Q6Cur &C, int j, h2 &mh, h2 &oh, h2 &ml, h2 &ol) {
    const int sc = __builtin_amdgcn_sbfe((int)C.S[j >> 2], 8 * (j & 3), 8);
    const int sh = sc >> 4, sl = sc & 15;
    const _Float16 fh = (_Float16)(float)sh, fo = (_Float16)(-1536.0f * (float)sh);
    const _Float16 gl = (_Float16)(0.0625f * (float)sl), go = (_Float16)(-96.0f * (float)sl);
    mh = h2{fh, fh};
    oh = h2{fo, fo};
    ml = h2{gl, gl};
    ol = h2{go, go};
  };
  // B fragments (both planes) of step s
  auto dequant = [&](const Q6Cur &C, int s, h2 mh, h2 oh, h2 ml, h2 ol, h8 &bh, h8 &bl) {
    const int t = s >> 2, j4 = s & 3;
    const uint32_t q0 = C.L[8 * (t & 1) + 2 * j4], q1 = C.L[8 * (t & 1) + 2 * j4 + 1];
    const uint32_t n0 = (t >> 1) ? (q0 & 0xF0F0F0F0u) : ((q0 << 4) & 0xF0F0F0F0u);
    const uint32_t n1 = (t >> 1) ? (q1 & 0xF0F0F0F0u) : ((q1 << 4) & 0xF0F0F0F0u);
    const uint32_t e0 = 0x64646464u | ((C.H[2 * j4] >> (2 * t)) & 0x03030303u);
    const uint32_t e1 = 0x64646464u | ((C.H[2 * j4 + 1] >> (2 * t)) & 0x03030303u);
    // (1024 + 16 q) pairs in element order: low byte 16 q (mod 256), high byte 0x64 | q >> 4
    const h2 p0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(e0, n0, 0x05010400u));
    const h2 p1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(e0, n0, 0x07030602u));
    const h2 p2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(e1, n1, 0x05010400u));
    const h2 p3 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(e1, n1, 0x07030602u));
    const h2 h0 = __builtin_elementwise_fma(p0, mh, oh), h1 = __builtin_elementwise_fma(p1, mh, oh);
    const h2 h2v = __builtin_elementwise_fma(p2, mh, oh), h3 = __builtin_elementwise_fma(p3, mh, oh);
    const h2 l0 = __builtin_elementwise_fma(p0, ml, ol), l1 = __builtin_elementwise_fma(p1, ml, ol);
    const h2 l2 = __builtin_elementwise_fma(p2, ml, ol), l3 = __builtin_elementwise_fma(p3, ml, ol);
    bh = h8{h0[0], h0[1], h1[0], h1[1], h2v[0], h2v[1], h3[0], h3[1]};
    bl = h8{l0[0], l0[1], l1[0], l1[1], l2[0], l2[1], l3[0], l3[1]};
  };

  // One super-block from bufA with weights C: 16 MFMA steps of 8 MFMAs (the
  // high plane of the four row blocks, then the low plane), then
  // acc += d * accs.  Step s's MFMAs issue while the A fragments and the B
  // fragments of step s + 1 are read and dequantised; the next super-block's
  // activations are copied into nbufA over steps 0-7.
  auto contract = [&](const _Float16 *bufA, const Q6Cur &C, int sb_next, _Float16 *nbufA) {
    h8 a[4], an[4], bh, bl;
    h2 mh, oh, ml, ol;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = a_at(bufA, a_addr(0), i);
    scales(C, 0, mh, oh, ml, ol);
    dequant(C, 0, mh, oh, ml, ol, bh, bl);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      if (s < 15) {
        const int ad = a_addr(s + 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) an[i] = a_at(bufA, ad, i);
      }
      if (s < 8) copy_piece(s, sb_next, nbufA);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        accs[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bh, s == 0 ? zero : accs[i], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) accs[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bl, accs[i], 0, 0, 0);
      __builtin_amdgcn_s_setprio(0);
      if (s < 15) {
        const int t = (s + 1) >> 2, j4 = (s + 1) & 3;
        if ((j4 & 1) == 0) scales(C, (j4 >> 1) + 2 * t, mh, oh, ml, ol);  // the scale changes every two steps
        dequant(C, s + 1, mh, oh, ml, ol, bh, bl);
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = an[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][e] = __builtin_fmaf(C.d, accs[i][e], acc[i][e]);
  };

  // Pipeline: super-block i reads activation buffer i & 1; at its start its
  // weights are realigned out of the raw registers, which then take the next
  // super-block's loads (past the last one they reload it into dead
  // registers, so every stage issues the same loads); its copy into the
  // other buffer is the last load a stage issues, so the one wait before the
  // stage's barrier waits for it and for the prefetch.
  const int last = nsb - 1;
  auto nxt = [&](int i) { return sb0 + (i + 1 < last ? i + 1 : last); };
  Q6Raw raw;
  Q6Cur cur;
#pragma unroll
  for (int t = 0; t < 8; ++t) copy_piece(t, sb0, q6A0);
  if (tid < kWM) q6R[tid] = m0 + tid < M ? rscale[m0 + tid] : 0.0f;
  ldw(sb0, raw);
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  __syncthreads();
  constexpr int kWaitAll = 0x0070;  // vmcnt(0) expcnt(7) lgkmcnt(0), gfx9 encoding
  for (int i = 0;; i += 2) {
    realign_all(raw, cur);
    ldw(nxt(i), raw);
    __builtin_amdgcn_sched_barrier(0);  // the prefetch issues first
    contract(q6A0, cur, nxt(i), q6A1);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    __builtin_amdgcn_s_barrier();
    if (i + 1 >= nsb) break;
    realign_all(raw, cur);
    ldw(nxt(i + 1), raw);
    __builtin_amdgcn_sched_barrier(0);
    contract(q6A1, cur, nxt(i + 1), q6A0);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    __builtin_amdgcn_s_barrier();
    if (i + 2 >= nsb) break;
  }

  // epilogue: lane (cl, g) holds rows 8 (e / 4) + 4 g + e % 4 of column cl
  // of each 32 x 32 block; split K stores the raw partial sums, otherwise the
  // row scale (from LDS) and the bias are applied.  A whole tile stores
  // without per-value row tests.
  const int col = n0 + 32 * wave + cl;
  const int rows = M - m0 < kWM ? M - m0 : kWM;
  // rows whose scale is NaN (computed by the pre-pass), tested by every lane
  // of the wave before any lane leaves for a column past N
  const bool flagged =
      __builtin_amdgcn_ballot_w64(__builtin_isnan(q6R[lane]) || __builtin_isnan(q6R[64 + lane])) != 0;
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
      // wrote their IEEE outputs
      auto store = [&](bool guard, bool skip) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r0 = 32 * i + 8 * j + 4 * g;
            const float4 rs = *reinterpret_cast<const float4 *>(q6R + r0);
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

int gemm_q6_tiles(int64_t M, int64_t N) { return (int)(((M + kWM - 1) / kWM) * ((N + kWN - 1) / kWN)); }

hipError_t launch_gemm_q6(const _Float16 *xhi, const float *rscale, const void *w, const float *bias, float *y,
                          int64_t M, int64_t N, int64_t K, int ksplit, float *part, hipStream_t s) {
  if (K % 256 != 0 || ksplit < 1 || ksplit > K / 256) return hipErrorInvalidValue;
  const int tiles_m = (int)((M + kWM - 1) / kWM);
  const int tiles = gemm_q6_tiles(M, N);
  const int per_xcd = (tiles * ksplit + 7) / 8;
  launch_timed(gemm_wide_q6k_kernel, dim3((unsigned)(per_xcd * 8)), dim3(512), 0u, s, xhi, rscale,
               static_cast<const uint8_t *>(w), bias, y, (int)M, (int)N, (int)K, tiles_m, tiles, ksplit, part);
  return hipGetLastError();
}

}  // namespace okq
