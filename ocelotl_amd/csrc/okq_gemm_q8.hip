// okq_gemm_q8.hip -- Q8_0 prefill dequant-GEMM on bf16 activations, the
// weights dequantised in registers: Y[M,N] = X[M,K] W[N,K]^T (+bias).
//
// Numerics.  A = the bf16 activations themselves, B = q itself (an int8, exact
// in bf16): every product x * q is exact in f32 (8 x 8 significant bits) and
// the MFMAs sum a block's 32 of them in f32; then acc += d * (block sum) in
// f32 with d the block's f16 scale widened exactly.  bf16 keeps f32's
// exponent range, so no activation pre-pass (row scale, fp16 planes) runs
// and infinities and NaNs take their IEEE course through the MFMAs and the
// fold: a block sum holding x = +-inf is +-inf (NaN with both signs or a NaN
// x; inf * 0 = NaN where q = 0, as the reference's x * (d * 0)), times d.
// d changes every 32 weights, so the fold costs one FMA per output value and
// block -- one VALU lane-op per 64 MFMA flops (the Q4_K kernels fold once per
// 256 weights).  The other way, B = d * q, is exact in neither bf16 nor fp16
// (up to 19 significant bits) and would need two planes, two MFMAs per
// product.
//
// Layout: wave w owns columns 32w .. 32w+31 of the tile for all 128 rows
// (four 32x32x16 MFMA blocks per B fragment).  gemm_q8_kernel: four waves on
// a 128 x 128 tile, two workgroups per CU (okq_gemm_pair.hip's layout), so
// the two waves of a SIMD belong to different tiles and one's MFMAs run while
// the other folds and dequantises; gemm_q8_wide_kernel: eight waves on a
// 128 x 256 tile, one workgroup per CU (each activation stage serves twice
// the columns), for grids whose wide tiles fill the CUs.  A stage is 128 K =
// four Q8_0 blocks (136 bytes per column); activations are double-buffered
// in LDS (2 x 32 KB), copied one stage ahead by buffer-to-LDS loads with
// 16-byte chunk c of row r at chunk c ^ (r & 15) (conflict-free fragment
// reads).
//
//   * K order: MFMA step s (0..7) of a stage covers block j = s / 2, lane
//     group g = lane / 32 its elements 16 g + 8 (s & 1) + [0, 8), so every
//     MFMA stays inside one block and the block's sums are whole after its
//     second step.
//   * Weights: lane group g loads bytes 68 g .. 68 g + 67 of the column's
//     stage -- blocks 2 g and 2 g + 1 whole, four 16-byte loads and one
//     dword, a stage ahead -- and the two lane groups then trade halves with
//     v_permlane32_swap (lanes l and l + 32 hold the same column): group 0
//     keeps the first 16 q bytes of its blocks and receives those of group
//     1's, group 1 the second 16.  The first block of each pair starts 2
//     bytes into a dword (34-byte blocks), realigned with v_alignbyte; the
//     four d travel the same way, packed two to a dword.  (Loading each
//     half-block where it is used takes ten scattered loads per stage instead
//     of five, and those loads, not the MFMAs, set the kernel's pace.)
//   * Dequant: each signed byte to f32 (v_cvt_f32_i32 with a sign-extending
//     byte select), the high halves of two such f32 packed into a bf16 pair
//     (v_perm_b32): 12 VALU instructions per 8 weights.
//   * Fold: block j's sums fold into acc at the first step of block j + 1,
//     tile by tile, each accs[i] just before its next MFMA restarts it, so a
//     wave's FMAs also overlap its own MFMAs; the stage's last block folds
//     after its second step (sums carried across the stage boundary cost the
//     register allocator a second accumulator set).
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

namespace {

typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef __attribute__((address_space(3))) void *LdsPtr;

constexpr int kQM = 128;                          // tile rows (the tile has 32 columns per wave)
constexpr uint32_t kStageBytes = 4u * kQ8Bytes;   // one stage of a column: 4 blocks, 128 K

__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Activation stages: two buffers of [128 rows][128 bf16] (swizzled 16-byte
// chunks); distinct objects, so that the fragment reads of one do not wait
// for the loads into the other.
__shared__ __attribute__((aligned(16))) uint16_t qA0[kQM * 128];
__shared__ __attribute__((aligned(16))) uint16_t qA1[kQM * 128];

// Signed bytes 2 h and 2 h + 1 of w as a bf16 pair (low half first): exact,
// an int8 has at most 8 significant bits.
__device__ __forceinline__ uint32_t bf16_pair(uint32_t w, int h) {
  const float f0 = (float)(int8_t)(w >> (16 * h)), f1 = (float)(int8_t)(w >> (16 * h + 8));
  return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}

// A lane's 68 bytes of a stage as loaded (blocks 2 g and 2 g + 1: d, 32 q,
// d, 32 q) and the stage as the MFMA steps use it: the lane group's 16 q
// bytes of each block and the four d (two per dword, block order).
struct Q8Raw {
  u32x4 v0, v1, v2, v3;
  uint32_t v4;
};
struct Q8Ready {
  uint32_t q[4][4];
  uint32_t d01, d23;
};

}  // namespace

// kW waves per workgroup on a 128 x 32 kW tile: 4 (two workgroups per CU)
// or 8 (one per CU: half the activation copies per MFMA, for grids that fill
// the CUs with the wider tiles).
template <int kW>
__device__ __forceinline__ void q8_body(const uint16_t *__restrict__ X, const uint8_t *__restrict__ W,
                                        const float *__restrict__ bias, float *__restrict__ Y, int M, int N, int K,
                                        int tiles_m, int tiles, int ksplit, float *__restrict__ part) {
  constexpr int kQN = 32 * kW;    // tile columns
  constexpr int kRW = kQM / kW;   // rows each wave copies
  constexpr int kCP = kRW / 4;    // its copy instructions per stage (4 rows each)
  // XCD-aware order: workgroup b runs on XCD b % 8; each XCD takes a
  // contiguous range of (slice, tile) jobs.
  const int b = (int)blockIdx.x;
  const int jobs = tiles * ksplit;
  const int per_xcd = (jobs + 7) / 8;
  const int job = (b % 8) * per_xcd + b / 8;
  if (job >= jobs) return;
  const int z = job / tiles, tile = job % tiles;
  // groups of up to 8 M-tiles: consecutive jobs walk a group's M-tiles, then
  // its N-tiles, so an XCD's jobs share both activation and weight tiles in
  // its L2 (M=2048: 8 x 8 tiles per XCD rather than 16 x 4, 2-3% faster)
  const int tiles_n = tiles / tiles_m;
  const int grp = tile / (8 * tiles_n), rg = tile % (8 * tiles_n);
  const int gm = tiles_m - 8 * grp < 8 ? tiles_m - 8 * grp : 8;
  const int m0 = (8 * grp + rg % gm) * kQM;
  const int n0 = (rg / gm) * kQN;

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, cl = lane & 31;
  const int nst_all = K >> 7;  // stages of 128 K
  const int st0 = (int)((int64_t)z * nst_all / ksplit);
  const int nst = (int)((int64_t)(z + 1) * nst_all / ksplit) - st0;
  const uint32_t row_bytes = (uint32_t)(K >> 5) * (uint32_t)kQ8Bytes;
  const uint32_t K2 = (uint32_t)K * 2u;

  const Rsrc rs_x = make_rsrc(X, (uint32_t)((size_t)M * K * 2));
  const Rsrc rs_w = make_rsrc(W, (uint32_t)((size_t)N * row_bytes));

  // Activation copy of stage st (slice-relative): wave w moves rows
  // kRW w .. kRW w + kRW - 1, four rows (1 KB) per instruction; lane L of
  // instruction t writes chunk L & 15 of row kRW w + 4t + L/16, which holds
  // the row's logical chunk (L & 15) ^ (row & 15).
  uint32_t a_off[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    a_off[t] = (uint32_t)(m0 + kRW * wave + (lane >> 4)) * K2 +
               16u * ((uint32_t)(lane & 15) ^ (uint32_t)(4 * t + (lane >> 4)));
  auto copy_piece = [&](int t, int st, uint16_t *bufA) {
    const uint32_t kb = (uint32_t)(st0 + st) * 128u;  // first K of the stage
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, (LdsPtr)(bufA + (kRW * wave + 4 * t) * 128), 16, a_off[t & 3],
                                             (int)((uint32_t)t * 4u * K2 + kb * 2u), 0, 0);
  };

  // This lane's weight column n0 + 32w + cl (columns past N read past the
  // tensor: zeros), bytes 68 g .. of each stage.
  const uint32_t w_lane = (uint32_t)(n0 + 32 * wave + cl) * row_bytes + 68u * (uint32_t)g;
  auto ld_raw = [&](int st, Q8Raw &r) {
    const int so = (int)((uint32_t)(st0 + st) * kStageBytes);
    r.v0 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, w_lane, so, 0);
    r.v1 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, w_lane + 16u, so, 0);
    r.v2 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, w_lane + 32u, so, 0);
    r.v3 = __builtin_amdgcn_raw_buffer_load_b128(rs_w, w_lane + 48u, so, 0);
    r.v4 = __builtin_amdgcn_raw_buffer_load_b32(rs_w, w_lane + 64u, so, 0);
  };
  // v_permlane32_swap(x, y) trades x's lanes 32-63 for y's lanes 0-31: with
  // x = a group's first-half dword and y its second-half dword, x becomes
  // "this group's half of the lower pair's block" in both groups and y "this
  // group's half of the upper pair's block".
  auto prepare = [&](const Q8Raw &r, Q8Ready &R) {
    const uint32_t w[17] = {r.v0.x, r.v0.y, r.v0.z, r.v0.w, r.v1.x, r.v1.y, r.v1.z, r.v1.w, r.v2.x,
                            r.v2.y, r.v2.z, r.v2.w, r.v3.x, r.v3.y, r.v3.z, r.v3.w, r.v4};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const auto a = __builtin_amdgcn_permlane32_swap(realign(w[k + 1], w[k], 2u), realign(w[k + 5], w[k + 4], 2u),
                                                      false, false);
      R.q[0][k] = a[0];
      R.q[2][k] = a[1];
      const auto b = __builtin_amdgcn_permlane32_swap(w[9 + k], w[13 + k], false, false);
      R.q[1][k] = b[0];
      R.q[3][k] = b[1];
    }
    const uint32_t dd = __builtin_amdgcn_perm(w[8], w[0], 0x07060100u);  // d of the lower block | d of the upper << 16
    const auto d = __builtin_amdgcn_permlane32_swap(dd, dd, false, false);
    R.d01 = d[0];
    R.d23 = d[1];
  };
  Q8Raw raw;
  Q8Ready S;

  f16x acc[4], accs[4];
  const f16x zero = {};
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = zero;

  // A fragment of row block i at MFMA step s: row 32 i + cl, logical chunk
  // c = 4 (s / 2) + 2 g + (s & 1), stored at chunk c ^ (cl & 15); c's bit 1 is
  // g alone, so the lane's part (2 g) ^ (cl & 15) is one register and each
  // step adds one XOR with its constant 4 (s / 2) + (s & 1)
  // (contract re-reads the lane's part through an empty asm, so that the
  // compiler computes each stage's eight addresses inside the loop instead of
  // hoisting them all out of it into registers)
  const int a_lane = cl * 256, a_x0 = (2 * g) ^ (cl & 15);
  int a_x = a_x0;
  auto a_addr = [&](int s) { return a_lane + 16 * ((4 * (s >> 1) + (s & 1)) ^ a_x); };
  auto a_at = [&](const uint16_t *bufA, int addr, int i) {
    return *reinterpret_cast<const b8 *>(reinterpret_cast<const char *>(bufA) + addr + 8192 * i);
  };

  // B fragment of step s: the 8 q bytes 8 (s & 1) .. of the lane group's
  // window of block s / 2, as bf16
  auto dequant = [&](int s) {
    const int j = s >> 1, t = s & 1;
    const uint32_t w0 = S.q[j][2 * t], w1 = S.q[j][2 * t + 1];
    return __builtin_bit_cast(b8, u32x4{bf16_pair(w0, 0), bf16_pair(w0, 1), bf16_pair(w1, 0), bf16_pair(w1, 1)});
  };

  // One stage from bufA with weights S: 8 MFMA steps of 4 MFMAs, then the
  // next stage's weights (loaded meanwhile) prepared into S.  At the
  // first step of blocks 1-3 the previous block's sums fold into acc, tile
  // by tile, ahead of the MFMA that restarts that tile's accs; block 3 folds
  // after step 7.  Step s's
  // MFMAs issue while the A fragments and the B fragment of step s + 1 are
  // read and dequantised; steps 0-3 copy stage st_next's activations into
  // nbufA, two copy instructions per step.
  auto contract = [&](const uint16_t *bufA, int st_next, uint16_t *nbufA) {
    a_x = a_x0;
    asm volatile("" : "+v"(a_x));
    const float dj[4] = {f16_bits_hw(S.d01 & 0xffffu), f16_bits_hw(S.d01 >> 16), f16_bits_hw(S.d23 & 0xffffu),
                         f16_bits_hw(S.d23 >> 16)};
    b8 a[4], an[4], bv;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = a_at(bufA, a_addr(0), i);
    bv = dequant(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s < 7) {
        const int ad = a_addr(s + 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) an[i] = a_at(bufA, ad, i);
      }
      if (s < 4) {
#pragma unroll
        for (int c = 0; c < kCP / 4; ++c) copy_piece(kCP / 4 * s + c, st_next, nbufA);
      }
      // the next step's fragment reads issue ahead of this step's MFMAs
      __builtin_amdgcn_sched_barrier(0);
      if ((s & 1) == 0) {
        const float dp = dj[s > 0 ? (s >> 1) - 1 : 0];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (s > 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][e] = __builtin_fmaf(dp, accs[i][e], acc[i][e]);
          }
          accs[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bv, zero, 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) accs[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bv, accs[i], 0, 0, 0);
        if (s == 7) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][e] = __builtin_fmaf(dj[3], accs[i][e], acc[i][e]);
        }
      }
      if (s < 7) {
        bv = dequant(s + 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = an[i];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    prepare(raw, S);
  };

  // Pipeline: stage st reads buffer st & 1 while stage st + 1's activations
  // go into the other buffer and its weights into the raw registers (first,
  // ahead of the copy).  Every stage issues the same loads (past the last
  // stage they reload it: idle buffer, registers dead at the end), so the
  // compiler's load counts stay exact on every path.
  const int last = nst - 1;
  auto cl_st = [&](int st) { return st < last ? st : last; };
#pragma unroll
  for (int t = 0; t < kCP; ++t) copy_piece(t, 0, qA0);
  ld_raw(0, raw);
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  prepare(raw, S);
  __syncthreads();
  constexpr int kWaitAll = 0x0070;  // vmcnt(0) expcnt(7) lgkmcnt(0), gfx9 encoding
  for (int st = 0;; st += 2) {
    ld_raw(cl_st(st + 1), raw);
    __builtin_amdgcn_sched_barrier(0);  // the prefetch issues first
    contract(qA0, cl_st(st + 1), qA1);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    __builtin_amdgcn_s_barrier();
    if (st + 1 >= nst) break;
    ld_raw(cl_st(st + 2), raw);
    __builtin_amdgcn_sched_barrier(0);
    contract(qA1, cl_st(st + 2), qA0);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    __builtin_amdgcn_s_barrier();
    if (st + 2 >= nst) break;
  }
  // The last stage's copy into the idle buffer and its reloads must land
  // before the workgroup's LDS is released.  The empty asm reads the
  // prefetched registers on the way out, so that the loads a stage issues
  // for the next one are live on both sides of the exit tests: the compiler
  // cannot sink them to just before their first use, where each would wait
  // out its latency.
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::"v"(raw.v0), "v"(raw.v1), "v"(raw.v2), "v"(raw.v3), "v"(raw.v4));

  // epilogue: lane (cl, g) holds rows 8 (e / 4) + 4 g + e % 4 of column cl
  // of each 32 x 32 block; split K stores the raw partial sums, otherwise the
  // bias is added.  A whole tile stores without per-value row tests.
  const int col = n0 + 32 * wave + cl;
  const int rows = M - m0 < kQM ? M - m0 : kQM;
  if (col < N) {
    float *dst = ksplit > 1 ? part + ((size_t)z * M + m0) * N + col : Y + (size_t)m0 * N + col;
    const float bv = ksplit > 1 || !bias ? 0.0f : bias[col];
    auto store = [&](bool guard) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
          if (!guard || r < rows) dst[(size_t)r * N] = ksplit > 1 ? acc[i][e] : acc[i][e] + bv;
        }
    };
    if (rows == kQM) {
      store(false);
    } else {
      store(true);
    }
  }
}

__global__ __launch_bounds__(256, 2) void gemm_q8_kernel(const uint16_t *__restrict__ X,
                                                         const uint8_t *__restrict__ W,
                                                         const float *__restrict__ bias, float *__restrict__ Y, int M,
                                                         int N, int K, int tiles_m, int tiles, int ksplit,
                                                         float *__restrict__ part) {
  q8_body<4>(X, W, bias, Y, M, N, K, tiles_m, tiles, ksplit, part);
}

__global__ __launch_bounds__(512, 1) void gemm_q8_wide_kernel(const uint16_t *__restrict__ X,
                                                              const uint8_t *__restrict__ W,
                                                              const float *__restrict__ bias, float *__restrict__ Y,
                                                              int M, int N, int K, int tiles_m, int tiles, int ksplit,
                                                              float *__restrict__ part) {
  q8_body<8>(X, W, bias, Y, M, N, K, tiles_m, tiles, ksplit, part);
}

int gemm_q8_tiles(int64_t M, int64_t N, int waves) {
  return (int)(((M + kQM - 1) / kQM) * ((N + 32 * waves - 1) / (32 * waves)));
}

hipError_t launch_gemm_q8(const void *x, const void *w, const float *bias, float *y, int64_t M, int64_t N, int64_t K,
                          int ksplit, int waves, float *part, hipStream_t s) {
  if (K % 256 != 0 || ksplit < 1 || ksplit > K / 128 || (waves != 4 && waves != 8)) return hipErrorInvalidValue;
  const int tiles_m = (int)((M + kQM - 1) / kQM);
  const int tiles = gemm_q8_tiles(M, N, waves);
  const int per_xcd = (tiles * ksplit + 7) / 8;
  launch_timed(waves == 8 ? gemm_q8_wide_kernel : gemm_q8_kernel, dim3((unsigned)(per_xcd * 8)), dim3(64 * waves), 0u,
               s, static_cast<const uint16_t *>(x), static_cast<const uint8_t *>(w), bias, y, (int)M, (int)N, (int)K,
               tiles_m, tiles, ksplit, part);
  return hipGetLastError();
}

}  // namespace okq
