/*
 * kquant_oracle.c -- CPU oracle for the k-quant linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product path (libokq.so) never links it.
 *
 * Contents and what each part restates:
 *   - fp16/bf16 -> f32 decode: crates/loader/src/safetensors_values.rs:115-123
 *     (bf16 << 16) and :155-183 (f16_bits_to_f32, incl. subnormal normalise
 *     loop, inf/NaN).  Pinned by the reference KATs :295-351.
 *   - f32 -> fp16 / bf16 rounding (round-to-nearest-even).  Not in the
 *     reference; IEEE 754 binary16 definition.  Pinned by exhaustive checks
 *     against numpy's float16 conversion.
 *   - GGUF block dequant for Q8_0 / Q4_K / Q6_K (the linear path's weights)
 *     and Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q2_K / Q3_K / Q5_K (the other block
 *     formats GgmlTensorType names, gguf_inspect.rs:132-167, served by the
 *     dequantize and row-gather entry points).  The reference has none
 *     (gguf_inspect.rs:208-219 leaves quantized byte_len = None); the layouts
 *     are the public GGUF/ggml block spec.  Pinned by an independent numpy
 *     bit-field decoder, closed forms and element-order probes.
 *   - Quantizers for the linear path's formats (Q8_0, Q4_K, Q5_K, Q6_K).
 *     The reference has none; this is the build's own algorithm (ggml-like,
 *     not bit-identical to ggml), defined exactly here so that the GPU
 *     quantizer can be checked byte-for-byte.
 *   - Seeded N(0, sigma) generator (SplitMix64 + Irwin-Hall(12) in integer
 *     arithmetic, so CPU and GPU produce identical floats).
 *   - The reference CPU linear path, restated with the same accumulation
 *     order: linear_out_by_in_compute (crates/kernels/src/lib.rs:1974-2123),
 *     linear_out_by_in_optimized_compute (:2216-2239), the AVX2 tile
 *     (crates/kernels/src/cpu_avx2.rs:58-253), the rows>=32 row-chunked
 *     dispatcher (lib.rs:2245, :2294-2390) and validate_linear_out_by_in
 *     (:2443-2497).
 *   - The projections' neighbours: rmsnorm (crates/kernels/src/rmsnorm.rs:
 *     73-128) and the gated SiLU of mlp_gated_silu (crates/kernels/src/mlp.rs:
 *     77-88, :233-238), same loops and order.  Pinned by the reference's own
 *     hand-checked values (rmsnorm.rs:150-258, mlp.rs:260-440).
 *
 * Build: gcc -O2 -ffp-contract=off (no FMA contraction: every product and sum
 * is rounded separately, as in the Rust scalar code).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>

#define OKR_API __attribute__((visibility("default")))

/* GGML type ids: crates/loader/src/gguf_inspect.rs:170-206. */
enum {
    OKR_F32 = 0, OKR_F16 = 1, OKR_Q4_0 = 2, OKR_Q4_1 = 3, OKR_Q5_0 = 6, OKR_Q5_1 = 7, OKR_Q8_0 = 8,
    OKR_Q2_K = 10, OKR_Q3_K = 11, OKR_Q4_K = 12, OKR_Q5_K = 13, OKR_Q6_K = 14, OKR_BF16 = 30
};

/* ------------------------------------------------------------------------ */
/* fp16 / bf16                                                               */
/* ------------------------------------------------------------------------ */

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* safetensors_values.rs:155-183 */
OKR_API float okr_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)(bits & 0x8000u)) << 16;
    uint32_t exp = (bits >> 10) & 0x1fu;
    uint32_t frac = bits & 0x03ffu;
    uint32_t out;
    if (exp == 0) {
        if (frac == 0) {
            out = sign;
        } else {
            uint32_t frac_norm = frac;
            int32_t exp_unbiased = -14;
            while ((frac_norm & 0x0400u) == 0) {
                frac_norm <<= 1;
                exp_unbiased -= 1;
            }
            frac_norm &= 0x03ffu;
            uint32_t exp32 = (uint32_t)(exp_unbiased + 127);
            out = sign | (exp32 << 23) | (frac_norm << 13);
        }
    } else if (exp == 0x1f) {
        out = sign | 0x7f800000u | (frac << 13);
    } else {
        out = sign | ((exp + (127 - 15)) << 23) | (frac << 13);
    }
    return bits_f32(out);
}

/* safetensors_values.rs:115-123 */
OKR_API float okr_bf16_to_f32(uint16_t bits) { return bits_f32(((uint32_t)bits) << 16); }

/* IEEE binary32 -> binary16, round to nearest even, subnormals kept,
 * overflow to inf, NaN kept quiet. */
OKR_API uint16_t okr_f32_to_f16(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t man = u & 0x7fffffu;
    if (exp == 0xff) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127; /* unbiased */
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        /* normal half: 10 mantissa bits kept, 13 rounded away */
        uint32_t half = ((uint32_t)(e + 15) << 10) | (man >> 13);
        uint32_t rem = man & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u; /* may carry into exp: fine */
        return (uint16_t)(sign | half);
    }
    if (e < -25) return sign; /* below half of the smallest subnormal */
    /* subnormal half: value = m * 2^-24 with m = round(full * 2^(e+24-23)) */
    uint32_t full = man | 0x800000u;          /* 24-bit significand */
    uint32_t shift = (uint32_t)(-e - 14 + 13); /* 14..24 */
    uint32_t half = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half & 1u))) half += 1u;
    return (uint16_t)(sign | half);
}

/* IEEE binary32 -> bfloat16, round to nearest even (NaN kept quiet). */
OKR_API uint16_t okr_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

OKR_API void okr_f16_to_f32_array(const uint16_t *src, int64_t n, float *dst) {
    for (int64_t i = 0; i < n; ++i) dst[i] = okr_f16_to_f32(src[i]);
}
OKR_API void okr_f32_to_f16_array(const float *src, int64_t n, uint16_t *dst) {
    for (int64_t i = 0; i < n; ++i) dst[i] = okr_f32_to_f16(src[i]);
}
OKR_API void okr_f32_to_bf16_array(const float *src, int64_t n, uint16_t *dst) {
    for (int64_t i = 0; i < n; ++i) dst[i] = okr_f32_to_bf16(src[i]);
}
OKR_API void okr_bf16_to_f32_array(const uint16_t *src, int64_t n, float *dst) {
    for (int64_t i = 0; i < n; ++i) dst[i] = okr_bf16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* Block formats (public GGUF spec; sizes 34 / 144 / 210 bytes)              */
/* ------------------------------------------------------------------------ */

OKR_API int64_t okr_block_elems(int type) {
    switch (type) {
    case OKR_Q4_0: case OKR_Q4_1: case OKR_Q5_0: case OKR_Q5_1: case OKR_Q8_0: return 32;
    case OKR_Q2_K: case OKR_Q3_K: case OKR_Q4_K: case OKR_Q5_K: case OKR_Q6_K: return 256;
    case OKR_F32: case OKR_F16: case OKR_BF16: return 1;
    default: return -1;
    }
}
OKR_API int64_t okr_block_bytes(int type) {
    switch (type) {
    case OKR_Q4_0: return 18;
    case OKR_Q4_1: return 20;
    case OKR_Q5_0: return 22;
    case OKR_Q5_1: return 24;
    case OKR_Q8_0: return 34;
    case OKR_Q2_K: return 84;
    case OKR_Q3_K: return 110;
    case OKR_Q4_K: return 144;
    case OKR_Q5_K: return 176;
    case OKR_Q6_K: return 210;
    case OKR_F32: return 4;
    case OKR_F16: case OKR_BF16: return 2;
    default: return -1;
    }
}

static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr_u16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* Q8_0 {f16 d; i8 qs[32]}: y[j] = qs[j] * d */
OKR_API int okr_dequant_q8_0(const uint8_t *src, int64_t n, float *dst) {
    if (n % 32) return 1;
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + b * 34;
        float d = okr_f16_to_f32(rd_u16(blk));
        for (int j = 0; j < 32; ++j) dst[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
    }
    return 0;
}

/* 6-bit (scale, min) of Q4_K sub-block j from the 12 packed bytes. */
static inline void q4k_scale_min(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* Q4_K {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}:
 * y[64c+l]    = (d*sc(2c))  *(qs[32c+l]&15) - (dmin*m(2c))
 * y[64c+32+l] = (d*sc(2c+1))*(qs[32c+l]>>4) - (dmin*m(2c+1)) */
OKR_API int okr_dequant_q4_k(const uint8_t *src, int64_t n, float *dst) {
    if (n % 256) return 1;
    for (int64_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = src + b * 144;
        float d = okr_f16_to_f32(rd_u16(blk));
        float dmin = okr_f16_to_f32(rd_u16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *qs = blk + 16;
        float *y = dst + b * 256;
        for (int c = 0; c < 4; ++c) {
            uint8_t sc, m;
            q4k_scale_min(2 * c, scales, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            q4k_scale_min(2 * c + 1, scales, &sc, &m);
            float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                y[64 * c + l] = d1 * (float)(qs[32 * c + l] & 15) - m1;
                y[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - m2;
            }
        }
    }
    return 0;
}

/* Q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}: see the spec in the
 * per-element comments below; y = (d*sc)*q with q in [-32, 31]. */
OKR_API int okr_dequant_q6_k(const uint8_t *src, int64_t n, float *dst) {
    if (n % 256) return 1;
    for (int64_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = src + b * 210;
        const uint8_t *ql = blk;
        const uint8_t *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        float d = okr_f16_to_f32(rd_u16(blk + 208));
        float *y = dst + b * 256;
        for (int h = 0; h < 2; ++h) {
            const uint8_t *qlh = ql + 64 * h;
            const uint8_t *qhh = qh + 32 * h;
            const int8_t *sch = sc + 8 * h;
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                int q1 = (int)((qlh[l] & 15) | (((qhh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((qlh[l + 32] & 15) | (((qhh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((qlh[l] >> 4) | (((qhh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((qlh[l + 32] >> 4) | (((qhh[l] >> 6) & 3) << 4)) - 32;
                y[128 * h + l] = (d * (float)sch[is + 0]) * (float)q1;
                y[128 * h + 32 + l] = (d * (float)sch[is + 2]) * (float)q2;
                y[128 * h + 64 + l] = (d * (float)sch[is + 4]) * (float)q3;
                y[128 * h + 96 + l] = (d * (float)sch[is + 6]) * (float)q4;
            }
        }
    }
    return 0;
}

/* ---- the other block formats (dequantize / row gather only) -------------- */

/* Q4_0 {f16 d; u8 qs[16]}: y[j] = ((qs[j]&15) - 8)*d, y[j+16] = ((qs[j]>>4) - 8)*d */
OKR_API int okr_dequant_q4_0(const uint8_t *src, int64_t n, float *dst) {
    if (n % 32) return 1;
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + b * 18;
        float d = okr_f16_to_f32(rd_u16(blk));
        for (int j = 0; j < 16; ++j) {
            dst[b * 32 + j] = (float)((blk[2 + j] & 15) - 8) * d;
            dst[b * 32 + j + 16] = (float)((blk[2 + j] >> 4) - 8) * d;
        }
    }
    return 0;
}

/* Q4_1 {f16 d; f16 m; u8 qs[16]}: y = q*d + m with q the nibble as above (no offset) */
OKR_API int okr_dequant_q4_1(const uint8_t *src, int64_t n, float *dst) {
    if (n % 32) return 1;
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + b * 20;
        float d = okr_f16_to_f32(rd_u16(blk));
        float m = okr_f16_to_f32(rd_u16(blk + 2));
        for (int j = 0; j < 16; ++j) {
            dst[b * 32 + j] = (float)(blk[4 + j] & 15) * d + m;
            dst[b * 32 + j + 16] = (float)(blk[4 + j] >> 4) * d + m;
        }
    }
    return 0;
}

/* Bit e (0..31) of the little-endian 32-bit high-bit word qh[4]: the fifth
 * bit of element e of a Q5_0 / Q5_1 block. */
static inline int q5_high_bit(const uint8_t *qh, int e) { return (qh[e >> 3] >> (e & 7)) & 1; }

/* Q5_0 {f16 d; u8 qh[4]; u8 qs[16]}: y[e] = ((nibble(e) | qh_bit(e)<<4) - 16)*d */
OKR_API int okr_dequant_q5_0(const uint8_t *src, int64_t n, float *dst) {
    if (n % 32) return 1;
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + b * 22;
        float d = okr_f16_to_f32(rd_u16(blk));
        const uint8_t *qh = blk + 2, *qs = blk + 6;
        for (int j = 0; j < 16; ++j) {
            int x0 = ((qs[j] & 15) | (q5_high_bit(qh, j) << 4)) - 16;
            int x1 = ((qs[j] >> 4) | (q5_high_bit(qh, j + 16) << 4)) - 16;
            dst[b * 32 + j] = (float)x0 * d;
            dst[b * 32 + j + 16] = (float)x1 * d;
        }
    }
    return 0;
}

/* Q5_1 {f16 d; f16 m; u8 qh[4]; u8 qs[16]}: y[e] = (nibble(e) | qh_bit(e)<<4)*d + m */
OKR_API int okr_dequant_q5_1(const uint8_t *src, int64_t n, float *dst) {
    if (n % 32) return 1;
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + b * 24;
        float d = okr_f16_to_f32(rd_u16(blk));
        float m = okr_f16_to_f32(rd_u16(blk + 2));
        const uint8_t *qh = blk + 4, *qs = blk + 8;
        for (int j = 0; j < 16; ++j) {
            int x0 = (qs[j] & 15) | (q5_high_bit(qh, j) << 4);
            int x1 = (qs[j] >> 4) | (q5_high_bit(qh, j + 16) << 4);
            dst[b * 32 + j] = (float)x0 * d + m;
            dst[b * 32 + j + 16] = (float)x1 * d + m;
        }
    }
    return 0;
}

/* Q2_K {u8 scales[16]; u8 qs[64]; f16 d; f16 dmin}: for half h (0,1) and
 * shift step j (0..3), the 32 elements 128h+32j+s (s < 32) take 2-bit
 * q = (qs[32h+s] >> 2j) & 3 and scale byte sc = scales[8h+2j+(s>=16)]
 * (= scales[e/16]):  y = (d*(sc&15))*q - (dmin*(sc>>4)). */
OKR_API int okr_dequant_q2_k(const uint8_t *src, int64_t n, float *dst) {
    if (n % 256) return 1;
    for (int64_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = src + b * 84;
        const uint8_t *scales = blk, *qs = blk + 16;
        float d = okr_f16_to_f32(rd_u16(blk + 80));
        float dmin = okr_f16_to_f32(rd_u16(blk + 82));
        float *y = dst + b * 256;
        for (int h = 0; h < 2; ++h) {
            for (int j = 0; j < 4; ++j) {
                for (int half16 = 0; half16 < 2; ++half16) {
                    uint8_t sc = scales[8 * h + 2 * j + half16];
                    float dl = d * (float)(sc & 15), ml = dmin * (float)(sc >> 4);
                    for (int l = 0; l < 16; ++l) {
                        int s = 16 * half16 + l;
                        int q = (qs[32 * h + s] >> (2 * j)) & 3;
                        y[128 * h + 32 * j + s] = dl * (float)q - ml;
                    }
                }
            }
        }
    }
    return 0;
}

/* 6-bit scale i (0..15) of a Q3_K block from its 12 packed bytes: low four
 * bits are the low nibble of byte i (i < 8) or the high nibble of byte i-8;
 * the top two bits are bits 2*(i/4)..+1 of byte 8 + i%4. */
static inline int q3k_scale(const uint8_t *s, int i) {
    int lo = i < 8 ? (s[i] & 15) : (s[i - 8] >> 4);
    int hi = (s[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
    return lo | (hi << 4);
}

/* Q3_K {u8 hmask[32]; u8 qs[64]; u8 scales[12]; f16 d}: element
 * e = 128h+32j+s takes the 2 low bits (qs[32h+s] >> 2j) & 3, minus 4 when bit
 * 4h+j of hmask[s] is clear:  y = (d*(scale(e/16) - 32)) * q. */
OKR_API int okr_dequant_q3_k(const uint8_t *src, int64_t n, float *dst) {
    if (n % 256) return 1;
    for (int64_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = src + b * 110;
        const uint8_t *hm = blk, *qs = blk + 32, *scales = blk + 96;
        float d = okr_f16_to_f32(rd_u16(blk + 108));
        float *y = dst + b * 256;
        for (int h = 0; h < 2; ++h) {
            for (int j = 0; j < 4; ++j) {
                for (int half16 = 0; half16 < 2; ++half16) {
                    int is = 8 * h + 2 * j + half16;
                    float dl = d * (float)(q3k_scale(scales, is) - 32);
                    for (int l = 0; l < 16; ++l) {
                        int s = 16 * half16 + l;
                        int q = ((qs[32 * h + s] >> (2 * j)) & 3) - (((hm[s] >> (4 * h + j)) & 1) ? 0 : 4);
                        y[128 * h + 32 * j + s] = dl * (float)q;
                    }
                }
            }
        }
    }
    return 0;
}

/* Q5_K {f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]}: as Q4_K with
 * a fifth bit, bit 2c+hi of qh[l], added as 16:
 * y[64c+32hi+l] = (d*sc(2c+hi)) * (nibble + 16*bit) - (dmin*m(2c+hi)). */
OKR_API int okr_dequant_q5_k(const uint8_t *src, int64_t n, float *dst) {
    if (n % 256) return 1;
    for (int64_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = src + b * 176;
        float d = okr_f16_to_f32(rd_u16(blk));
        float dmin = okr_f16_to_f32(rd_u16(blk + 2));
        const uint8_t *scales = blk + 4, *qh = blk + 16, *qs = blk + 48;
        float *y = dst + b * 256;
        for (int c = 0; c < 4; ++c) {
            uint8_t sc, m;
            q4k_scale_min(2 * c, scales, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            q4k_scale_min(2 * c + 1, scales, &sc, &m);
            float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                int q1 = (qs[32 * c + l] & 15) + (((qh[l] >> (2 * c)) & 1) ? 16 : 0);
                int q2 = (qs[32 * c + l] >> 4) + (((qh[l] >> (2 * c + 1)) & 1) ? 16 : 0);
                y[64 * c + l] = d1 * (float)q1 - m1;
                y[64 * c + 32 + l] = d2 * (float)q2 - m2;
            }
        }
    }
    return 0;
}

OKR_API int okr_dequantize(int type, const uint8_t *src, int64_t n, float *dst) {
    switch (type) {
    case OKR_Q4_0: return okr_dequant_q4_0(src, n, dst);
    case OKR_Q4_1: return okr_dequant_q4_1(src, n, dst);
    case OKR_Q5_0: return okr_dequant_q5_0(src, n, dst);
    case OKR_Q5_1: return okr_dequant_q5_1(src, n, dst);
    case OKR_Q2_K: return okr_dequant_q2_k(src, n, dst);
    case OKR_Q3_K: return okr_dequant_q3_k(src, n, dst);
    case OKR_Q5_K: return okr_dequant_q5_k(src, n, dst);
    case OKR_Q8_0: return okr_dequant_q8_0(src, n, dst);
    case OKR_Q4_K: return okr_dequant_q4_k(src, n, dst);
    case OKR_Q6_K: return okr_dequant_q6_k(src, n, dst);
    default: return 2;
    }
}

/* ------------------------------------------------------------------------ */
/* Quantizers (the build's own algorithm, fixed exactly here)                */
/* ------------------------------------------------------------------------ */

static inline float minf_(float a, float b) { return a < b ? a : b; }
static inline float maxf_(float a, float b) { return a > b ? a : b; }
static inline int clampi_(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Q8_0: d = amax/127 (f32), id = 1/d, q = rint(x*id) clamped to +-127,
 * stored d = fp16(d). */
OKR_API int okr_quantize_q8_0(const float *x, int64_t n, uint8_t *dst) {
    if (n % 32) return 1;
    for (int64_t b = 0; b < n / 32; ++b) {
        const float *xb = x + b * 32;
        uint8_t *blk = dst + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = maxf_(amax, fabsf(xb[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr_u16(blk, okr_f32_to_f16(d));
        for (int j = 0; j < 32; ++j) {
            int q = (int)rintf(xb[j] * id);
            blk[2 + j] = (uint8_t)(int8_t)clampi_(q, -127, 127);
        }
    }
    return 0;
}

/* Q4_K (levels 15) and Q5_K (levels 31): per 32-sub-block
 * mn = min(0, min x), mx = max x, scale = (mx - mn)/levels, mmin = -mn;
 * super-block d = max(scale)/63, dmin = max(mmin)/63; 6-bit
 * ls = rint(scale*63/max_scale), lm likewise;
 * q = clamp(rint((x + dmin16*lm) / (d16*ls)), 0, levels).  Q5_K stores the
 * low four bits of q in qs and bit 4 of element l of chunk c in bit 2c (low
 * nibble) or 2c+1 (high nibble) of qh[l]. */
static int quantize_q45_k(const float *x, int64_t n, uint8_t *dst, int q5) {
    if (n % 256) return 1;
    const float levels = q5 ? 31.0f : 15.0f;
    const int maxq = q5 ? 31 : 15;
    const int64_t bytes = q5 ? 176 : 144;
    for (int64_t b = 0; b < n / 256; ++b) {
        const float *xb = x + b * 256;
        uint8_t *blk = dst + b * bytes;
        float scale[8], mmin[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int s = 0; s < 8; ++s) {
            float mn = xb[32 * s], mx = xb[32 * s];
            for (int j = 1; j < 32; ++j) {
                mn = minf_(mn, xb[32 * s + j]);
                mx = maxf_(mx, xb[32 * s + j]);
            }
            mn = minf_(mn, 0.0f);
            scale[s] = (mx - mn) / levels;
            mmin[s] = -mn;
            max_scale = maxf_(max_scale, scale[s]);
            max_min = maxf_(max_min, mmin[s]);
        }
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        uint8_t ls[8], lm[8];
        for (int s = 0; s < 8; ++s) {
            ls[s] = (uint8_t)clampi_((int)rintf(inv_scale * scale[s]), 0, 63);
            lm[s] = (uint8_t)clampi_((int)rintf(inv_min * mmin[s]), 0, 63);
        }
        uint16_t dh = okr_f32_to_f16(max_scale / 63.0f);
        uint16_t dminh = okr_f32_to_f16(max_min / 63.0f);
        wr_u16(blk, dh);
        wr_u16(blk + 2, dminh);
        uint8_t *sc = blk + 4;
        for (int j = 0; j < 8; ++j) {
            if (j < 4) {
                sc[j] = ls[j];
                sc[j + 4] = lm[j];
            } else {
                sc[j + 4] = (uint8_t)((ls[j] & 0x0f) | ((lm[j] & 0x0f) << 4));
                sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
                sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
            }
        }
        float d16 = okr_f16_to_f32(dh), dmin16 = okr_f16_to_f32(dminh);
        uint8_t L[256];
        for (int s = 0; s < 8; ++s) {
            float de = d16 * (float)ls[s];
            float me = dmin16 * (float)lm[s];
            for (int j = 0; j < 32; ++j) {
                int q = 0;
                if (de != 0.0f) q = clampi_((int)rintf((xb[32 * s + j] + me) / de), 0, maxq);
                L[32 * s + j] = (uint8_t)q;
            }
        }
        uint8_t *qs = blk + (q5 ? 48 : 16);
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l)
                qs[32 * c + l] = (uint8_t)((L[64 * c + l] & 15) | ((L[64 * c + 32 + l] & 15) << 4));
        if (q5) {
            uint8_t *qh = blk + 16;
            for (int l = 0; l < 32; ++l) {
                uint8_t h = 0;
                for (int c = 0; c < 4; ++c)
                    h |= (uint8_t)(((L[64 * c + l] >> 4) << (2 * c)) | ((L[64 * c + 32 + l] >> 4) << (2 * c + 1)));
                qh[l] = h;
            }
        }
    }
    return 0;
}

OKR_API int okr_quantize_q4_k(const float *x, int64_t n, uint8_t *dst) { return quantize_q45_k(x, n, dst, 0); }
OKR_API int okr_quantize_q5_k(const float *x, int64_t n, uint8_t *dst) { return quantize_q45_k(x, n, dst, 1); }

/* Q6_K: per 16-sub-block the signed value of largest |x| (first on ties)
 * gives scale = -mx/32; super-block iscale = -128/max_scale (signed, largest
 * |scale|), sc = clamp(rint(iscale*scale), -128, 127), d = fp16(1/iscale);
 * q = clamp(rint(x/(d16*sc)), -32, 31) stored as q+32. */
OKR_API int okr_quantize_q6_k(const float *x, int64_t n, uint8_t *dst) {
    if (n % 256) return 1;
    for (int64_t b = 0; b < n / 256; ++b) {
        const float *xb = x + b * 256;
        uint8_t *blk = dst + b * 210;
        float scale[16];
        float max_scale = 0.0f, max_abs_scale = 0.0f;
        for (int s = 0; s < 16; ++s) {
            float mx = 0.0f, amax = 0.0f;
            for (int j = 0; j < 16; ++j) {
                float v = xb[16 * s + j];
                float a = fabsf(v);
                if (a > amax) { amax = a; mx = v; }
            }
            scale[s] = -mx / 32.0f;
            float as = fabsf(scale[s]);
            if (as > max_abs_scale) { max_abs_scale = as; max_scale = scale[s]; }
        }
        float iscale = max_scale != 0.0f ? -128.0f / max_scale : 0.0f;
        float d = iscale != 0.0f ? 1.0f / iscale : 0.0f;
        uint16_t dh = okr_f32_to_f16(d);
        float d16 = okr_f16_to_f32(dh);
        int8_t scs[16];
        for (int s = 0; s < 16; ++s) scs[s] = (int8_t)clampi_((int)rintf(iscale * scale[s]), -128, 127);
        uint8_t L[256];
        for (int s = 0; s < 16; ++s) {
            float de = d16 * (float)scs[s];
            for (int j = 0; j < 16; ++j) {
                int q = 0;
                if (de != 0.0f) q = clampi_((int)rintf(xb[16 * s + j] / de), -32, 31);
                L[16 * s + j] = (uint8_t)(q + 32);
            }
        }
        uint8_t *ql = blk, *qh = blk + 128;
        for (int h = 0; h < 2; ++h) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t *Lh = L + 128 * h;
                ql[64 * h + l] = (uint8_t)((Lh[l] & 15) | ((Lh[64 + l] & 15) << 4));
                ql[64 * h + 32 + l] = (uint8_t)((Lh[32 + l] & 15) | ((Lh[96 + l] & 15) << 4));
                qh[32 * h + l] = (uint8_t)((Lh[l] >> 4) | ((Lh[32 + l] >> 4) << 2) | ((Lh[64 + l] >> 4) << 4) |
                                           ((Lh[96 + l] >> 4) << 6));
            }
        }
        memcpy(blk + 192, scs, 16);
        wr_u16(blk + 208, dh);
    }
    return 0;
}

OKR_API int okr_quantize(int type, const float *x, int64_t n, uint8_t *dst) {
    switch (type) {
    case OKR_Q8_0: return okr_quantize_q8_0(x, n, dst);
    case OKR_Q4_K: return okr_quantize_q4_k(x, n, dst);
    case OKR_Q5_K: return okr_quantize_q5_k(x, n, dst);
    case OKR_Q6_K: return okr_quantize_q6_k(x, n, dst);
    default: return 2;
    }
}

/* ------------------------------------------------------------------------ */
/* Seeded N(0, sigma): SplitMix64 counter stream, Irwin-Hall of 12 24-bit    */
/* uniforms summed in integers; one int->float rounding, exact 2^-24 scale,  */
/* one multiply by sigma.                                                    */
/* ------------------------------------------------------------------------ */

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

OKR_API float okr_normal_at(uint64_t seed, int64_t i, float sigma) {
    uint64_t key = mix64(seed);
    int32_t s = 0;
    for (int j = 0; j < 6; ++j) {
        uint64_t z = mix64(key + ((uint64_t)i * 6u + (uint64_t)j + 1u) * 0x9E3779B97F4A7C15ull);
        s += (int32_t)(z & 0xffffffu) + (int32_t)((z >> 32) & 0xffffffu);
    }
    s -= 6 * 0xffffff;
    float u = (float)s * 5.9604644775390625e-08f; /* 2^-24 */
    return u * sigma;
}

OKR_API void okr_fill_normal(uint64_t seed, int64_t offset, int64_t n, float sigma, float *dst) {
    for (int64_t i = 0; i < n; ++i) dst[i] = okr_normal_at(seed, offset + i, sigma);
}

/* ------------------------------------------------------------------------ */
/* Reference CPU linear path                                                */
/* ------------------------------------------------------------------------ */

static char g_err[512];
OKR_API const char *okr_last_error(void) { return g_err; }

static int checked_mul(int64_t a, int64_t b, int64_t *out) {
    if (a < 0 || b < 0) return 1;
    if (a != 0 && b > INT64_MAX / a) return 1;
    *out = a * b;
    return 0;
}

/* validate_linear_out_by_in (lib.rs:2443-2497): lengths in elements. */
OKR_API int okr_validate_linear(int64_t x_len, int64_t rows, int64_t in_f, int64_t w_len, int64_t out_f,
                                int64_t bias_len, int64_t out_len) {
    int64_t xe, we, oe;
    if (checked_mul(rows, in_f, &xe)) { snprintf(g_err, sizeof g_err, "linear_out_by_in x length overflows"); return 1; }
    if (checked_mul(out_f, in_f, &we)) { snprintf(g_err, sizeof g_err, "linear_out_by_in weight length overflows"); return 1; }
    if (checked_mul(rows, out_f, &oe)) { snprintf(g_err, sizeof g_err, "linear_out_by_in out length overflows"); return 1; }
    if (x_len != xe) {
        snprintf(g_err, sizeof g_err, "linear_out_by_in x.len()=%lld does not match rows*in_features=%lld*%lld=%lld",
                 (long long)x_len, (long long)rows, (long long)in_f, (long long)xe);
        return 1;
    }
    if (w_len != we) {
        snprintf(g_err, sizeof g_err,
                 "linear_out_by_in weight.len()=%lld does not match out_features*in_features=%lld*%lld=%lld",
                 (long long)w_len, (long long)out_f, (long long)in_f, (long long)we);
        return 1;
    }
    if (bias_len >= 0 && bias_len != out_f) {
        snprintf(g_err, sizeof g_err, "linear_out_by_in bias.len()=%lld does not match out_features=%lld",
                 (long long)bias_len, (long long)out_f);
        return 1;
    }
    if (out_len != oe) {
        snprintf(g_err, sizeof g_err, "linear_out_by_in out.len()=%lld does not match rows*out_features=%lld*%lld=%lld",
                 (long long)out_len, (long long)rows, (long long)out_f, (long long)oe);
        return 1;
    }
    return 0;
}

#define BIAS(o) (bias ? bias[(o)] : 0.0f)

/* linear_out_by_in_compute (lib.rs:1974-2123): 4 rows x 4 outputs register
 * tile, accumulators start at bias, sequential += over k, then the output
 * tail (4 rows x 1 output) and the row tail (1 row x 4 outputs, then 1x1). */
static void linear_scalar_compute(const float *x, int64_t rows, int64_t in_f, const float *w, int64_t out_f,
                                  const float *bias, float *out) {
    int64_t tiled_rows = rows - rows % 4;
    int64_t tiled_out = out_f - out_f % 4;
    for (int64_t row = 0; row < tiled_rows; row += 4) {
        const float *x0 = x + row * in_f, *x1 = x0 + in_f, *x2 = x1 + in_f, *x3 = x2 + in_f;
        for (int64_t o = 0; o < tiled_out; o += 4) {
            float a00 = BIAS(o), a01 = a00, a02 = a00, a03 = a00;
            float a10 = BIAS(o + 1), a11 = a10, a12 = a10, a13 = a10;
            float a20 = BIAS(o + 2), a21 = a20, a22 = a20, a23 = a20;
            float a30 = BIAS(o + 3), a31 = a30, a32 = a30, a33 = a30;
            const float *w0 = w + o * in_f, *w1 = w0 + in_f, *w2 = w1 + in_f, *w3 = w2 + in_f;
            for (int64_t k = 0; k < in_f; ++k) {
                float wv0 = w0[k], wv1 = w1[k], wv2 = w2[k], wv3 = w3[k];
                float xv0 = x0[k], xv1 = x1[k], xv2 = x2[k], xv3 = x3[k];
                a00 += xv0 * wv0; a10 += xv0 * wv1; a20 += xv0 * wv2; a30 += xv0 * wv3;
                a01 += xv1 * wv0; a11 += xv1 * wv1; a21 += xv1 * wv2; a31 += xv1 * wv3;
                a02 += xv2 * wv0; a12 += xv2 * wv1; a22 += xv2 * wv2; a32 += xv2 * wv3;
                a03 += xv3 * wv0; a13 += xv3 * wv1; a23 += xv3 * wv2; a33 += xv3 * wv3;
            }
            float *r0 = out + row * out_f + o, *r1 = r0 + out_f, *r2 = r1 + out_f, *r3 = r2 + out_f;
            r0[0] = a00; r0[1] = a10; r0[2] = a20; r0[3] = a30;
            r1[0] = a01; r1[1] = a11; r1[2] = a21; r1[3] = a31;
            r2[0] = a02; r2[1] = a12; r2[2] = a22; r2[3] = a32;
            r3[0] = a03; r3[1] = a13; r3[2] = a23; r3[3] = a33;
        }
        for (int64_t o = tiled_out; o < out_f; ++o) {
            float a0 = BIAS(o), a1 = a0, a2 = a0, a3 = a0;
            const float *wr = w + o * in_f;
            for (int64_t k = 0; k < in_f; ++k) {
                float wv = wr[k];
                a0 += x0[k] * wv; a1 += x1[k] * wv; a2 += x2[k] * wv; a3 += x3[k] * wv;
            }
            out[row * out_f + o] = a0;
            out[(row + 1) * out_f + o] = a1;
            out[(row + 2) * out_f + o] = a2;
            out[(row + 3) * out_f + o] = a3;
        }
    }
    for (int64_t row = tiled_rows; row < rows; ++row) {
        const float *xr = x + row * in_f;
        float *orow = out + row * out_f;
        for (int64_t o = 0; o < tiled_out; o += 4) {
            float a0 = BIAS(o), a1 = BIAS(o + 1), a2 = BIAS(o + 2), a3 = BIAS(o + 3);
            const float *w0 = w + o * in_f, *w1 = w0 + in_f, *w2 = w1 + in_f, *w3 = w2 + in_f;
            for (int64_t k = 0; k < in_f; ++k) {
                float xv = xr[k];
                a0 += xv * w0[k]; a1 += xv * w1[k]; a2 += xv * w2[k]; a3 += xv * w3[k];
            }
            orow[o] = a0; orow[o + 1] = a1; orow[o + 2] = a2; orow[o + 3] = a3;
        }
        for (int64_t o = tiled_out; o < out_f; ++o) {
            float a = BIAS(o);
            for (int64_t k = 0; k < in_f; ++k) a += xr[k] * w[o * in_f + k];
            orow[o] = a;
        }
    }
}

/* linear_out_by_in_optimized_compute (lib.rs:2216-2239): out row = bias,
 * then for each k an axpy over all outputs (strided weight walk). */
static void linear_optimized_compute(const float *x, int64_t rows, int64_t in_f, const float *w, int64_t out_f,
                                     const float *bias, float *out) {
    for (int64_t row = 0; row < rows; ++row) {
        float *orow = out + row * out_f;
        for (int64_t o = 0; o < out_f; ++o) orow[o] = BIAS(o);
        const float *xr = x + row * in_f;
        for (int64_t k = 0; k < in_f; ++k) {
            float xv = xr[k];
            for (int64_t o = 0; o < out_f; ++o) orow[o] += xv * w[o * in_f + k];
        }
    }
}

__attribute__((target("avx2"))) static inline float hsum256(__m256 v) {
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 s = _mm_add_ps(hi, lo);
    __m128 sh = _mm_movehdup_ps(s);
    __m128 s64 = _mm_add_ps(s, sh);
    __m128 sh2 = _mm_movehl_ps(sh, s64);
    return _mm_cvtss_f32(_mm_add_ss(s64, sh2));
}

/* linear_out_by_in_compute_avx2 (cpu_avx2.rs:58-253): 4x4 tile of 8-wide FMA
 * accumulators starting at zero, hsum, scalar K tail, then + bias; output
 * tail and row tail are scalar with bias-initialised accumulators. */
__attribute__((target("avx2,fma"))) static void linear_avx2_compute(const float *x, int64_t rows, int64_t in_f,
                                                                   const float *w, int64_t out_f,
                                                                   const float *bias, float *out) {
    int64_t tiled_rows = rows - rows % 4;
    int64_t tiled_out = out_f - out_f % 4;
    int64_t k_simd = in_f - in_f % 8;
    for (int64_t row = 0; row < tiled_rows; row += 4) {
        const float *xb0 = x + row * in_f, *xb1 = xb0 + in_f, *xb2 = xb1 + in_f, *xb3 = xb2 + in_f;
        for (int64_t o = 0; o < tiled_out; o += 4) {
            const float *wb0 = w + o * in_f, *wb1 = wb0 + in_f, *wb2 = wb1 + in_f, *wb3 = wb2 + in_f;
            __m256 acc[4][4];
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 4; ++j) acc[i][j] = _mm256_setzero_ps();
            int64_t k = 0;
            for (; k < k_simd; k += 8) {
                __m256 xv[4] = {_mm256_loadu_ps(xb0 + k), _mm256_loadu_ps(xb1 + k), _mm256_loadu_ps(xb2 + k),
                                _mm256_loadu_ps(xb3 + k)};
                __m256 wv[4] = {_mm256_loadu_ps(wb0 + k), _mm256_loadu_ps(wb1 + k), _mm256_loadu_ps(wb2 + k),
                                _mm256_loadu_ps(wb3 + k)};
                for (int i = 0; i < 4; ++i)
                    for (int j = 0; j < 4; ++j) acc[i][j] = _mm256_fmadd_ps(xv[i], wv[j], acc[i][j]);
            }
            float s[4][4];
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 4; ++j) s[i][j] = hsum256(acc[i][j]);
            const float *xs[4] = {xb0, xb1, xb2, xb3};
            const float *ws[4] = {wb0, wb1, wb2, wb3};
            for (int64_t kt = k_simd; kt < in_f; ++kt)
                for (int i = 0; i < 4; ++i)
                    for (int j = 0; j < 4; ++j) s[i][j] += xs[i][kt] * ws[j][kt];
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 4; ++j) out[(row + i) * out_f + o + j] = s[i][j] + BIAS(o + j);
        }
        for (int64_t o = tiled_out; o < out_f; ++o) {
            const float *wb = w + o * in_f;
            float b = BIAS(o);
            float s0 = b, s1 = b, s2 = b, s3 = b;
            for (int64_t k = 0; k < in_f; ++k) {
                float wv = wb[k];
                s0 += xb0[k] * wv; s1 += xb1[k] * wv; s2 += xb2[k] * wv; s3 += xb3[k] * wv;
            }
            out[row * out_f + o] = s0;
            out[(row + 1) * out_f + o] = s1;
            out[(row + 2) * out_f + o] = s2;
            out[(row + 3) * out_f + o] = s3;
        }
    }
    for (int64_t row = tiled_rows; row < rows; ++row) {
        const float *xb = x + row * in_f;
        for (int64_t o = 0; o < out_f; ++o) {
            const float *wb = w + o * in_f;
            float s = BIAS(o);
            for (int64_t k = 0; k < in_f; ++k) s += xb[k] * wb[k];
            out[row * out_f + o] = s;
        }
    }
}

/* Modes: 0 scalar, 1 optimized, 2 avx2 (CpuKernelMode, lib.rs). */
typedef void (*compute_fn)(const float *, int64_t, int64_t, const float *, int64_t, const float *, float *);
static compute_fn mode_fn(int mode) {
    switch (mode) {
    case 0: return linear_scalar_compute;
    case 1: return linear_optimized_compute;
    case 2: return linear_avx2_compute;
    default: return NULL;
    }
}

OKR_API int okr_has_avx2(void) { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }

typedef struct {
    compute_fn fn;
    const float *x, *w, *bias;
    float *out;
    int64_t rows, in_f, out_f;
} chunk_job;

static void *chunk_main(void *p) {
    chunk_job *j = (chunk_job *)p;
    j->fn(j->x, j->rows, j->in_f, j->w, j->out_f, j->bias, j->out);
    return NULL;
}

/* CpuKernelBackend::linear_out_by_in (lib.rs:1159-1213) with a pool of
 * `threads` threads: serial below 32 rows (:2245), otherwise the row-chunked
 * dispatcher (:2294-2390) -- chunks of ceil(ceil(rows/4)/threads)*4 rows, each
 * computed by the serial body, so results are bit-identical to serial.
 * threads <= 1 means "no pool" (always serial). */
OKR_API int okr_linear_out_by_in(int mode, int threads, const float *x, int64_t rows, int64_t in_f, const float *w,
                                 int64_t out_f, const float *bias, float *out) {
    compute_fn fn = mode_fn(mode);
    if (!fn) { snprintf(g_err, sizeof g_err, "unknown cpu kernel mode %d", mode); return 2; }
    if (mode == 2 && !okr_has_avx2()) {
        snprintf(g_err, sizeof g_err, "CpuKernelMode::Avx2 requires runtime avx2 + fma support");
        return 2;
    }
    if (threads <= 1 || rows < 32) {
        fn(x, rows, in_f, w, out_f, bias, out);
        return 0;
    }
    int64_t tiles_total = (rows + 3) / 4;
    int64_t tiles_per_chunk = (tiles_total + threads - 1) / threads;
    if (tiles_per_chunk < 1) tiles_per_chunk = 1;
    int64_t rows_per_chunk = tiles_per_chunk * 4;
    int64_t nchunks = (rows + rows_per_chunk - 1) / rows_per_chunk;
    pthread_t *tids = (pthread_t *)calloc((size_t)nchunks, sizeof(pthread_t));
    chunk_job *jobs = (chunk_job *)calloc((size_t)nchunks, sizeof(chunk_job));
    if (!tids || !jobs) { free(tids); free(jobs); return 3; }
    for (int64_t c = 0; c < nchunks; ++c) {
        int64_t r0 = c * rows_per_chunk;
        int64_t nr = rows - r0 < rows_per_chunk ? rows - r0 : rows_per_chunk;
        jobs[c] = (chunk_job){fn, x + r0 * in_f, w, bias, out + r0 * out_f, nr, in_f, out_f};
        pthread_create(&tids[c], NULL, chunk_main, &jobs[c]);
    }
    for (int64_t c = 0; c < nchunks; ++c) pthread_join(tids[c], NULL);
    free(tids);
    free(jobs);
    return 0;
}

/* Quantized reference path: dequantize with the oracle, then the f32 linear
 * above.  Convenience for tests; weights are [out_f, in_f] GGUF rows. */
OKR_API int okr_linear_q(int type, int mode, int threads, const float *x, int64_t rows, int64_t in_f,
                         const uint8_t *wq, int64_t out_f, const float *bias, float *out) {
    float *w = (float *)malloc((size_t)(out_f * in_f) * sizeof(float));
    if (!w) return 3;
    int rc = okr_dequantize(type, wq, out_f * in_f, w);
    if (rc == 0) rc = okr_linear_out_by_in(mode, threads, x, rows, in_f, w, out_f, bias, out);
    free(w);
    return rc;
}

/* ---- neighbours of the projections -------------------------------------- */

/* rmsnorm, crates/kernels/src/rmsnorm.rs:116-128: sequential f32 sum of
 * squares per row, mean, sqrt(mean + eps), reciprocal, then
 * out = row[i] * inv_rms * weight[i] left to right. */
OKR_API void okr_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *weight, float eps, float *out) {
  const float hidden_f = (float)hidden;
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * hidden;
    float sum_sq = 0.0f;
    for (int64_t i = 0; i < hidden; ++i) sum_sq += row[i] * row[i];
    const float mean_sq = sum_sq / hidden_f;
    const float rms = sqrtf(mean_sq + eps);
    const float inv_rms = 1.0f / rms;
    for (int64_t i = 0; i < hidden; ++i) out[r * hidden + i] = row[i] * inv_rms * weight[i];
  }
}

/* silu_inplace then the element-wise product with up, mlp.rs:77-88 and
 * :233-238: sigmoid = 1 / (1 + exp(-g)); g *= sigmoid; g *= up. */
OKR_API void okr_swiglu(const float *gate, const float *up, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) {
    float v = gate[i];
    const float sigmoid = 1.0f / (1.0f + expf(-v));
    v *= sigmoid;
    out[i] = v * up[i];
  }
}
