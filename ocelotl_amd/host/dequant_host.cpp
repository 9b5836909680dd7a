// dequant_host.cpp -- GGUF block dequantization on the host (see
// dequant_host.hpp).  Built with -ffp-contract=off: each product and each
// difference below is its own rounding, as in the block definitions.
#include "dequant_host.hpp"

#include <cstring>
#include <string>

namespace ocelotl {

namespace {

float bits_to_f32(uint32_t u) {
  float f;
  std::memcpy(&f, &u, sizeof f);
  return f;
}

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// Q4_K / Q5_K 6-bit (scale, min) of sub-block j < 8 from the 12 packed bytes:
// j < 4 takes the low six bits of bytes j and j + 4; j >= 4 a nibble of byte
// j + 4 plus the top two bits of bytes j - 4 (scale) and j (min).
void kquant_scale_min(int j, const uint8_t *s, int &sc, int &m) {
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// Q8_0: {f16 d; int8 q[32]} (34 bytes), y = q * d.
void block_q8_0(const uint8_t *b, float *y) {
  const float d = half_to_f32(rd16(b));
  for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
}

// Q4_K: {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]} (144 bytes).  64-element
// chunk c: y[64c + l] = d*sc(2c) * lo(qs[32c + l]) - dmin*m(2c),
// y[64c + 32 + l] = d*sc(2c+1) * hi(qs[32c + l]) - dmin*m(2c+1).
void block_q4_k(const uint8_t *b, float *y) {
  const float d = half_to_f32(rd16(b)), dmin = half_to_f32(rd16(b + 2));
  const uint8_t *sc = b + 4, *qs = b + 16;
  for (int c = 0; c < 4; ++c) {
    int s0, m0, s1, m1;
    kquant_scale_min(2 * c, sc, s0, m0);
    kquant_scale_min(2 * c + 1, sc, s1, m1);
    const float d1 = d * (float)s0, mn1 = dmin * (float)m0;
    const float d2 = d * (float)s1, mn2 = dmin * (float)m1;
    for (int l = 0; l < 32; ++l) {
      y[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0x0F) - mn1;
      y[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - mn2;
    }
  }
}

// Q5_K: {f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]} (176 bytes).
// As Q4_K with a fifth bit per element: bit 2c of qh[l] for the low nibbles
// of chunk c, bit 2c + 1 for the high ones (+16 when set).
void block_q5_k(const uint8_t *b, float *y) {
  const float d = half_to_f32(rd16(b)), dmin = half_to_f32(rd16(b + 2));
  const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
  for (int c = 0; c < 4; ++c) {
    int s0, m0, s1, m1;
    kquant_scale_min(2 * c, sc, s0, m0);
    kquant_scale_min(2 * c + 1, sc, s1, m1);
    const float d1 = d * (float)s0, mn1 = dmin * (float)m0;
    const float d2 = d * (float)s1, mn2 = dmin * (float)m1;
    for (int l = 0; l < 32; ++l) {
      const int lo = (qs[32 * c + l] & 0x0F) + (((qh[l] >> (2 * c)) & 1) << 4);
      const int hi = (qs[32 * c + l] >> 4) + (((qh[l] >> (2 * c + 1)) & 1) << 4);
      y[64 * c + l] = d1 * (float)lo - mn1;
      y[64 * c + 32 + l] = d2 * (float)hi - mn2;
    }
  }
}

// Q6_K: {u8 ql[128]; u8 qh[64]; int8 scales[16]; f16 d} (210 bytes, d last).
// Half h (ql + 64h, qh + 32h, scales + 8h), l < 32, is = l / 16: four 6-bit
// values (low or high nibble of ql[l] / ql[l + 32], two bits of qh[l]) minus
// 32, at y[128h + l + 32t] with scale sc[is + 2t]: y = (d * sc) * q.
void block_q6_k(const uint8_t *b, float *y) {
  const float d = half_to_f32(rd16(b + 208));
  for (int h = 0; h < 2; ++h) {
    const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
    const int8_t *sc = reinterpret_cast<const int8_t *>(b + 192 + 8 * h);
    float *yh = y + 128 * h;
    for (int l = 0; l < 32; ++l) {
      const int is = l / 16;
      const int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
      const int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
      const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      yh[l] = (d * (float)sc[is]) * (float)q1;
      yh[l + 32] = (d * (float)sc[is + 2]) * (float)q2;
      yh[l + 64] = (d * (float)sc[is + 4]) * (float)q3;
      yh[l + 96] = (d * (float)sc[is + 6]) * (float)q4;
    }
  }
}

}  // namespace

float half_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1F, mant = h & 0x3FF;
  if (exp == 0x1F) return bits_to_f32(sign | 0x7F800000u | (mant << 13));  // inf / NaN (payload kept)
  if (exp == 0) {
    if (mant == 0) return bits_to_f32(sign);
    // subnormal: normalise the mantissa
    int e = -1;
    do {
      ++e;
      mant <<= 1;
    } while (!(mant & 0x400));
    return bits_to_f32(sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3FF) << 13));
  }
  return bits_to_f32(sign | ((exp + 127 - 15) << 23) | (mant << 13));
}

bool host_dequant_supports(GgmlTensorType type) {
  return type == GgmlTensorType::Q8_0 || type == GgmlTensorType::Q4K || type == GgmlTensorType::Q5K ||
         type == GgmlTensorType::Q6K;
}

Result<void> dequantize_host(GgmlTensorType type, const uint8_t *src, size_t src_len, size_t n, float *out) {
  if (!host_dequant_supports(type))
    return OcelotlError::unsupported("host_dequantize", std::to_string((uint32_t)type), {"Q8_0", "Q4K", "Q5K", "Q6K"});
  auto info = block_info(type);
  if (info.is_err()) return info.error();
  const size_t elems = (size_t)info.value().first, bytes = (size_t)info.value().second;
  if (n % elems != 0)
    return OcelotlError::kernel("cpu", "dequantize: " + std::to_string(n) + " elements is not a whole number of " +
                                           std::to_string(elems) + "-element blocks");
  const size_t blocks = n / elems;
  if (src_len < blocks * bytes)
    return OcelotlError::kernel("cpu", "dequantize: " + std::to_string(src_len) + " bytes hold fewer than " +
                                           std::to_string(blocks) + " blocks of " + std::to_string(bytes));
  if (n > 0 && (src == nullptr || out == nullptr)) return OcelotlError::kernel("cpu", "dequantize: null pointer");
  for (size_t i = 0; i < blocks; ++i) {
    const uint8_t *b = src + i * bytes;
    float *y = out + i * elems;
    switch (type) {
    case GgmlTensorType::Q8_0: block_q8_0(b, y); break;
    case GgmlTensorType::Q4K: block_q4_k(b, y); break;
    case GgmlTensorType::Q5K: block_q5_k(b, y); break;
    default: block_q6_k(b, y); break;
    }
  }
  return {};
}

}  // namespace ocelotl
