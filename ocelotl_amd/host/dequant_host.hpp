// dequant_host.hpp -- GGUF block dequantization on the host, for the
// KernelBackend trait's default quantized linear (dequantize, then the f32
// linear_out_by_in every backend has; the shape of the reference's trait
// defaults, crates/kernels/src/lib.rs:186-217).
//
// Bit-exact with the block definitions the GPU kernels implement: every
// product and difference rounded to f32 separately, in the order of the
// formulas below (this file is built without FMA contraction), f16 scales
// widened exactly.
#pragma once

#include <cstddef>
#include <cstdint>

#include "kernel_backend.hpp"

namespace ocelotl {

// The block formats decoded on the host: the four the linear path executes
// (Q8_0, Q4K, Q5K, Q6K).
bool host_dequant_supports(GgmlTensorType type);

// Decodes n elements (a multiple of the format's block) of `src` (src_len
// bytes, at least n's blocks) into out.  Unsupported for other formats, a
// KernelError for a short or misaligned input.
Result<void> dequantize_host(GgmlTensorType type, const uint8_t *src, size_t src_len, size_t n, float *out);

// Exact IEEE half -> f32 (subnormals, infinities and NaNs included; the
// decode of crates/loader/src/safetensors_values.rs:155-183).
float half_to_f32(uint16_t bits);

}  // namespace ocelotl
