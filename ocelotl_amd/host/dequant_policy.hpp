// dequant_policy.hpp -- the execution gate for quantized GGUF tensors, with
// this backend's dequant policy in place.
//
// The reference refuses every quantized model before any compute:
// Gemma4Config::requires_dequant_policy (crates/models/src/gemma/gemma4.rs:
// 59-64) holds for a quantized file type or any quantized tensor
// (is_quantized_tensor_type, :299-311), and ensure_supported_for_execution
// (:66-92) then returns Unsupported{feature: "gemma4.execution_features",
// requested: "...,quantization=q4_k_m", supported: ["none for Gemma4
// execution yet"]}.  That check is the hook a dequant policy flips.  With
// the hip-gfx950 backend a quantized tensor is executable when its type has
// an execution here; the gate refuses only the types that have none, with
// the same error kind.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "gguf.hpp"
#include "kernel_backend.hpp"

namespace ocelotl {

// gemma4.rs:299-311: every GGML type except the plain numeric ones (F32, F16,
// BF16, I8, I16, I32, I64, F64) is quantized, unknown ids included.
bool is_quantized_tensor_type(uint32_t raw_type);

// The reference's Debug name of a raw GGML type id (gguf_inspect.rs:132-206),
// "Unknown(<id>)" for ids it does not name.
std::string ggml_type_name(uint32_t raw_type);

// How this backend executes a tensor of a GGML type:
//   Float           -- not quantized: the reference's own f32 path
//   QuantizedLinear -- Q8_0, Q4K, Q5K, Q6K: linear_d / linear_out_by_in on the GGUF
//                      blocks (decode GEMV, MFMA GEMM), dequantize and
//                      embedding_rows
//   DequantizeToF32 -- Q4_0, Q4_1, Q5_0, Q5_1, Q2K, Q3K: dequantize /
//                      embedding_rows on the GPU, then the f32 path
//   None            -- every other block format (Q8_1, Q8K, the IQ and TQ
//                      formats, MXFP4, unknown ids)
enum class TensorExecution { Float, QuantizedLinear, DequantizeToF32, None };
TensorExecution tensor_execution(uint32_t raw_type);

// requires_dequant_policy for a file (gemma4.rs:59-64): some tensor is
// quantized.
bool requires_dequant_policy(const GgufManifest &manifest);

// The gate with the policy in place: Ok when every quantized tensor type has
// an execution, else Unsupported{feature: "quantized_tensor_types",
// requested: the refused types' names joined with "," (in first-seen order),
// supported: the executable block formats}.
Result<void> ensure_supported_for_execution(const std::vector<uint32_t> &tensor_types);
Result<void> ensure_supported_for_execution(const GgufManifest &manifest);

}  // namespace ocelotl
