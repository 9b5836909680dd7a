// dequant_policy.cpp -- the quantized-execution gate of dequant_policy.hpp.
#include "dequant_policy.hpp"

#include <algorithm>

namespace ocelotl {

bool is_quantized_tensor_type(uint32_t raw_type) {
  switch (raw_type) {
  case 0:   // F32
  case 1:   // F16
  case 30:  // BF16
  case 24:  // I8
  case 25:  // I16
  case 26:  // I32
  case 27:  // I64
  case 28:  // F64
    return false;
  default:
    return true;
  }
}

std::string ggml_type_name(uint32_t raw_type) {
  static const char *const kNames[] = {
      "F32",    "F16",    "Q4_0",   "Q4_1", "",     "",    "Q5_0",  "Q5_1",  "Q8_0",  "Q8_1",  "Q2K",   "Q3K",
      "Q4K",    "Q5K",    "Q6K",    "Q8K",  "Iq2Xxs", "Iq2Xs", "Iq3Xxs", "Iq1S", "Iq4Nl", "Iq3S", "Iq2S", "Iq4Xs",
      "I8",     "I16",    "I32",    "I64",  "F64",  "Iq1M", "BF16"};
  if (raw_type < sizeof kNames / sizeof kNames[0] && kNames[raw_type][0] != '\0') return kNames[raw_type];
  if (raw_type == 34) return "Tq1_0";
  if (raw_type == 35) return "Tq2_0";
  if (raw_type == 39) return "MXFP4";
  return "Unknown(" + std::to_string(raw_type) + ")";
}

TensorExecution tensor_execution(uint32_t raw_type) {
  if (!is_quantized_tensor_type(raw_type)) return TensorExecution::Float;
  switch (raw_type) {
  case 8:   // Q8_0
  case 12:  // Q4K
  case 13:  // Q5K
  case 14:  // Q6K
    return TensorExecution::QuantizedLinear;
  case 2: case 3: case 6: case 7:  // Q4_0, Q4_1, Q5_0, Q5_1
  case 10: case 11:                // Q2K, Q3K
    return TensorExecution::DequantizeToF32;
  default:
    return TensorExecution::None;
  }
}

bool requires_dequant_policy(const GgufManifest &manifest) {
  return std::any_of(manifest.tensors.begin(), manifest.tensors.end(),
                     [](const GgufTensorEntry &t) { return is_quantized_tensor_type(t.tensor_type); });
}

Result<void> ensure_supported_for_execution(const std::vector<uint32_t> &tensor_types) {
  std::vector<uint32_t> refused;
  for (uint32_t t : tensor_types)
    if (tensor_execution(t) == TensorExecution::None && std::find(refused.begin(), refused.end(), t) == refused.end())
      refused.push_back(t);
  if (refused.empty()) return {};
  std::string requested;
  for (size_t i = 0; i < refused.size(); ++i) requested += (i ? "," : "") + ggml_type_name(refused[i]);
  return OcelotlError::unsupported("quantized_tensor_types", requested,
                                   {"Q8_0", "Q4K", "Q5K", "Q6K", "Q4_0 (dequantized)", "Q4_1 (dequantized)",
                                    "Q5_0 (dequantized)", "Q5_1 (dequantized)", "Q2K (dequantized)",
                                    "Q3K (dequantized)"});
}

Result<void> ensure_supported_for_execution(const GgufManifest &manifest) {
  std::vector<uint32_t> types;
  types.reserve(manifest.tensors.size());
  for (const GgufTensorEntry &t : manifest.tensors) types.push_back(t.tensor_type);
  return ensure_supported_for_execution(types);
}

}  // namespace ocelotl
