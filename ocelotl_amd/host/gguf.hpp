// gguf.hpp -- GGUF v3 manifest inspection and tensor payload loading for the
// k-quant path, in C++17 over the HIP kernel backend.
//
// Mirrors inspect_gguf (crates/loader/src/gguf_inspect.rs:224-414): the same
// header walk, limits, alignment rule (general.alignment, default 32, a
// positive multiple of 8), offset checks and error kinds (InvalidModel for a
// malformed file, Io for a failed read, Unsupported for a version other than
// 3).  Two things are added that the reference leaves for a later stage:
//   * byte_len for the block-quantized types this path executes (Q8_0, Q4_K,
//     Q6_K), where fixed_element_size (:208-219) returns None, so their byte
//     ranges are checked against the file length like the unquantized ones;
//   * reading a tensor's payload at file_offset and uploading its raw blocks
//     as a QuantizedWeight (no conversion: the kernels read the file layout).
#pragma once

#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "kernel_backend.hpp"

namespace ocelotl {

// GGUF metadata value types (gguf_inspect.rs:84-115).
enum class GgufMetadataType : uint32_t {
  U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, Bool = 7, String = 8, Array = 9, U64 = 10,
  I64 = 11, F64 = 12
};

// A metadata value.  Integers are held in `u` (unsigned types, Bool) or `i`
// (signed types), floats in `f`, strings in `s`; arrays keep only their
// element type and length, as the reference does.
struct GgufMetadataValue {
  GgufMetadataType type = GgufMetadataType::U8;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0.0;
  std::string s;
  GgufMetadataType element_type = GgufMetadataType::U8;
  uint64_t len = 0;
};

struct GgufMetadataEntry {
  std::string key;
  GgufMetadataValue value;
};

// GgufTensorEntry (gguf_inspect.rs:118-130); `tensor_type` is the raw GGML id.
struct GgufTensorEntry {
  std::string name;
  std::vector<uint64_t> shape;  // ne order: shape[0] is the row length
  uint32_t tensor_type = 0;
  uint64_t offset = 0;       // relative to the tensor-data section
  uint64_t file_offset = 0;  // absolute
  std::optional<uint64_t> byte_len;
};

struct GgufManifest {
  uint32_t version = 0;
  std::vector<GgufMetadataEntry> metadata;
  std::vector<GgufTensorEntry> tensors;
  uint64_t alignment = 0;
  uint64_t data_start = 0;
  uint64_t file_len = 0;

  const GgufMetadataValue *metadata_value(const std::string &key) const;
  const GgufTensorEntry *tensor(const std::string &name) const;
};

// Byte length of a tensor of raw type `type` and ne-order `shape`: element
// size times count for the fixed-size types of fixed_element_size, whole
// blocks for Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K and Q6_K,
// nullopt for the other block formats (Q8_1, Q8_K, IQ*, TQ*, MXFP4).  A
// quantized row that is not a whole number of blocks is an error string.
struct ByteLen {
  std::optional<uint64_t> bytes;
  std::string error;  // non-empty: malformed shape or overflow
};
ByteLen gguf_byte_len(uint32_t type, const std::vector<uint64_t> &shape);

// Parse the header of the GGUF file at `path` (no payload read).
Result<GgufManifest> inspect_gguf(const std::string &path);

// The payload bytes of `entry` (its byte_len must be known).
Result<std::vector<uint8_t>> read_tensor_bytes(const std::string &path, const GgufManifest &manifest,
                                               const GgufTensorEntry &entry);

// Read tensor `name` and upload its blocks as a QuantizedWeight of shape
// [ne0 = shape[0], ne1 = product of the other dims].
Result<QuantizedWeight> load_quantized_weight(const HipKernelBackend &backend, const std::string &path,
                                              const GgufManifest &manifest, const std::string &name);

}  // namespace ocelotl
