// kernel_backend.hpp -- C++ host-side mirror of Ocelotl's kernel dispatch
// boundary for the k-quant linear path, layered on the C-ABI of libokq.so.
//
// The reference is Rust: the trait KernelBackend (crates/kernels/src/lib.rs:
// 84-495), the f32 DeviceTensor (crates/kernels/src/tensor.rs:45-268) and the
// error types OcelotlError / KernelError / UnsupportedError
// (crates/core/src/lib.rs:15-99).  This header restates the part of that
// surface the quantized linear needs, with the same names, argument order and
// error behaviour, in C++17:
//   * Result<T> stands for ocelotl_core::Result<T>: a value or an
//     OcelotlError, never an exception;
//   * slices (&[f32]) are (pointer, length) pairs and are length-checked
//     before anything is launched, like validate_linear_out_by_in
//     (lib.rs:2443-2497);
//   * the quantized weight takes the place of the f32 weight_out_by_in
//     (lib.rs:106-116) as raw GGUF blocks of shape [ne0 = in, ne1 = out].
// Only functions of okq.h are used: device memory comes from okq_alloc, work
// is queued on the backend's stream (a hipStream_t passed as void*).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <variant>
#include <vector>

namespace ocelotl {

// ---- errors (crates/core/src/lib.rs) -------------------------------------

// KernelError{backend, message} (core lib.rs:63-66).
struct KernelError {
  std::string backend;
  std::string message;
};

// UnsupportedError{feature, requested, supported} (core lib.rs:47-51).
struct UnsupportedError {
  std::string feature;
  std::optional<std::string> requested;
  std::vector<std::string> supported;
};

// InvalidModelError{path, field, message} (core lib.rs:37-46): a malformed
// model artifact (the GGUF loader's errors).
struct InvalidModelError {
  std::optional<std::string> path;
  std::optional<std::string> field;
  std::string message;
};

// IoError{path, source} (core lib.rs:87-93); `code` is the errno of the
// failed call and `message` its strerror text.
struct IoError {
  std::optional<std::string> path;
  int code;
  std::string message;
};

// The OcelotlError variants this path produces (core lib.rs:15-31).
class OcelotlError {
 public:
  enum class Kind { Kernel, Unsupported, InvalidModel, Io };

  static OcelotlError kernel(std::string backend, std::string message);
  static OcelotlError unsupported(std::string feature, std::optional<std::string> requested,
                                  std::vector<std::string> supported);
  static OcelotlError invalid_model(std::optional<std::string> path, std::optional<std::string> field,
                                    std::string message);
  static OcelotlError io(std::optional<std::string> path, int code);

  Kind kind() const { return static_cast<Kind>(v_.index()); }
  const KernelError *as_kernel() const { return std::get_if<KernelError>(&v_); }
  const UnsupportedError *as_unsupported() const { return std::get_if<UnsupportedError>(&v_); }
  const InvalidModelError *as_invalid_model() const { return std::get_if<InvalidModelError>(&v_); }
  const IoError *as_io() const { return std::get_if<IoError>(&v_); }
  // Display text in the reference's format ("kernel error on backend `b`: m").
  std::string to_string() const;

 private:
  using V = std::variant<KernelError, UnsupportedError, InvalidModelError, IoError>;
  explicit OcelotlError(V v) : v_(std::move(v)) {}
  V v_;
};

// ocelotl_core::Result<T>.
template <class T>
class [[nodiscard]] Result {
 public:
  Result(T value) : v_(std::move(value)) {}                  // NOLINT: Ok(value)
  Result(OcelotlError error) : v_(std::move(error)) {}       // NOLINT: Err(error)
  bool is_ok() const { return v_.index() == 0; }
  bool is_err() const { return v_.index() == 1; }
  T &value() { return std::get<0>(v_); }
  const T &value() const { return std::get<0>(v_); }
  const OcelotlError &error() const { return std::get<1>(v_); }

 private:
  std::variant<T, OcelotlError> v_;
};

template <>
class [[nodiscard]] Result<void> {
 public:
  Result() = default;                                        // Ok(())
  Result(OcelotlError error) : e_(std::move(error)) {}       // NOLINT: Err(error)
  bool is_ok() const { return !e_.has_value(); }
  bool is_err() const { return e_.has_value(); }
  const OcelotlError &error() const { return *e_; }

 private:
  std::optional<OcelotlError> e_;
};

// ---- device, types ---------------------------------------------------------

// Device::Cpu | Device::Gpu{ordinal} (core lib.rs:438-441).
struct Device {
  enum class Kind { Cpu, Gpu } kind;
  int ordinal;
  static Device gpu(int ordinal) { return Device{Kind::Gpu, ordinal}; }
};

struct KernelContext {
  Device device;
};

// Raw GGML tensor type ids (crates/loader/src/gguf_inspect.rs:170-206): the
// block formats this path dequantizes and gathers (the linear kernels execute
// Q8_0, Q4K, Q5K and Q6K) plus the unquantized float types.
enum class GgmlTensorType : uint32_t {
  F32 = 0,
  F16 = 1,
  Q4_0 = 2,
  Q4_1 = 3,
  Q5_0 = 6,
  Q5_1 = 7,
  Q8_0 = 8,
  Q2K = 10,
  Q3K = 11,
  Q4K = 12,
  Q5K = 13,
  Q6K = 14,
  BF16 = 30
};

// (elements, bytes) per block: the byte_len that GgmlTensorType::
// fixed_element_size leaves as None for quantized types (gguf_inspect.rs:208-219).
Result<std::pair<int64_t, int64_t>> block_info(GgmlTensorType type);
// Byte length of a GGUF tensor from its ne-order shape (gguf_inspect.rs:331-342).
Result<uint64_t> tensor_byte_len(GgmlTensorType type, const std::vector<int64_t> &shape_ne);

// ---- buffers (crates/kernels/src/tensor.rs) --------------------------------

struct DeviceAllocation;  // okq_alloc'd bytes, freed with the last owner

// Where a tensor's data lives (tensor.rs:272-275): on the host, or on the
// device of the backend named by `backend`.
struct Residency {
  enum class Kind { Host, Device } kind;
  const char *backend;  // "hip-gfx950" for Device, null for Host
};

// The f32 tensor handle of tensor.rs:45-268 with its three variants:
//   Host   -- a host vector behind a mutex (from_host, host_zeros);
//   Device -- a buffer of this backend (HipKernelBackend::alloc / upload);
//   View   -- a read-only (source, offset, len) range of another tensor,
//             which must not itself be a view.
// Copies share the backing, as DeviceTensor's Arc does; mutation goes through
// `const` methods (the reference's interior mutability).
class DeviceTensor {
 public:
  // tensor.rs:89-101
  static DeviceTensor from_host(std::vector<float> v);
  static DeviceTensor host_zeros(size_t len);
  // tensor.rs:106-129: range and nesting are checked
  static Result<DeviceTensor> view(const DeviceTensor &source, size_t offset, size_t len);

  size_t len() const { return len_; }
  bool is_empty() const { return len_ == 0; }
  Residency residency() const;  // a view reports its source's
  bool is_view() const { return source_ != nullptr; }
  // The device buffer of a Device tensor (null for Host and View tensors).
  float *device_ptr() const;
  // tensor.rs:204-222: Host copies, Device reads back, View copies its range.
  Result<std::vector<float>> to_host_owned() const;
  // tensor.rs:224-245: length-checked; views are read-only.
  Result<void> write_from_host_slice(const float *src, size_t len) const;

 private:
  friend class HipKernelBackend;
  struct HostStore;
  DeviceTensor(std::shared_ptr<DeviceAllocation> buf, size_t len, void *stream)
      : buf_(std::move(buf)), len_(len), stream_(stream) {}
  DeviceTensor() = default;
  std::shared_ptr<HostStore> host_;                 // Host
  std::shared_ptr<DeviceAllocation> buf_;           // Device
  std::shared_ptr<const DeviceTensor> source_;      // View
  size_t offset_ = 0;                               // View
  size_t len_ = 0;
  void *stream_ = nullptr;                          // Device
};

// A GGUF weight tensor in its file layout: [ne0 = in_features, ne1 =
// out_features], rows of consecutive blocks (gguf_inspect.rs:118-130).
// Device-resident (HipKernelBackend::upload_quantized) or host-resident
// (from_host: blocks as read from a file, for a backend without a device or
// the trait defaults below).
class QuantizedWeight {
 public:
  // Host blocks; the byte length is checked against the shape.
  static Result<QuantizedWeight> from_host(GgmlTensorType type, size_t ne0, size_t ne1, std::vector<uint8_t> blocks);

  GgmlTensorType tensor_type() const { return type_; }
  size_t ne0() const { return ne0_; }
  size_t ne1() const { return ne1_; }
  size_t in_features() const { return ne0_; }
  size_t out_features() const { return ne1_; }
  uint64_t byte_len() const { return bytes_; }
  Residency residency() const;
  // The device blocks (null for a host weight).
  const void *device_ptr() const;
  // The blocks in host memory: a host weight's own bytes, or a device
  // weight's read back.
  Result<std::vector<uint8_t>> to_host_bytes() const;

 private:
  friend class HipKernelBackend;
  QuantizedWeight(GgmlTensorType t, size_t ne0, size_t ne1, uint64_t bytes, std::shared_ptr<DeviceAllocation> buf)
      : type_(t), ne0_(ne0), ne1_(ne1), bytes_(bytes), buf_(std::move(buf)) {}
  GgmlTensorType type_;
  size_t ne0_, ne1_;
  uint64_t bytes_;
  std::shared_ptr<DeviceAllocation> buf_;              // device
  std::shared_ptr<const std::vector<uint8_t>> host_;  // host
};

// ---- the backend (crates/kernels/src/lib.rs:84-495) ------------------------

// The slice of KernelBackend the quantized linear touches.  A backend
// implements the f32 linear_out_by_in (lib.rs:106-116, required as in the
// reference); the quantized entry points have defaults in the reference's
// style (lib.rs:186-217: correct on any backend, slow), which a backend with
// a native path overrides:
//   * dequantize: the host decoders (dequant_host.hpp, bit-exact);
//   * linear_out_by_in with a QuantizedWeight: the weight's blocks on the
//     host, dequantize, then the f32 linear_out_by_in;
//   * linear_d: the host bounce -- read x and bias back, linear_out_by_in on
//     the slices, write out.
class KernelBackend {
 public:
  virtual ~KernelBackend() = default;
  virtual const char *name() const = 0;
  virtual const KernelContext &context() const = 0;
  // lib.rs:171-181
  virtual Result<DeviceTensor> upload(const float *host, size_t len) const = 0;
  virtual Result<DeviceTensor> alloc(size_t len) const = 0;
  // linear_out_by_in over host slices with f32 weights W[out, in]
  // (lib.rs:106-116): out[r, o] = bias[o] + sum_k x[r, k] * W[o, k].  `bias`
  // may be null (bias_len 0).
  virtual Result<void> linear_out_by_in(const float *x, size_t x_len, size_t rows, size_t in_features,
                                        const float *weight, size_t weight_len, size_t out_features,
                                        const float *bias, size_t bias_len, float *out, size_t out_len) const = 0;
  // The same contract with a quantized weight.
  virtual Result<void> linear_out_by_in(const float *x, size_t x_len, size_t rows, size_t in_features,
                                        const QuantizedWeight &weight, size_t out_features, const float *bias,
                                        size_t bias_len, float *out, size_t out_len) const;
  // n elements of raw GGUF blocks (src_len bytes) decoded into out, host
  // slices (no reference counterpart: the reference has no dequantization;
  // the signature follows its slice style).
  virtual Result<void> dequantize(GgmlTensorType type, const uint8_t *src, size_t src_len, size_t n,
                                  float *out) const;
  // linear_d (lib.rs:186-217); `out` is caller-supplied and written in place.
  virtual Result<void> linear_d(const DeviceTensor &x, size_t rows, size_t in_features, const QuantizedWeight &weight,
                                size_t out_features, const DeviceTensor *bias, const DeviceTensor &out) const;
};

// The gfx950 backend: name() == "hip-gfx950" (the backend_id convention of
// crates/kernels/src/cubecl_backend.rs:2268-2272).
class HipKernelBackend final : public KernelBackend {
 public:
  // okq_init(ordinal); a missing or non-gfx950 device is
  // Unsupported{feature: "gpu_backend"} (require_gpu, lib.rs:1662-1671).
  static Result<HipKernelBackend> create(int ordinal);

  const char *name() const override;
  const KernelContext &context() const override { return ctx_; }
  Result<DeviceTensor> upload(const float *host, size_t len) const override;
  Result<DeviceTensor> alloc(size_t len) const override;
  // f32 weights are not offloaded by this backend: Unsupported{feature:
  // "f32_linear_out_by_in"} (the path it serves is the quantized one).
  Result<void> linear_out_by_in(const float *x, size_t x_len, size_t rows, size_t in_features, const float *weight,
                                size_t weight_len, size_t out_features, const float *bias, size_t bias_len, float *out,
                                size_t out_len) const override;
  // Quantized weights on the GPU (a host-resident weight is uploaded first).
  Result<void> linear_out_by_in(const float *x, size_t x_len, size_t rows, size_t in_features,
                                const QuantizedWeight &weight, size_t out_features, const float *bias, size_t bias_len,
                                float *out, size_t out_len) const override;
  // Device-resident x, bias and out run on the device directly; any other
  // residency (host tensors, views) takes the trait default's bounce.
  Result<void> linear_d(const DeviceTensor &x, size_t rows, size_t in_features, const QuantizedWeight &weight,
                        size_t out_features, const DeviceTensor *bias, const DeviceTensor &out) const override;
  // Host slices decoded on the GPU (okq_dequantize; every block format).
  Result<void> dequantize(GgmlTensorType type, const uint8_t *src, size_t src_len, size_t n,
                          float *out) const override;

  // Uploads raw GGUF blocks after checking their byte length against the
  // shape; any block format is accepted (Unsupported otherwise).  linear_d
  // takes Q8_0 / Q4K / Q5K / Q6K weights, dequantize and embedding_rows all of them.
  Result<QuantizedWeight> upload_quantized(GgmlTensorType type, size_t ne0, size_t ne1, const uint8_t *blocks,
                                           size_t len) const;
  // The weight dequantized to f32 on the device (bit-exact with the CPU
  // definition).
  Result<DeviceTensor> dequantize(const QuantizedWeight &weight) const;

  // KernelBackend::rmsnorm over host slices (lib.rs:139-147,
  // rmsnorm.rs:73-128), and the same on device tensors.
  Result<void> rmsnorm(const float *x, size_t x_len, size_t rows, size_t hidden, const float *weight,
                       size_t weight_len, float epsilon, float *out, size_t out_len) const;
  Result<void> rmsnorm_d(const DeviceTensor &x, size_t rows, size_t hidden, const DeviceTensor &weight,
                         float epsilon, const DeviceTensor &out) const;
  // KernelBackend::mlp_gated_silu (lib.rs:150-162, mlp.rs:139-250) with GGUF
  // weights on device tensors: out = down(silu(gate(x)) * up(x)).  gate and
  // up are [ne0 = hidden, ne1 = intermediate], down is [intermediate, hidden]
  // (rows are output features).  gate_buf / up_buf are [rows, intermediate]
  // scratch.
  Result<void> mlp_gated_silu_q(const DeviceTensor &x, size_t rows, size_t hidden, size_t intermediate,
                                const QuantizedWeight &gate, const QuantizedWeight &up, const QuantizedWeight &down,
                                const DeviceTensor &gate_buf, const DeviceTensor &up_buf,
                                const DeviceTensor &out) const;
  // Token embedding lookup from a quantized [hidden, vocab] table: row ids[j]
  // dequantized into row j of the result (the f32 row copy of
  // qwen2_5/prefill.rs:95-105 for a GGUF table).
  Result<DeviceTensor> embedding_rows(const QuantizedWeight &table, const uint32_t *ids, size_t n) const;
  // Waits for the backend's stream.
  Result<void> synchronize() const;

  // Work is queued on this hipStream_t (null = the null stream).
  void set_stream(void *stream) { stream_ = stream; }
  void *stream() const { return stream_; }

 private:
  explicit HipKernelBackend(int ordinal) : ctx_{Device::gpu(ordinal)} {}
  KernelContext ctx_;
  void *stream_ = nullptr;
};

}  // namespace ocelotl
