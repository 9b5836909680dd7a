// kernel_backend.cpp -- the C++ mirror of the kernel boundary over libokq.so.
// Validation order and messages follow validate_linear_out_by_in
// (crates/kernels/src/lib.rs:2443-2497); every check happens before a launch.
#include "kernel_backend.hpp"

#include <cstdint>
#include <optional>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>

#include "dequant_host.hpp"
#include "okq.h"

namespace ocelotl {

namespace {

constexpr const char *kBackend = "hip-gfx950";

const std::vector<std::string> &quantized_names() {
  static const std::vector<std::string> v = {"Q8_0", "Q4K", "Q5K", "Q6K"};
  return v;
}

const std::vector<std::string> &block_format_names() {
  static const std::vector<std::string> v = {"Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0",
                                             "Q2K",  "Q3K",  "Q4K",  "Q5K",  "Q6K"};
  return v;
}

bool is_block_format(GgmlTensorType t) {
  switch (t) {
  case GgmlTensorType::Q4_0: case GgmlTensorType::Q4_1: case GgmlTensorType::Q5_0: case GgmlTensorType::Q5_1:
  case GgmlTensorType::Q8_0: case GgmlTensorType::Q2K: case GgmlTensorType::Q3K: case GgmlTensorType::Q4K:
  case GgmlTensorType::Q5K: case GgmlTensorType::Q6K: return true;
  default: return false;
  }
}

std::string last_error() {
  char buf[512];
  const size_t n = okq_last_error(buf, sizeof buf);
  (void)n;
  return std::string(buf);
}

// okq_status -> the reference's error kinds: OKQ_E_TYPE is a type this path
// does not execute (Unsupported), OKQ_E_NODEV is the require_gpu error
// (lib.rs:1662-1671), everything else is a KernelError with the library's
// message.
OcelotlError status_error(okq_status st, std::optional<uint32_t> type_id) {
  if (st == OKQ_E_TYPE) {
    std::optional<std::string> req;
    if (type_id) req = std::to_string(*type_id);
    return OcelotlError::unsupported("quantized_tensor_type", req, quantized_names());
  }
  if (st == OKQ_E_NODEV) return OcelotlError::unsupported("gpu_backend", std::string("gfx950"), {});
  return OcelotlError::kernel(kBackend, last_error());
}

Result<void> check(okq_status st, std::optional<uint32_t> type_id = std::nullopt) {
  if (st == OKQ_OK) return {};
  return status_error(st, type_id);
}

OcelotlError kernel_err(const std::string &message) { return OcelotlError::kernel(kBackend, message); }

std::string len_mismatch(const char *what, size_t got, const char *expr, size_t a, size_t b) {
  char buf[256];
  std::snprintf(buf, sizeof buf, "linear_out_by_in %s=%zu does not match %s=%zu*%zu=%zu", what, got, expr, a, b,
                a * b);
  return buf;
}

}  // namespace

// ---- errors ------------------------------------------------------------------

OcelotlError OcelotlError::kernel(std::string backend, std::string message) {
  return OcelotlError(KernelError{std::move(backend), std::move(message)});
}

OcelotlError OcelotlError::unsupported(std::string feature, std::optional<std::string> requested,
                                       std::vector<std::string> supported) {
  return OcelotlError(UnsupportedError{std::move(feature), std::move(requested), std::move(supported)});
}

OcelotlError OcelotlError::invalid_model(std::optional<std::string> path, std::optional<std::string> field,
                                         std::string message) {
  return OcelotlError(InvalidModelError{std::move(path), std::move(field), std::move(message)});
}

OcelotlError OcelotlError::io(std::optional<std::string> path, int code) {
  return OcelotlError(IoError{std::move(path), code, std::strerror(code)});
}

std::string OcelotlError::to_string() const {
  if (const KernelError *k = as_kernel()) return "kernel error on backend `" + k->backend + "`: " + k->message;
  if (const InvalidModelError *m = as_invalid_model()) {
    std::string s = "invalid model artifact";
    if (m->path) s += " at `" + *m->path + "`";
    if (m->field) s += " (field `" + *m->field + "`)";
    return s + ": " + m->message;
  }
  if (const IoError *e = as_io()) return "IO error" + (e->path ? " on `" + *e->path + "`" : std::string()) + ": " + e->message;
  const UnsupportedError *u = as_unsupported();
  std::string s = "unsupported feature `" + u->feature + "`";
  if (u->requested) s += " (requested `" + *u->requested + "`)";
  s += ": supported = [";
  for (size_t i = 0; i < u->supported.size(); ++i) s += (i ? ", " : "") + u->supported[i];
  return s + "]";
}

// ---- layout --------------------------------------------------------------------

Result<std::pair<int64_t, int64_t>> block_info(GgmlTensorType type) {
  int64_t e = 0, b = 0;
  const okq_status st = okq_type_info((uint32_t)type, &e, &b);
  if (st != OKQ_OK) return status_error(st, (uint32_t)type);
  return std::make_pair(e, b);
}

Result<uint64_t> tensor_byte_len(GgmlTensorType type, const std::vector<int64_t> &shape_ne) {
  uint64_t out = 0;
  const okq_status st = okq_tensor_bytes((uint32_t)type, shape_ne.data(), (int)shape_ne.size(), &out);
  if (st != OKQ_OK) return status_error(st, (uint32_t)type);
  return out;
}

// ---- buffers -------------------------------------------------------------------

struct DeviceAllocation {
  void *ptr = nullptr;
  ~DeviceAllocation() {
    if (ptr) (void)okq_free(ptr);
  }
};

namespace {
Result<std::shared_ptr<DeviceAllocation>> device_alloc(size_t bytes) {
  auto a = std::make_shared<DeviceAllocation>();
  if (bytes > 0) {
    const okq_status st = okq_alloc(&a->ptr, bytes);
    if (st != OKQ_OK) return status_error(st, std::nullopt);
  }
  return a;
}
}  // namespace

struct DeviceTensor::HostStore {
  std::mutex mu;
  std::vector<float> v;
};

namespace {
// The reference's tensor errors carry backend "tensor" (tensor.rs:319-324).
OcelotlError tensor_err(const std::string &message) { return OcelotlError::kernel("tensor", message); }
}  // namespace

DeviceTensor DeviceTensor::from_host(std::vector<float> v) {
  DeviceTensor t;
  t.host_ = std::make_shared<HostStore>();
  t.len_ = v.size();
  t.host_->v = std::move(v);
  return t;
}

DeviceTensor DeviceTensor::host_zeros(size_t len) { return from_host(std::vector<float>(len, 0.0f)); }

Result<DeviceTensor> DeviceTensor::view(const DeviceTensor &source, size_t offset, size_t len) {
  const size_t src_len = source.len();
  if (offset > SIZE_MAX - len || offset + len > src_len) {
    const size_t end = offset > SIZE_MAX - len ? SIZE_MAX : offset + len;
    return tensor_err("DeviceTensor::view range " + std::to_string(offset) + ".." + std::to_string(end) +
                      " exceeds source length " + std::to_string(src_len));
  }
  if (source.is_view()) return tensor_err("DeviceTensor::view does not nest; resolve the source view first");
  DeviceTensor t;
  t.source_ = std::make_shared<const DeviceTensor>(source);
  t.offset_ = offset;
  t.len_ = len;
  return t;
}

Residency DeviceTensor::residency() const {
  if (source_) return source_->residency();
  if (buf_) return Residency{Residency::Kind::Device, kBackend};
  return Residency{Residency::Kind::Host, nullptr};
}

float *DeviceTensor::device_ptr() const { return buf_ ? static_cast<float *>(buf_->ptr) : nullptr; }

Result<std::vector<float>> DeviceTensor::to_host_owned() const {
  if (host_) {
    std::lock_guard<std::mutex> lock(host_->mu);
    return host_->v;
  }
  if (source_) {
    auto parent = source_->to_host_owned();
    if (parent.is_err()) return parent.error();
    return std::vector<float>(parent.value().begin() + (ptrdiff_t)offset_,
                              parent.value().begin() + (ptrdiff_t)(offset_ + len_));
  }
  std::vector<float> v(len_);
  if (len_ == 0) return v;
  Result<void> r = check(okq_memcpy_d2h(v.data(), buf_->ptr, len_ * sizeof(float), stream_));
  if (r.is_err()) return r.error();
  r = check(okq_sync(stream_));
  if (r.is_err()) return r.error();
  return v;
}

Result<void> DeviceTensor::write_from_host_slice(const float *src, size_t len) const {
  if (len != len_) {
    return tensor_err("DeviceTensor::write_from_host_slice: src.len()=" + std::to_string(len) + " != tensor len " +
                      std::to_string(len_));
  }
  if (source_) return tensor_err("DeviceTensor::write_from_host_slice: views are read-only");
  if (host_) {
    std::lock_guard<std::mutex> lock(host_->mu);
    if (len) std::memcpy(host_->v.data(), src, len * sizeof(float));
    return {};
  }
  if (len == 0) return {};
  Result<void> r = check(okq_memcpy_h2d(buf_->ptr, src, len * sizeof(float), stream_));
  if (r.is_err()) return r;
  return check(okq_sync(stream_));  // the host slice may be reused on return
}

Result<QuantizedWeight> QuantizedWeight::from_host(GgmlTensorType type, size_t ne0, size_t ne1,
                                                   std::vector<uint8_t> blocks) {
  auto want = tensor_byte_len(type, {(int64_t)ne0, (int64_t)ne1});
  if (want.is_err()) return want.error();
  if (blocks.size() != want.value()) {
    return kernel_err("quantized weight has " + std::to_string(blocks.size()) + " bytes, shape [" +
                      std::to_string(ne0) + ", " + std::to_string(ne1) + "] needs " + std::to_string(want.value()));
  }
  QuantizedWeight w(type, ne0, ne1, blocks.size(), nullptr);
  w.host_ = std::make_shared<const std::vector<uint8_t>>(std::move(blocks));
  return w;
}

Residency QuantizedWeight::residency() const {
  if (host_) return Residency{Residency::Kind::Host, nullptr};
  return Residency{Residency::Kind::Device, kBackend};
}

const void *QuantizedWeight::device_ptr() const { return buf_ ? buf_->ptr : nullptr; }

Result<std::vector<uint8_t>> QuantizedWeight::to_host_bytes() const {
  if (host_) return *host_;
  std::vector<uint8_t> v((size_t)bytes_);
  if (v.empty()) return v;
  Result<void> r = check(okq_memcpy_d2h(v.data(), buf_->ptr, v.size(), nullptr));
  if (r.is_err()) return r.error();
  r = check(okq_sync(nullptr));
  if (r.is_err()) return r.error();
  return v;
}

// ---- trait defaults ------------------------------------------------------------

namespace {
// The checks of validate_linear_out_by_in (lib.rs:2443-2497) for a quantized
// weight, in order: weight shape against the features, then x, bias and out
// lengths.
Result<void> validate_quantized_linear(const char *backend, size_t x_len, size_t rows, size_t in_features,
                                       const QuantizedWeight &weight, size_t out_features, bool has_bias,
                                       size_t bias_len, size_t out_len) {
  auto err = [&](const std::string &m) { return OcelotlError::kernel(backend, m); };
  if (weight.ne0() != in_features || weight.ne1() != out_features) {
    return err("linear_out_by_in weight shape [" + std::to_string(weight.ne0()) + ", " + std::to_string(weight.ne1()) +
               "] does not match in_features=" + std::to_string(in_features) +
               " out_features=" + std::to_string(out_features));
  }
  if (rows != 0 && in_features > SIZE_MAX / rows) return err("linear_out_by_in rows*in_features overflows");
  if (x_len != rows * in_features) return err(len_mismatch("x.len()", x_len, "rows*in_features", rows, in_features));
  if (has_bias && bias_len != out_features) {
    return err("linear_out_by_in bias.len()=" + std::to_string(bias_len) +
               " does not match out_features=" + std::to_string(out_features));
  }
  if (rows != 0 && out_features > SIZE_MAX / rows) return err("linear_out_by_in rows*out_features overflows");
  if (out_len != rows * out_features)
    return err(len_mismatch("out.len()", out_len, "rows*out_features", rows, out_features));
  return {};
}
}  // namespace

Result<void> KernelBackend::dequantize(GgmlTensorType type, const uint8_t *src, size_t src_len, size_t n,
                                       float *out) const {
  return dequantize_host(type, src, src_len, n, out);
}

// The weight's blocks on the host, dequantized, then this backend's f32
// linear_out_by_in.
Result<void> KernelBackend::linear_out_by_in(const float *x, size_t x_len, size_t rows, size_t in_features,
                                             const QuantizedWeight &weight, size_t out_features, const float *bias,
                                             size_t bias_len, float *out, size_t out_len) const {
  Result<void> v = validate_quantized_linear(name(), x_len, rows, in_features, weight, out_features, bias != nullptr,
                                             bias_len, out_len);
  if (v.is_err()) return v;
  auto blocks = weight.to_host_bytes();
  if (blocks.is_err()) return blocks.error();
  const size_t n = in_features * out_features;
  std::vector<float> wf(n);
  Result<void> r = dequantize(weight.tensor_type(), blocks.value().data(), blocks.value().size(), n, wf.data());
  if (r.is_err()) return r;
  return linear_out_by_in(x, x_len, rows, in_features, wf.data(), wf.size(), out_features, bias, bias_len, out,
                          out_len);
}

// lib.rs:193-217: x and bias read back, linear_out_by_in on the slices, out
// written from the host.
Result<void> KernelBackend::linear_d(const DeviceTensor &x, size_t rows, size_t in_features,
                                     const QuantizedWeight &weight, size_t out_features, const DeviceTensor *bias,
                                     const DeviceTensor &out) const {
  auto xh = x.to_host_owned();
  if (xh.is_err()) return xh.error();
  std::vector<float> bh;
  if (bias) {
    auto b = bias->to_host_owned();
    if (b.is_err()) return b.error();
    bh = std::move(b.value());
  }
  std::vector<float> oh(out.len(), 0.0f);
  Result<void> r = linear_out_by_in(xh.value().data(), xh.value().size(), rows, in_features, weight, out_features,
                                    bias ? bh.data() : nullptr, bh.size(), oh.data(), oh.size());
  if (r.is_err()) return r;
  return out.write_from_host_slice(oh.data(), oh.size());
}

// ---- backend -------------------------------------------------------------------

Result<HipKernelBackend> HipKernelBackend::create(int ordinal) {
  Result<void> r = check(okq_init(ordinal));
  if (r.is_err()) return r.error();
  return HipKernelBackend(ordinal);
}

const char *HipKernelBackend::name() const { return okq_backend_name(); }

Result<DeviceTensor> HipKernelBackend::alloc(size_t len) const {
  auto a = device_alloc(len * sizeof(float));
  if (a.is_err()) return a.error();
  DeviceTensor t(a.value(), len, stream_);
  if (len > 0) {  // zero-filled, like the trait's default (lib.rs:177-181)
    const std::vector<float> zeros(len, 0.0f);
    Result<void> r = t.write_from_host_slice(zeros.data(), len);
    if (r.is_err()) return r.error();
  }
  return t;
}

Result<DeviceTensor> HipKernelBackend::upload(const float *host, size_t len) const {
  auto a = device_alloc(len * sizeof(float));
  if (a.is_err()) return a.error();
  DeviceTensor t(a.value(), len, stream_);
  Result<void> r = t.write_from_host_slice(host, len);
  if (r.is_err()) return r.error();
  return t;
}

Result<QuantizedWeight> HipKernelBackend::upload_quantized(GgmlTensorType type, size_t ne0, size_t ne1,
                                                           const uint8_t *blocks, size_t len) const {
  if (!is_block_format(type))
    return OcelotlError::unsupported("quantized_tensor_type", std::to_string((uint32_t)type), block_format_names());
  auto want = tensor_byte_len(type, {(int64_t)ne0, (int64_t)ne1});
  if (want.is_err()) return want.error();
  if (len != want.value()) {
    return kernel_err("quantized weight has " + std::to_string(len) + " bytes, shape [" + std::to_string(ne0) + ", " +
                      std::to_string(ne1) + "] needs " + std::to_string(want.value()));
  }
  auto a = device_alloc(len);
  if (a.is_err()) return a.error();
  if (len > 0) {
    Result<void> r = check(okq_memcpy_h2d(a.value()->ptr, blocks, len, stream_));
    if (r.is_err()) return r.error();
    r = check(okq_sync(stream_));
    if (r.is_err()) return r.error();
  }
  return QuantizedWeight(type, ne0, ne1, len, a.value());
}

Result<void> HipKernelBackend::linear_out_by_in(const float *, size_t, size_t, size_t, const float *, size_t,
                                                size_t, const float *, size_t, float *, size_t) const {
  return OcelotlError::unsupported("f32_linear_out_by_in", std::string(kBackend),
                                   {"quantized weights: Q8_0", "Q4K", "Q5K", "Q6K"});
}

Result<void> HipKernelBackend::dequantize(GgmlTensorType type, const uint8_t *src, size_t src_len, size_t n,
                                          float *out) const {
  if (!is_block_format(type))
    return OcelotlError::unsupported("quantized_tensor_type", std::to_string((uint32_t)type), block_format_names());
  auto info = block_info(type);
  if (info.is_err()) return info.error();
  const size_t elems = (size_t)info.value().first, bytes = (size_t)info.value().second;
  if (n % elems != 0 || src_len < n / elems * bytes) {
    return kernel_err("dequantize: " + std::to_string(n) + " elements need whole " + std::to_string(elems) +
                      "-element blocks within the " + std::to_string(src_len) + " source bytes");
  }
  if (n == 0) return {};
  auto a = device_alloc(n / elems * bytes);
  if (a.is_err()) return a.error();
  auto o = device_alloc(n * sizeof(float));
  if (o.is_err()) return o.error();
  Result<void> r = check(okq_memcpy_h2d(a.value()->ptr, src, n / elems * bytes, stream_));
  if (r.is_err()) return r;
  r = check(okq_dequantize((uint32_t)type, a.value()->ptr, (int64_t)n, static_cast<float *>(o.value()->ptr), stream_),
            (uint32_t)type);
  if (r.is_err()) return r;
  r = check(okq_memcpy_d2h(out, o.value()->ptr, n * sizeof(float), stream_));
  if (r.is_err()) return r;
  return check(okq_sync(stream_));
}

Result<DeviceTensor> HipKernelBackend::dequantize(const QuantizedWeight &weight) const {
  if (weight.device_ptr() == nullptr && weight.byte_len() > 0) {
    auto blocks = weight.to_host_bytes();
    if (blocks.is_err()) return blocks.error();
    auto dw = upload_quantized(weight.tensor_type(), weight.ne0(), weight.ne1(), blocks.value().data(),
                               blocks.value().size());
    if (dw.is_err()) return dw.error();
    return dequantize(dw.value());
  }
  const size_t n = weight.ne0() * weight.ne1();
  auto a = device_alloc(n * sizeof(float));
  if (a.is_err()) return a.error();
  DeviceTensor t(a.value(), n, stream_);
  Result<void> r = check(okq_dequantize((uint32_t)weight.tensor_type(), weight.device_ptr(), (int64_t)n,
                                        t.device_ptr(), stream_),
                         (uint32_t)weight.tensor_type());
  if (r.is_err()) return r.error();
  return t;
}

Result<void> HipKernelBackend::synchronize() const { return check(okq_sync(stream_)); }

// ---- neighbours -------------------------------------------------------------------

Result<void> HipKernelBackend::rmsnorm_d(const DeviceTensor &x, size_t rows, size_t hidden, const DeviceTensor &weight,
                                         float epsilon, const DeviceTensor &out) const {
  // rmsnorm.rs:81-114, in order
  if (hidden == 0) return kernel_err("rmsnorm hidden dimension must be non-zero");
  if (weight.len() != hidden)
    return kernel_err("rmsnorm weight length " + std::to_string(weight.len()) + " does not match hidden " +
                      std::to_string(hidden));
  if (x.len() != rows * hidden)
    return kernel_err("rmsnorm x slice length " + std::to_string(x.len()) + " does not match shape " +
                      std::to_string(rows) + "x" + std::to_string(hidden));
  if (out.len() != x.len())
    return kernel_err("rmsnorm out slice length " + std::to_string(out.len()) + " does not match x length " +
                      std::to_string(x.len()));
  if (!(epsilon >= 0.0f) || epsilon == std::numeric_limits<float>::infinity()) {
    char buf[128];
    std::snprintf(buf, sizeof buf, "rmsnorm epsilon must be finite and non-negative, got %g", (double)epsilon);
    return kernel_err(buf);
  }
  if (rows == 0) return {};
  return check(okq_rmsnorm(x.device_ptr(), (int64_t)rows, (int64_t)hidden, weight.device_ptr(), epsilon,
                           out.device_ptr(), stream_));
}

Result<void> HipKernelBackend::rmsnorm(const float *x, size_t x_len, size_t rows, size_t hidden, const float *weight,
                                       size_t weight_len, float epsilon, float *out, size_t out_len) const {
  auto xd = upload(x, x_len);
  if (xd.is_err()) return xd.error();
  auto wd = upload(weight, weight_len);
  if (wd.is_err()) return wd.error();
  auto od = alloc(out_len);
  if (od.is_err()) return od.error();
  Result<void> r = rmsnorm_d(xd.value(), rows, hidden, wd.value(), epsilon, od.value());
  if (r.is_err()) return r;
  auto host = od.value().to_host_owned();
  if (host.is_err()) return host.error();
  if (out_len) std::memcpy(out, host.value().data(), out_len * sizeof(float));
  return {};
}

Result<void> HipKernelBackend::mlp_gated_silu_q(const DeviceTensor &x, size_t rows, size_t hidden,
                                                size_t intermediate, const QuantizedWeight &gate,
                                                const QuantizedWeight &up, const QuantizedWeight &down,
                                                const DeviceTensor &gate_buf, const DeviceTensor &up_buf,
                                                const DeviceTensor &out) const {
  // mlp.rs:151-227: zero dimensions, then every length against its shape
  if (rows == 0) return kernel_err("mlp_gated_silu seq_len must be non-zero");
  if (hidden == 0) return kernel_err("mlp_gated_silu hidden must be non-zero");
  if (intermediate == 0) return kernel_err("mlp_gated_silu intermediate must be non-zero");
  const std::string hs = std::to_string(hidden), is = std::to_string(intermediate), rs = std::to_string(rows);
  if (x.len() != rows * hidden)
    return kernel_err("mlp_gated_silu x slice length " + std::to_string(x.len()) + " does not match shape " + rs +
                      "x" + hs);
  auto shape_err = [&](const char *name, const QuantizedWeight &w, size_t ne0, size_t ne1) {
    return kernel_err(std::string("mlp_gated_silu ") + name + " shape [" + std::to_string(w.ne0()) + ", " +
                      std::to_string(w.ne1()) + "] does not match [" + std::to_string(ne0) + ", " +
                      std::to_string(ne1) + "]");
  };
  if (gate.ne0() != hidden || gate.ne1() != intermediate) return shape_err("gate_w", gate, hidden, intermediate);
  if (up.ne0() != hidden || up.ne1() != intermediate) return shape_err("up_w", up, hidden, intermediate);
  if (down.ne0() != intermediate || down.ne1() != hidden) return shape_err("down_w", down, intermediate, hidden);
  if (gate_buf.len() != rows * intermediate)
    return kernel_err("mlp_gated_silu gate_buf length " + std::to_string(gate_buf.len()) + " does not match shape " +
                      rs + "x" + is);
  if (up_buf.len() != rows * intermediate)
    return kernel_err("mlp_gated_silu up_buf length " + std::to_string(up_buf.len()) + " does not match shape " +
                      rs + "x" + is);
  if (out.len() != rows * hidden)
    return kernel_err("mlp_gated_silu out length " + std::to_string(out.len()) + " does not match shape " + rs + "x" +
                      hs);
  return check(okq_mlp_gated_silu_q(x.device_ptr(), (int64_t)rows, (int64_t)hidden, (int64_t)intermediate,
                                    (uint32_t)gate.tensor_type(), gate.device_ptr(), gate.byte_len(),
                                    (uint32_t)up.tensor_type(), up.device_ptr(), up.byte_len(),
                                    (uint32_t)down.tensor_type(), down.device_ptr(), down.byte_len(),
                                    gate_buf.device_ptr(), up_buf.device_ptr(), out.device_ptr(), stream_));
}

Result<DeviceTensor> HipKernelBackend::embedding_rows(const QuantizedWeight &table, const uint32_t *ids,
                                                      size_t n) const {
  auto a = device_alloc(n * table.ne0() * sizeof(float));
  if (a.is_err()) return a.error();
  DeviceTensor t(a.value(), n * table.ne0(), stream_);
  Result<void> r = check(okq_get_rows_q((uint32_t)table.tensor_type(), table.device_ptr(), table.byte_len(),
                                        (int64_t)table.ne0(), (int64_t)table.ne1(), ids, (int64_t)n, t.device_ptr(),
                                        stream_),
                         (uint32_t)table.tensor_type());
  if (r.is_err()) return r.error();
  return t;
}

Result<void> HipKernelBackend::linear_d(const DeviceTensor &x, size_t rows, size_t in_features,
                                        const QuantizedWeight &weight, size_t out_features, const DeviceTensor *bias,
                                        const DeviceTensor &out) const {
  if (weight.device_ptr() == nullptr && weight.byte_len() > 0) {
    // a host-resident weight: a device copy for this call
    auto blocks = weight.to_host_bytes();
    if (blocks.is_err()) return blocks.error();
    auto dw = upload_quantized(weight.tensor_type(), weight.ne0(), weight.ne1(), blocks.value().data(),
                               blocks.value().size());
    if (dw.is_err()) return dw.error();
    return linear_d(x, rows, in_features, dw.value(), out_features, bias, out);
  }
  if (weight.ne0() != in_features || weight.ne1() != out_features) {
    return kernel_err("linear_d weight shape [" + std::to_string(weight.ne0()) + ", " + std::to_string(weight.ne1()) +
                      "] does not match in_features=" + std::to_string(in_features) +
                      " out_features=" + std::to_string(out_features));
  }
  if (x.len() != rows * in_features) return kernel_err(len_mismatch("x.len()", x.len(), "rows*in_features", rows, in_features));
  if (bias && bias->len() != out_features) {
    return kernel_err("linear_out_by_in bias.len()=" + std::to_string(bias->len()) +
                      " does not match out_features=" + std::to_string(out_features));
  }
  if (out.len() != rows * out_features)
    return kernel_err(len_mismatch("out.len()", out.len(), "rows*out_features", rows, out_features));
  auto on_device = [](const DeviceTensor &t) { return !t.is_view() && t.device_ptr() != nullptr; };
  if (!on_device(x) || (bias && !on_device(*bias)) || (!on_device(out) && out.len() > 0)) {
    // wrong residency: the trait default's host bounce (lib.rs:193-217, the
    // fallback of cubecl_backend.rs:280-292), slow but correct
    auto xh = x.to_host_owned();
    if (xh.is_err()) return xh.error();
    std::vector<float> bh;
    if (bias) {
      auto b = bias->to_host_owned();
      if (b.is_err()) return b.error();
      bh = std::move(b.value());
    }
    std::vector<float> oh(rows * out_features, 0.0f);
    Result<void> r = linear_out_by_in(xh.value().data(), xh.value().size(), rows, in_features, weight, out_features,
                                      bias ? bh.data() : nullptr, bh.size(), oh.data(), oh.size());
    if (r.is_err()) return r;
    return out.write_from_host_slice(oh.data(), oh.size());
  }
  return check(okq_linear_out_by_in_q(x.device_ptr(), (int64_t)rows, (int64_t)in_features,
                                      (uint32_t)weight.tensor_type(), weight.device_ptr(), weight.byte_len(),
                                      (int64_t)out_features, bias ? bias->device_ptr() : nullptr, out.device_ptr(),
                                      stream_),
               (uint32_t)weight.tensor_type());
}

// Host slices: the trait default's bounce (lib.rs:193-217) -- upload x and
// bias, run on the device, read `out` back.
Result<void> HipKernelBackend::linear_out_by_in(const float *x, size_t x_len, size_t rows, size_t in_features,
                                                const QuantizedWeight &weight, size_t out_features, const float *bias,
                                                size_t bias_len, float *out, size_t out_len) const {
  if (x_len != rows * in_features) return kernel_err(len_mismatch("x.len()", x_len, "rows*in_features", rows, in_features));
  if (bias && bias_len != out_features) {
    return kernel_err("linear_out_by_in bias.len()=" + std::to_string(bias_len) +
                      " does not match out_features=" + std::to_string(out_features));
  }
  if (out_len != rows * out_features)
    return kernel_err(len_mismatch("out.len()", out_len, "rows*out_features", rows, out_features));
  auto xd = upload(x, x_len);
  if (xd.is_err()) return xd.error();
  std::optional<DeviceTensor> bd;
  if (bias) {
    auto b = upload(bias, bias_len);
    if (b.is_err()) return b.error();
    bd = b.value();
  }
  auto od = alloc(out_len);
  if (od.is_err()) return od.error();
  Result<void> r = linear_d(xd.value(), rows, in_features, weight, out_features, bd ? &*bd : nullptr, od.value());
  if (r.is_err()) return r;
  auto host = od.value().to_host_owned();
  if (host.is_err()) return host.error();
  if (out_len) std::memcpy(out, host.value().data(), out_len * sizeof(float));
  return {};
}

}  // namespace ocelotl
