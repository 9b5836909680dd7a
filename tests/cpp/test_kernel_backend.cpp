// test_kernel_backend.cpp -- tests of the C++ mirror of the kernel boundary
// (ocelotl_amd/host/kernel_backend.hpp), written the way the reference tests
// its backends (crates/kernels/src/lib.rs:2809-3070, :3339-3430;
// cubecl_backend.rs:2538-2737): same inputs to the reference CPU path and to
// the backend, compared with the reference rule abs <= tol || rel <= tol.
//
// The CPU path is the oracle (oracle/liboracle.so, linked by this test only).
// Usage: test_kernel_backend cpu|gpu   (cpu: needs no GPU; gpu: an MI355X)
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "dequant_policy.hpp"
#include "kernel_backend.hpp"

extern "C" {
// oracle/kquant_oracle.c
void okr_fill_normal(uint64_t seed, int64_t offset, int64_t n, float sigma, float *dst);
int okr_quantize(int type, const float *x, int64_t n, uint8_t *dst);
int okr_dequantize(int type, const uint8_t *src, int64_t n, float *dst);
int okr_linear_q(int type, int mode, int threads, const float *x, int64_t rows, int64_t in_f, const uint8_t *wq,
                 int64_t out_f, const float *bias, float *out);
int64_t okr_block_elems(int type);
int64_t okr_block_bytes(int type);
void okr_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *weight, float eps, float *out);
void okr_swiglu(const float *gate, const float *up, int64_t n, float *out);
int okr_linear_out_by_in(int mode, int threads, const float *x, int64_t rows, int64_t in_f, const float *w,
                         int64_t out_f, const float *bias, float *out);
}

using namespace ocelotl;

namespace {

struct Failure {
  std::string what;
};

#define CHECK(cond, msg)                                                                     \
  do {                                                                                       \
    if (!(cond)) throw Failure{std::string(msg) + "  [" #cond "] line " + std::to_string(__LINE__)}; \
  } while (0)

template <class T>
T ok(Result<T> r, const char *what) {
  if (r.is_err()) throw Failure{std::string(what) + ": " + r.error().to_string()};
  return std::move(r.value());
}
void ok(Result<void> r, const char *what) {
  if (r.is_err()) throw Failure{std::string(what) + ": " + r.error().to_string()};
}

constexpr int kScalarMode = 0;  // oracle: linear_out_by_in_compute (lib.rs:1974-2123)

std::vector<float> normal(uint64_t seed, size_t n, float sigma) {
  std::vector<float> v(n);
  okr_fill_normal(seed, 0, (int64_t)n, sigma, v.data());
  return v;
}

std::vector<uint8_t> quantize(GgmlTensorType t, const std::vector<float> &w) {
  const int64_t blocks = (int64_t)w.size() / okr_block_elems((int)t);
  std::vector<uint8_t> q((size_t)(blocks * okr_block_bytes((int)t)));
  CHECK(okr_quantize((int)t, w.data(), (int64_t)w.size(), q.data()) == 0, "oracle quantize");
  return q;
}

std::vector<float> reference(GgmlTensorType t, const std::vector<float> &x, size_t rows, size_t in, const std::vector<uint8_t> &wq,
                             size_t out_f, const float *bias) {
  std::vector<float> y(rows * out_f);
  CHECK(okr_linear_q((int)t, kScalarMode, 1, x.data(), (int64_t)rows, (int64_t)in, wq.data(), (int64_t)out_f, bias,
                     y.data()) == 0,
        "oracle linear");
  return y;
}

// The reference's comparison (lib.rs:2995-3002): per element abs <= tol or rel <= tol.
void assert_close(const std::vector<float> &got, const std::vector<float> &want, double tol, const char *what) {
  CHECK(got.size() == want.size(), what);
  for (size_t i = 0; i < got.size(); ++i) {
    const double g = got[i], w = want[i];
    const double abs = std::fabs(g - w), rel = abs / std::max(std::fabs(w), 1e-30);
    if (!(abs <= tol || rel <= tol)) {
      char buf[200];
      std::snprintf(buf, sizeof buf, "%s: element %zu got %.9g want %.9g", what, i, g, w);
      throw Failure{buf};
    }
  }
}

bool same_bits(const std::vector<float> &a, const std::vector<float> &b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

const GgmlTensorType kTypes[] = {GgmlTensorType::Q8_0, GgmlTensorType::Q4K, GgmlTensorType::Q5K, GgmlTensorType::Q6K};

// A backend with only the required f32 linear_out_by_in -- the reference CPU
// path (the oracle) -- so every quantized entry point runs the trait's
// defaults: host dequantization (product code), then this f32 linear.
class F32OnlyBackend final : public KernelBackend {
 public:
  const char *name() const override { return "cpu"; }
  const KernelContext &context() const override { return ctx_; }
  Result<DeviceTensor> upload(const float *host, size_t len) const override {
    return DeviceTensor::from_host(std::vector<float>(host, host + len));
  }
  Result<DeviceTensor> alloc(size_t len) const override { return DeviceTensor::host_zeros(len); }
  using KernelBackend::linear_out_by_in;
  Result<void> linear_out_by_in(const float *x, size_t x_len, size_t rows, size_t in_features, const float *weight,
                                size_t weight_len, size_t out_features, const float *bias, size_t bias_len, float *out,
                                size_t out_len) const override {
    if (x_len != rows * in_features || weight_len != out_features * in_features ||
        (bias && bias_len != out_features) || out_len != rows * out_features)
      return OcelotlError::kernel("cpu", "length mismatch");
    if (okr_linear_out_by_in(kScalarMode, 1, x, (int64_t)rows, (int64_t)in_features, weight, (int64_t)out_features,
                             bias, out) != 0)
      return OcelotlError::kernel("cpu", "oracle linear failed");
    ++f32_calls;
    return {};
  }
  mutable int f32_calls = 0;

 private:
  KernelContext ctx_{Device{Device::Kind::Cpu, 0}};
};

// Random blocks whose f16 scales are finite (the low byte random, the high
// byte kept in the normal range), so the decoders see every quant pattern.
std::vector<uint8_t> random_blocks(GgmlTensorType t, size_t blocks, uint64_t seed) {
  const auto info = ok(block_info(t), "block_info");
  std::vector<uint8_t> b(blocks * (size_t)info.second);
  uint64_t z = seed;
  for (auto &v : b) {
    z += 0x9E3779B97F4A7C15ull;
    uint64_t r = z;
    r = (r ^ (r >> 30)) * 0xBF58476D1CE4E5B9ull;
    r = (r ^ (r >> 27)) * 0x94D049BB133111EBull;
    v = (uint8_t)(r ^ (r >> 31));
  }
  auto fix_half = [&](size_t off) { b[off + 1] = (uint8_t)(0x18 + (b[off + 1] & 0x0F)); };  // |h| in [2^-9, 2^-1)
  for (size_t i = 0; i < blocks; ++i) {
    const size_t o = i * (size_t)info.second;
    if (t == GgmlTensorType::Q6K) {
      fix_half(o + 208);
    } else {
      fix_half(o);
      if (t == GgmlTensorType::Q4K || t == GgmlTensorType::Q5K) fix_half(o + 2);
    }
  }
  return b;
}

bool same_bits_nan_equal(const std::vector<float> &a, const std::vector<float> &b) {
  if (a.size() != b.size()) return false;
  for (size_t i = 0; i < a.size(); ++i) {
    if (std::isnan(a[i]) && std::isnan(b[i])) continue;
    if (std::memcmp(&a[i], &b[i], sizeof(float)) != 0) return false;
  }
  return true;
}

// ---- tests that need no GPU ---------------------------------------------------

void trait_default_dequantize_matches_the_cpu_definition() {
  F32OnlyBackend be;
  for (GgmlTensorType t : {GgmlTensorType::Q8_0, GgmlTensorType::Q4K, GgmlTensorType::Q5K, GgmlTensorType::Q6K}) {
    const auto info = ok(block_info(t), "block_info");
    const size_t blocks = 97, n = blocks * (size_t)info.first;
    const auto q = random_blocks(t, blocks, 4100 + (uint64_t)t);
    std::vector<float> got(n), want(n);
    ok(be.dequantize(t, q.data(), q.size(), n, got.data()), "default dequantize");
    CHECK(okr_dequantize((int)t, q.data(), (int64_t)n, want.data()) == 0, "oracle dequant");
    CHECK(same_bits_nan_equal(got, want), "host dequant must be bit-exact with the CPU definition");
    // special halves: zero, subnormal, infinity as the scale
    if (t == GgmlTensorType::Q8_0) {
      auto q2 = q;
      const uint16_t halves[] = {0x0000, 0x0001, 0x03ff, 0x7c00, 0xfc00};
      for (size_t i = 0; i < 5; ++i) {
        q2[i * 34] = (uint8_t)(halves[i] & 0xff);
        q2[i * 34 + 1] = (uint8_t)(halves[i] >> 8);
      }
      ok(be.dequantize(t, q2.data(), q2.size(), n, got.data()), "default dequantize (special scales)");
      CHECK(okr_dequantize((int)t, q2.data(), (int64_t)n, want.data()) == 0, "oracle dequant");
      CHECK(same_bits_nan_equal(got, want), "special f16 scales");
    }
  }
  // a format the host decoders do not cover is Unsupported; a short input a KernelError
  std::vector<float> y(32);
  std::vector<uint8_t> q40(18);
  auto e = be.dequantize(GgmlTensorType::Q4_0, q40.data(), q40.size(), 32, y.data());
  CHECK(e.is_err() && e.error().kind() == OcelotlError::Kind::Unsupported, "Q4_0 host dequant is unsupported");
  std::vector<uint8_t> shortq(33);
  e = be.dequantize(GgmlTensorType::Q8_0, shortq.data(), shortq.size(), 32, y.data());
  CHECK(e.is_err() && e.error().kind() == OcelotlError::Kind::Kernel, "short input");
}

void trait_default_quantized_linear_is_host_dequant_then_f32_linear() {
  // rows 5 x in 512 x out 37 (tails of the 4x4 tile), with and without bias:
  // the default must give the reference CPU path's bits (same dequant, same
  // f32 linear_out_by_in)
  F32OnlyBackend be;
  const size_t rows = 5, in = 512, out_f = 37;
  const auto x = normal(4200, rows * in, 1.0f);
  const auto bias = normal(4201, out_f, 0.1f);
  for (GgmlTensorType t : {GgmlTensorType::Q8_0, GgmlTensorType::Q4K, GgmlTensorType::Q5K, GgmlTensorType::Q6K}) {
    const auto q = quantize(t, normal(4203 + (uint64_t)t, out_f * in, 0.02f));
    auto w = ok(QuantizedWeight::from_host(t, in, out_f, q), "from_host");
    CHECK(w.residency().kind == Residency::Kind::Host && w.device_ptr() == nullptr, "host residency");
    for (const float *b : {(const float *)nullptr, bias.data()}) {
      std::vector<float> got(rows * out_f, -1.0f);
      const int calls = be.f32_calls;
      ok(be.linear_out_by_in(x.data(), x.size(), rows, in, w, out_f, b, b ? out_f : 0, got.data(), got.size()),
         "default quantized linear");
      CHECK(be.f32_calls == calls + 1, "the default runs the backend's f32 linear_out_by_in once");
      CHECK(same_bits(got, reference(t, x, rows, in, q, out_f, b)), "default quantized linear vs reference path");
    }
    // linear_d over host tensors: the default bounce, same bits
    auto xd = DeviceTensor::from_host(x);
    auto od = DeviceTensor::host_zeros(rows * out_f);
    ok(be.linear_d(xd, rows, in, w, out_f, nullptr, od), "default linear_d");
    CHECK(same_bits(ok(od.to_host_owned(), "read out"), reference(t, x, rows, in, q, out_f, nullptr)),
          "default linear_d vs reference path");
  }
  // validation before any work: a weight whose shape disagrees with the features
  const auto q = quantize(GgmlTensorType::Q8_0, normal(4204, 64 * 32, 0.02f));
  auto w = ok(QuantizedWeight::from_host(GgmlTensorType::Q8_0, 64, 32, q), "from_host");
  std::vector<float> xs(2 * 64), ys(2 * 31);
  const int calls = be.f32_calls;
  auto e = be.linear_out_by_in(xs.data(), xs.size(), 2, 64, w, 31, nullptr, 0, ys.data(), ys.size());
  CHECK(e.is_err() && e.error().kind() == OcelotlError::Kind::Kernel && be.f32_calls == calls,
        "shape mismatch is a KernelError before any compute");
  auto bad = QuantizedWeight::from_host(GgmlTensorType::Q8_0, 64, 32, std::vector<uint8_t>(q.size() - 1));
  CHECK(bad.is_err(), "from_host checks the byte length");
}

void block_info_matches_gguf_block_sizes() {
  struct Case { GgmlTensorType t; int64_t e, b; };
  for (Case c : {Case{GgmlTensorType::Q8_0, 32, 34}, Case{GgmlTensorType::Q4K, 256, 144},
                 Case{GgmlTensorType::Q6K, 256, 210}, Case{GgmlTensorType::F32, 1, 4},
                 Case{GgmlTensorType::F16, 1, 2}, Case{GgmlTensorType::BF16, 1, 2},
                 Case{GgmlTensorType::Q4_0, 32, 18}, Case{GgmlTensorType::Q4_1, 32, 20},
                 Case{GgmlTensorType::Q5_0, 32, 22}, Case{GgmlTensorType::Q5_1, 32, 24},
                 Case{GgmlTensorType::Q2K, 256, 84}, Case{GgmlTensorType::Q3K, 256, 110},
                 Case{GgmlTensorType::Q5K, 256, 176}}) {
    auto info = ok(block_info(c.t), "block_info");
    CHECK(info.first == c.e && info.second == c.b, "block sizes");
  }
  auto q8_1 = block_info((GgmlTensorType)9);  // Q8_1: named by the loader, no block format here
  CHECK(q8_1.is_err(), "Q8_1 must be unsupported");
  CHECK(q8_1.error().kind() == OcelotlError::Kind::Unsupported, "Q8_1 error kind");
  CHECK(q8_1.error().as_unsupported()->feature == "quantized_tensor_type", "Q8_1 feature");
}

void tensor_byte_len_of_the_gemma4_fixture_tensor() {
  // fixtures/metadata/gemma4_e4b_it_q4_k_m_gguf_metadata.json: token_embd.weight [2560, 262144] q4_k
  const uint64_t b = ok(tensor_byte_len(GgmlTensorType::Q4K, {2560, 262144}), "byte len");
  CHECK(b == 262144ull * (2560 / 256) * 144, "q4_k byte length");
  auto bad = tensor_byte_len(GgmlTensorType::Q4K, {100, 2});  // rows not block aligned
  CHECK(bad.is_err() && bad.error().kind() == OcelotlError::Kind::Kernel, "unaligned rows rejected");
}

void error_display_matches_the_reference_format() {
  CHECK(OcelotlError::kernel("hip-gfx950", "boom").to_string() == "kernel error on backend `hip-gfx950`: boom",
        "KernelError display");
  CHECK(OcelotlError::unsupported("gpu_backend", std::string("gpu"), {"cpu"}).to_string() ==
            "unsupported feature `gpu_backend` (requested `gpu`): supported = [cpu]",
        "UnsupportedError display");
  CHECK(OcelotlError::unsupported("x", std::nullopt, {"a", "b"}).to_string() ==
            "unsupported feature `x`: supported = [a, b]",
        "UnsupportedError display without request");
}

void create_without_a_gfx950_device_is_unsupported() {
  auto be = HipKernelBackend::create(0);
  if (be.is_ok()) {
    std::printf("         (a gfx950 device is present: nothing to check)\n");
    return;
  }
  CHECK(be.error().kind() == OcelotlError::Kind::Unsupported, "require_gpu kind");
  CHECK(be.error().as_unsupported()->feature == "gpu_backend", "require_gpu feature");
}

// DeviceTensor residency (tensor.rs:45-268): host tensors, views and their
// errors, as the reference's own tensor tests check them.
void host_tensors_and_views_follow_the_reference_semantics() {
  DeviceTensor h = DeviceTensor::from_host({1.0f, 2.0f, 3.0f, 4.0f, 5.0f});
  CHECK(h.len() == 5 && !h.is_empty() && h.residency().kind == Residency::Kind::Host, "host tensor");
  CHECK(h.device_ptr() == nullptr, "a host tensor has no device buffer");
  DeviceTensor v = ok(DeviceTensor::view(h, 1, 3), "view");
  CHECK(v.len() == 3 && v.is_view() && v.residency().kind == Residency::Kind::Host, "view of host");
  CHECK(ok(v.to_host_owned(), "view readback") == std::vector<float>({2.0f, 3.0f, 4.0f}), "view contents");
  auto nested = DeviceTensor::view(v, 0, 1);
  CHECK(nested.is_err() && nested.error().as_kernel()->backend == "tensor" &&
            nested.error().as_kernel()->message == "DeviceTensor::view does not nest; resolve the source view first",
        "views do not nest");
  auto range = DeviceTensor::view(h, 4, 2);
  CHECK(range.is_err() && range.error().as_kernel()->message == "DeviceTensor::view range 4..6 exceeds source length 5",
        "view range checked");
  const float w3[3] = {9.0f, 9.0f, 9.0f};
  auto ro = v.write_from_host_slice(w3, 3);
  CHECK(ro.is_err() && ro.error().as_kernel()->message == "DeviceTensor::write_from_host_slice: views are read-only",
        "views are read-only");
  auto bad_len = h.write_from_host_slice(w3, 3);
  CHECK(bad_len.is_err() &&
            bad_len.error().as_kernel()->message == "DeviceTensor::write_from_host_slice: src.len()=3 != tensor len 5",
        "write length checked");
  const float w5[5] = {5.0f, 4.0f, 3.0f, 2.0f, 1.0f};
  ok(h.write_from_host_slice(w5, 5), "write host");
  CHECK(ok(v.to_host_owned(), "view after write") == std::vector<float>({4.0f, 3.0f, 2.0f}), "views share storage");
  DeviceTensor copy = h;  // copies share the backing, as the reference's Arc does
  ok(copy.write_from_host_slice(w5, 5), "write through a copy");
  CHECK(ok(h.to_host_owned(), "shared")[0] == 5.0f, "copies share storage");
  CHECK(ok(DeviceTensor::host_zeros(3).to_host_owned(), "zeros") == std::vector<float>(3, 0.0f), "host_zeros");
}

// gemma4.rs:299-311 and the gate it feeds (:59-92), with the dequant policy.
void dequant_policy_gate_flips_for_executable_types() {
  for (uint32_t t = 0; t < 64; ++t) {
    const bool plain = t == 0 || t == 1 || t == 30 || (t >= 24 && t <= 28);
    CHECK(is_quantized_tensor_type(t) == !plain, "is_quantized_tensor_type " + std::to_string(t));
  }
  CHECK(is_quantized_tensor_type(1000), "unknown ids are quantized");
  CHECK(tensor_execution(12) == TensorExecution::QuantizedLinear && tensor_execution(8) == TensorExecution::QuantizedLinear &&
            tensor_execution(13) == TensorExecution::QuantizedLinear && tensor_execution(14) == TensorExecution::QuantizedLinear,
        "Q8_0, Q4K, Q5K, Q6K run the quantized linear");
  for (uint32_t t : {2u, 3u, 6u, 7u, 10u, 11u}) CHECK(tensor_execution(t) == TensorExecution::DequantizeToF32, "dequantized");
  for (uint32_t t : {9u, 15u, 16u, 23u, 29u, 34u, 39u, 77u}) CHECK(tensor_execution(t) == TensorExecution::None, "refused");
  CHECK(tensor_execution(0) == TensorExecution::Float && tensor_execution(30) == TensorExecution::Float, "float");
  CHECK(ggml_type_name(16) == "Iq2Xxs" && ggml_type_name(9) == "Q8_1" && ggml_type_name(39) == "MXFP4" &&
            ggml_type_name(77) == "Unknown(77)",
        "Debug names");
  // the gemma4 fixture (fixtures/metadata/gemma4_e4b_it_q4_k_m_gguf_metadata.json): a Q4_K
  // embedding table and an f32 norm -- the reference refuses it, the policy runs it
  GgufManifest m;
  m.tensors.push_back(GgufTensorEntry{"token_embd.weight", {2560, 262144}, 12, 0, 0, std::nullopt});
  m.tensors.push_back(GgufTensorEntry{"output_norm.weight", {2560}, 0, 0, 0, std::nullopt});
  CHECK(requires_dequant_policy(m), "a quantized tensor requires the dequant policy");
  ok(ensure_supported_for_execution(m), "Q4_K file passes the gate");
  m.tensors.push_back(GgufTensorEntry{"blk.0.attn_q.weight", {2560, 2048}, 16, 0, 0, std::nullopt});
  m.tensors.push_back(GgufTensorEntry{"blk.0.attn_k.weight", {2560, 512}, 9, 0, 0, std::nullopt});
  m.tensors.push_back(GgufTensorEntry{"blk.1.attn_q.weight", {2560, 2048}, 16, 0, 0, std::nullopt});
  auto refused = ensure_supported_for_execution(m);
  CHECK(refused.is_err() && refused.error().kind() == OcelotlError::Kind::Unsupported, "refused kind");
  CHECK(refused.error().as_unsupported()->feature == "quantized_tensor_types" &&
            refused.error().as_unsupported()->requested == std::string("Iq2Xxs,Q8_1"),
        "refused types in first-seen order, once each");
  GgufManifest f32_only;
  f32_only.tensors.push_back(GgufTensorEntry{"w", {8}, 0, 0, 0, std::nullopt});
  CHECK(!requires_dequant_policy(f32_only), "f32 files need no policy");
  ok(ensure_supported_for_execution(f32_only), "f32 files pass");
}

// ---- GPU tests ----------------------------------------------------------------------

HipKernelBackend backend() { return ok(HipKernelBackend::create(0), "create"); }

void backend_identity() {
  HipKernelBackend be = backend();
  CHECK(std::string(be.name()) == "hip-gfx950", "name");
  CHECK(be.context().device.kind == Device::Kind::Gpu && be.context().device.ordinal == 0, "context");
}

void linear_d_matches_reference_cpu_path() {
  HipKernelBackend be = backend();
  struct Shape { size_t rows, out_f, in; };
  for (GgmlTensorType t : kTypes) {
    for (Shape s : {Shape{1, 300, 1024}, Shape{3, 257, 2048}, Shape{6, 64, 4096}, Shape{40, 96, 512}}) {
      const auto wq = quantize(t, normal(100 + (int)t + s.in, s.out_f * s.in, 0.02f));
      const auto x = normal(200 + s.rows, s.rows * s.in, 1.0f);
      const auto bias = normal(300, s.out_f, 0.1f);
      QuantizedWeight w = ok(be.upload_quantized(t, s.in, s.out_f, wq.data(), wq.size()), "upload_quantized");
      DeviceTensor xd = ok(be.upload(x.data(), x.size()), "upload x");
      DeviceTensor bd = ok(be.upload(bias.data(), bias.size()), "upload bias");
      DeviceTensor od = ok(be.alloc(s.rows * s.out_f), "alloc out");
      ok(be.linear_d(xd, s.rows, s.in, w, s.out_f, &bd, od), "linear_d");
      const auto got = ok(od.to_host_owned(), "readback");
      assert_close(got, reference(t, x, s.rows, s.in, wq, s.out_f, bias.data()), 1e-3, "linear_d vs reference");
    }
  }
}

void linear_out_by_in_host_slices_match_linear_d_bit_for_bit() {
  HipKernelBackend be = backend();
  const size_t rows = 2, in = 2048, out_f = 130;
  for (GgmlTensorType t : kTypes) {
    const auto wq = quantize(t, normal(400 + (int)t, out_f * in, 0.02f));
    const auto x = normal(401, rows * in, 1.0f);
    QuantizedWeight w = ok(be.upload_quantized(t, in, out_f, wq.data(), wq.size()), "upload_quantized");
    std::vector<float> host_out(rows * out_f, NAN);
    ok(be.linear_out_by_in(x.data(), x.size(), rows, in, w, out_f, nullptr, 0, host_out.data(), host_out.size()),
       "linear_out_by_in");
    DeviceTensor xd = ok(be.upload(x.data(), x.size()), "upload");
    DeviceTensor od = ok(be.alloc(rows * out_f), "alloc");
    ok(be.linear_d(xd, rows, in, w, out_f, nullptr, od), "linear_d");
    CHECK(same_bits(host_out, ok(od.to_host_owned(), "readback")), "host-slice and device paths agree");
  }
}

// A host-resident weight (QuantizedWeight::from_host) is uploaded for the
// call and gives the device weight's bits; the f32 linear is Unsupported on
// this backend; dequantize over host slices runs on the GPU, bit-exact.
void host_weights_and_slices_on_the_hip_backend() {
  HipKernelBackend be = backend();
  const size_t rows = 3, in = 1024, out_f = 70;
  for (GgmlTensorType t : kTypes) {
    const auto wq = quantize(t, normal(450 + (int)t, out_f * in, 0.02f));
    const auto x = normal(451, rows * in, 1.0f);
    QuantizedWeight wd = ok(be.upload_quantized(t, in, out_f, wq.data(), wq.size()), "upload_quantized");
    QuantizedWeight wh = ok(QuantizedWeight::from_host(t, in, out_f, wq), "from_host");
    std::vector<float> a(rows * out_f, NAN), b(rows * out_f, NAN);
    ok(be.linear_out_by_in(x.data(), x.size(), rows, in, wd, out_f, nullptr, 0, a.data(), a.size()), "device weight");
    ok(be.linear_out_by_in(x.data(), x.size(), rows, in, wh, out_f, nullptr, 0, b.data(), b.size()), "host weight");
    CHECK(same_bits(a, b), "a host weight gives the device weight's bits");
    CHECK(ok(wd.to_host_bytes(), "read back blocks") == wq, "device blocks read back");
    std::vector<float> deq(out_f * in), want(out_f * in);
    ok(be.dequantize(t, wq.data(), wq.size(), deq.size(), deq.data()), "dequantize host slices");
    CHECK(okr_dequantize((int)t, wq.data(), (int64_t)want.size(), want.data()) == 0, "oracle dequant");
    CHECK(same_bits(deq, want), "GPU dequantize of host slices is bit-exact");
  }
  std::vector<float> x(4), w(4), y(1);
  auto e = be.linear_out_by_in(x.data(), 4, 1, 4, w.data(), 4, 1, nullptr, 0, y.data(), 1);
  CHECK(e.is_err() && e.error().kind() == OcelotlError::Kind::Unsupported, "f32 weights are not offloaded");
}

// Wrong residency stays correct: host-resident x, bias and out, and views of
// device tensors, take the trait default's bounce (lib.rs:193-217) and give
// the device path's bits.
void linear_d_with_host_tensors_and_views_takes_the_bounce() {
  HipKernelBackend be = backend();
  const size_t rows = 3, in = 1024, out_f = 200;
  for (GgmlTensorType t : kTypes) {
    const auto wq = quantize(t, normal(450 + (int)t, out_f * in, 0.02f));
    const auto x = normal(451, (rows + 2) * in, 1.0f);
    const auto bias = normal(452, out_f, 0.1f);
    QuantizedWeight w = ok(be.upload_quantized(t, in, out_f, wq.data(), wq.size()), "upload_quantized");
    const std::vector<float> xr(x.begin() + (ptrdiff_t)in, x.begin() + (ptrdiff_t)((rows + 1) * in));  // rows 1..3
    DeviceTensor xd = ok(be.upload(xr.data(), xr.size()), "upload x");
    DeviceTensor bd = ok(be.upload(bias.data(), bias.size()), "upload bias");
    DeviceTensor od = ok(be.alloc(rows * out_f), "alloc");
    ok(be.linear_d(xd, rows, in, w, out_f, &bd, od), "device linear_d");
    const auto want = ok(od.to_host_owned(), "readback");
    // host x, host bias, host out
    DeviceTensor xh = DeviceTensor::from_host(xr), bh = DeviceTensor::from_host(bias);
    DeviceTensor oh = DeviceTensor::host_zeros(rows * out_f);
    ok(be.linear_d(xh, rows, in, w, out_f, &bh, oh), "host linear_d");
    CHECK(oh.residency().kind == Residency::Kind::Host, "out stays on the host");
    CHECK(same_bits(ok(oh.to_host_owned(), "host out"), want), "host bounce equals the device path");
    // a view of a device tensor as x, device out
    DeviceTensor xall = ok(be.upload(x.data(), x.size()), "upload all");
    DeviceTensor xv = ok(DeviceTensor::view(xall, in, rows * in), "view");
    DeviceTensor od2 = ok(be.alloc(rows * out_f), "alloc 2");
    ok(be.linear_d(xv, rows, in, w, out_f, &bd, od2), "view linear_d");
    CHECK(same_bits(ok(od2.to_host_owned(), "view out"), want), "view bounce equals the device path");
    // device x, host out
    DeviceTensor oh2 = DeviceTensor::host_zeros(rows * out_f);
    ok(be.linear_d(xd, rows, in, w, out_f, &bd, oh2), "host out linear_d");
    CHECK(same_bits(ok(oh2.to_host_owned(), "host out 2"), want), "host out equals the device path");
    // a view is read-only: as out it is an error, nothing written
    DeviceTensor ov = ok(DeviceTensor::view(xall, 0, rows * out_f), "view out");
    auto r = be.linear_d(xd, rows, in, w, out_f, &bd, ov);
    CHECK(r.is_err() && r.error().as_kernel()->message == "DeviceTensor::write_from_host_slice: views are read-only",
          "views are read-only outputs");
  }
}

void linear_d_rejects_mismatched_lengths_before_launch() {
  HipKernelBackend be = backend();
  const size_t in = 256, out_f = 8;
  const auto wq = quantize(GgmlTensorType::Q4K, normal(500, out_f * in, 0.02f));
  QuantizedWeight w = ok(be.upload_quantized(GgmlTensorType::Q4K, in, out_f, wq.data(), wq.size()), "upload");
  std::vector<float> sentinel(2 * out_f, 7.0f);
  DeviceTensor od = ok(be.upload(sentinel.data(), sentinel.size()), "out");
  DeviceTensor x_short = ok(be.alloc(2 * in - 1), "x");
  auto r = be.linear_d(x_short, 2, in, w, out_f, nullptr, od);
  CHECK(r.is_err() && r.error().kind() == OcelotlError::Kind::Kernel, "short x is a KernelError");
  CHECK(r.error().as_kernel()->backend == "hip-gfx950", "backend named");
  CHECK(r.error().as_kernel()->message == "linear_out_by_in x.len()=511 does not match rows*in_features=2*256=512",
        "message: " + r.error().as_kernel()->message);
  DeviceTensor x = ok(be.alloc(2 * in), "x");
  DeviceTensor bias_bad = ok(be.alloc(out_f + 1), "bias");
  CHECK(be.linear_d(x, 2, in, w, out_f, &bias_bad, od).is_err(), "bias length");
  DeviceTensor od_short = ok(be.alloc(2 * out_f - 1), "out");
  CHECK(be.linear_d(x, 2, in, w, out_f, nullptr, od_short).is_err(), "out length");
  CHECK(be.linear_d(x, 2, in, w, out_f + 1, nullptr, od).is_err(), "weight shape");
  CHECK(same_bits(ok(od.to_host_owned(), "readback"), sentinel), "nothing was launched");
}

void upload_quantized_validates_type_and_byte_length() {
  HipKernelBackend be = backend();
  std::vector<uint8_t> bytes(144 * 4, 0);
  CHECK(be.upload_quantized(GgmlTensorType::Q4K, 256, 4, bytes.data(), bytes.size()).is_ok(), "exact length");
  auto short_len = be.upload_quantized(GgmlTensorType::Q4K, 256, 4, bytes.data(), bytes.size() - 1);
  CHECK(short_len.is_err() && short_len.error().kind() == OcelotlError::Kind::Kernel, "wrong length");
  auto f32 = be.upload_quantized(GgmlTensorType::F32, 256, 4, bytes.data(), bytes.size());
  CHECK(f32.is_err() && f32.error().kind() == OcelotlError::Kind::Unsupported, "unquantized type");
}

void dequantize_is_bit_exact_with_the_cpu_definition() {
  HipKernelBackend be = backend();
  for (GgmlTensorType t : kTypes) {
    const size_t in = 1024, out_f = 33;
    const auto wq = quantize(t, normal(600 + (int)t, out_f * in, 0.02f));
    QuantizedWeight w = ok(be.upload_quantized(t, in, out_f, wq.data(), wq.size()), "upload");
    const auto got = ok(ok(be.dequantize(w), "dequantize").to_host_owned(), "readback");
    std::vector<float> want(out_f * in);
    CHECK(okr_dequantize((int)t, wq.data(), (int64_t)want.size(), want.data()) == 0, "oracle dequant");
    CHECK(same_bits(got, want), "dequant bits");
  }
}

void linear_d_one_hot_column_is_exact() {
  // x = e_j reproduces column j of the dequantized weight exactly
  HipKernelBackend be = backend();
  for (GgmlTensorType t : kTypes) {
    const size_t in = 512, out_f = 40;
    const auto wq = quantize(t, normal(700 + (int)t, out_f * in, 0.02f));
    std::vector<float> wdeq(out_f * in);
    CHECK(okr_dequantize((int)t, wq.data(), (int64_t)wdeq.size(), wdeq.data()) == 0, "oracle dequant");
    QuantizedWeight w = ok(be.upload_quantized(t, in, out_f, wq.data(), wq.size()), "upload");
    for (size_t j : {size_t(0), size_t(31), size_t(257), in - 1}) {
      std::vector<float> x(in, 0.0f);
      x[j] = 1.0f;
      DeviceTensor xd = ok(be.upload(x.data(), in), "x");
      DeviceTensor od = ok(be.alloc(out_f), "out");
      ok(be.linear_d(xd, 1, in, w, out_f, nullptr, od), "linear_d");
      const auto got = ok(od.to_host_owned(), "readback");
      for (size_t o = 0; o < out_f; ++o) CHECK(got[o] == wdeq[o * in + j], "one-hot column");
    }
  }
}

// ---- neighbours (rmsnorm, gated MLP, embedding rows) ---------------------------

void rmsnorm_matches_the_reference_and_its_kats() {
  HipKernelBackend be = ok(HipKernelBackend::create(0), "create");
  // rmsnorm.rs:150-165: x = [1, 2, 3], unit weight, eps 1e-6
  const float x3[3] = {1, 2, 3}, w3[3] = {1, 1, 1};
  float o3[3] = {0, 0, 0};
  ok(be.rmsnorm(x3, 3, 1, 3, w3, 3, 1e-6f, o3, 3), "rmsnorm kat");
  const float want3[3] = {0.46291006f, 0.9258201f, 1.3887302f};
  for (int i = 0; i < 3; ++i) CHECK(std::fabs(o3[i] - want3[i]) <= 1e-6f, "rmsnorm kat value");
  const size_t rows = 5, hidden = 4096;
  std::vector<float> x = normal(61, rows * hidden, 2.0f), w = normal(62, hidden, 1.0f), got(rows * hidden),
                     want(rows * hidden);
  ok(be.rmsnorm(x.data(), x.size(), rows, hidden, w.data(), w.size(), 1e-5f, got.data(), got.size()), "rmsnorm");
  okr_rmsnorm(x.data(), (int64_t)rows, (int64_t)hidden, w.data(), 1e-5f, want.data());
  assert_close(got, want, 1e-5, "rmsnorm vs reference order");
  // validation before launch, with the reference's messages (rmsnorm.rs:81-114)
  auto e1 = be.rmsnorm(x.data(), x.size(), rows, hidden, w.data(), w.size() - 1, 1e-5f, got.data(), got.size());
  CHECK(e1.is_err() && e1.error().as_kernel()->message.find("weight length 4095 does not match hidden 4096") !=
                           std::string::npos,
        "weight length message");
  auto e2 = be.rmsnorm(x.data(), x.size(), rows, hidden, w.data(), w.size(), -1.0f, got.data(), got.size());
  CHECK(e2.is_err() && e2.error().as_kernel()->message.find("epsilon must be finite and non-negative") !=
                           std::string::npos,
        "epsilon message");
}

void mlp_gated_silu_q_matches_the_reference_chain() {
  HipKernelBackend be = ok(HipKernelBackend::create(0), "create");
  const size_t hidden = 1024, inter = 2816;
  auto gq = quantize(GgmlTensorType::Q4K, normal(71, inter * hidden, 0.02f));
  auto uq = quantize(GgmlTensorType::Q4K, normal(72, inter * hidden, 0.02f));
  auto dq = quantize(GgmlTensorType::Q6K, normal(73, hidden * inter, 0.02f));
  auto G = ok(be.upload_quantized(GgmlTensorType::Q4K, hidden, inter, gq.data(), gq.size()), "gate");
  auto U = ok(be.upload_quantized(GgmlTensorType::Q4K, hidden, inter, uq.data(), uq.size()), "up");
  auto D = ok(be.upload_quantized(GgmlTensorType::Q6K, inter, hidden, dq.data(), dq.size()), "down");
  for (size_t rows : {1, 3, 12}) {  // fused decode row, multi-row GEMV, MFMA GEMM
    std::vector<float> x = normal(74 + rows, rows * hidden, 1.0f);
    auto xd = ok(be.upload(x.data(), x.size()), "x");
    auto gb = ok(be.alloc(rows * inter), "gate_buf");
    auto ub = ok(be.alloc(rows * inter), "up_buf");
    auto od = ok(be.alloc(rows * hidden), "out");
    ok(be.mlp_gated_silu_q(xd, rows, hidden, inter, G, U, D, gb, ub, od), "mlp");
    std::vector<float> got = ok(od.to_host_owned(), "out host");
    std::vector<float> gate = reference(GgmlTensorType::Q4K, x, rows, hidden, gq, inter, nullptr);
    std::vector<float> up = reference(GgmlTensorType::Q4K, x, rows, hidden, uq, inter, nullptr);
    std::vector<float> h(rows * inter);
    okr_swiglu(gate.data(), up.data(), (int64_t)h.size(), h.data());
    std::vector<float> want = reference(GgmlTensorType::Q6K, h, rows, inter, dq, hidden, nullptr);
    // normwise over the chain: silu(gate) * up amplifies the projections'
    // per-element differences (each projection alone meets the element rule)
    double m = 0, e = 0;
    for (size_t i = 0; i < want.size(); ++i) m = std::max(m, (double)std::fabs(want[i])), e = std::max(e, (double)std::fabs(got[i] - want[i]));
    CHECK(e <= 1e-3 * m, "mlp chain normwise");
    assert_close(ok(ub.to_host_owned(), "up host"), up, 1e-3, "up(x) in up_buf");
  }
  // zero rows is an error (mlp.rs:151-155), checked before launch
  auto xd = ok(be.upload(std::vector<float>(hidden, 1.0f).data(), hidden), "x");
  auto gb = ok(be.alloc(inter), "gb");
  auto ub = ok(be.alloc(inter), "ub");
  auto od = ok(be.alloc(hidden), "od");
  auto r0 = be.mlp_gated_silu_q(xd, 0, hidden, inter, G, U, D, gb, ub, od);
  CHECK(r0.is_err() && r0.error().as_kernel()->message == "mlp_gated_silu seq_len must be non-zero", "rows 0");
  auto r1 = be.mlp_gated_silu_q(xd, 1, hidden, inter, G, D, D, gb, ub, od);
  CHECK(r1.is_err() && r1.error().as_kernel()->message.find("up_w shape") != std::string::npos, "up shape");
}

void embedding_rows_are_the_dequantized_rows() {
  HipKernelBackend be = ok(HipKernelBackend::create(0), "create");
  const size_t hidden = 2560, vocab = 300;
  for (GgmlTensorType t : kTypes) {
    auto q = quantize(t, normal(81 + (int)t, hidden * vocab, 0.02f));
    auto table = ok(be.upload_quantized(t, hidden, vocab, q.data(), q.size()), "table");
    std::vector<float> all(hidden * vocab);
    CHECK(okr_dequantize((int)t, q.data(), (int64_t)all.size(), all.data()) == 0, "oracle dequant");
    const uint32_t ids[5] = {299, 0, 17, 17, 150};
    std::vector<float> got = ok(ok(be.embedding_rows(table, ids, 5), "rows").to_host_owned(), "rows host");
    for (size_t j = 0; j < 5; ++j)
      CHECK(std::memcmp(got.data() + j * hidden, all.data() + ids[j] * hidden, hidden * sizeof(float)) == 0,
            "row bits");
    const uint32_t bad[1] = {300};
    auto e = be.embedding_rows(table, bad, 1);
    CHECK(e.is_err() && e.error().as_kernel()->message.find("out of range") != std::string::npos, "id range");
  }
}

struct Test {
  const char *name;
  std::function<void()> fn;
};

}  // namespace

int main(int argc, char **argv) {
  const std::string suite = argc > 1 ? argv[1] : "cpu";
  std::vector<Test> tests;
  if (suite == "cpu") {
    tests = {{"block_info_matches_gguf_block_sizes", block_info_matches_gguf_block_sizes},
             {"tensor_byte_len_of_the_gemma4_fixture_tensor", tensor_byte_len_of_the_gemma4_fixture_tensor},
             {"error_display_matches_the_reference_format", error_display_matches_the_reference_format},
             {"create_without_a_gfx950_device_is_unsupported", create_without_a_gfx950_device_is_unsupported},
             {"host_tensors_and_views_follow_the_reference_semantics",
              host_tensors_and_views_follow_the_reference_semantics},
             {"dequant_policy_gate_flips_for_executable_types", dequant_policy_gate_flips_for_executable_types},
             {"trait_default_dequantize_matches_the_cpu_definition",
              trait_default_dequantize_matches_the_cpu_definition},
             {"trait_default_quantized_linear_is_host_dequant_then_f32_linear",
              trait_default_quantized_linear_is_host_dequant_then_f32_linear}};
  } else if (suite == "gpu") {
    tests = {{"backend_identity", backend_identity},
             {"linear_d_matches_reference_cpu_path", linear_d_matches_reference_cpu_path},
             {"linear_out_by_in_host_slices_match_linear_d_bit_for_bit",
              linear_out_by_in_host_slices_match_linear_d_bit_for_bit},
             {"linear_d_rejects_mismatched_lengths_before_launch", linear_d_rejects_mismatched_lengths_before_launch},
             {"linear_d_with_host_tensors_and_views_takes_the_bounce",
              linear_d_with_host_tensors_and_views_takes_the_bounce},
             {"upload_quantized_validates_type_and_byte_length", upload_quantized_validates_type_and_byte_length},
             {"dequantize_is_bit_exact_with_the_cpu_definition", dequantize_is_bit_exact_with_the_cpu_definition},
             {"linear_d_one_hot_column_is_exact", linear_d_one_hot_column_is_exact},
             {"rmsnorm_matches_the_reference_and_its_kats", rmsnorm_matches_the_reference_and_its_kats},
             {"mlp_gated_silu_q_matches_the_reference_chain", mlp_gated_silu_q_matches_the_reference_chain},
             {"embedding_rows_are_the_dequantized_rows", embedding_rows_are_the_dequantized_rows},
             {"host_weights_and_slices_on_the_hip_backend", host_weights_and_slices_on_the_hip_backend}};
  } else {
    std::fprintf(stderr, "usage: %s cpu|gpu\n", argv[0]);
    return 2;
  }
  int failed = 0;
  for (const Test &t : tests) {
    std::printf("[ RUN  ] %s\n", t.name);
    std::fflush(stdout);
    try {
      t.fn();
      std::printf("[  OK  ] %s\n", t.name);
    } catch (const Failure &f) {
      ++failed;
      std::printf("[ FAIL ] %s: %s\n", t.name, f.what.c_str());
    }
    std::fflush(stdout);
  }
  std::printf("%zu tests, %d failed\n", tests.size(), failed);
  return failed ? 1 : 0;
}
