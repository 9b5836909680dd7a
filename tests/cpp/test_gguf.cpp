// test_gguf.cpp -- tests of the GGUF loader (ocelotl_amd/host/gguf.hpp).
//
// The cpu suite restates, as behaviours, the reference's inspect_gguf tests
// (crates/loader/src/gguf_inspect.rs:808-965): a minimal v3 manifest, a
// missing file, a truncated header, an unsupported version, a tensor past the
// end, an oversized metadata string and an unaligned offset, each on a file
// written here; plus what this loader adds: byte lengths of Q8_0 / Q4_K /
// Q6_K tensors (checked against the file length) and the Gemma4 fixture's
// token_embd shape.  The gpu suite writes quantized tensors into a GGUF file,
// loads them onto the device and compares the dequantized weights and a
// linear with the CPU oracle.
// Usage: test_gguf cpu|gpu
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <unistd.h>
#include <vector>

#include "gguf.hpp"

extern "C" {
// oracle/kquant_oracle.c
void okr_fill_normal(uint64_t seed, int64_t offset, int64_t n, float sigma, float *dst);
int okr_quantize(int type, const float *x, int64_t n, uint8_t *dst);
int okr_dequantize(int type, const uint8_t *src, int64_t n, float *dst);
int okr_linear_q(int type, int mode, int threads, const float *x, int64_t rows, int64_t in_f, const uint8_t *wq,
                 int64_t out_f, const float *bias, float *out);
}

using namespace ocelotl;

namespace {

struct Failure {
  std::string what;
};

#define CHECK(cond, msg)                                                                                  \
  do {                                                                                                    \
    if (!(cond)) throw Failure{std::string(msg) + "  [" #cond "] line " + std::to_string(__LINE__)};    \
  } while (0)

template <class T>
T ok(Result<T> r, const char *what) {
  if (r.is_err()) throw Failure{std::string(what) + ": " + r.error().to_string()};
  return std::move(r.value());
}

// ---- fixture writer (GGUF v3, little-endian) ---------------------------------

struct Writer {
  std::vector<uint8_t> b;
  void u32(uint32_t v) { b.insert(b.end(), (uint8_t *)&v, (uint8_t *)&v + 4); }
  void u64(uint64_t v) { b.insert(b.end(), (uint8_t *)&v, (uint8_t *)&v + 8); }
  void str(const std::string &s) {
    u64(s.size());
    b.insert(b.end(), s.begin(), s.end());
  }
  void kv_str(const std::string &k, const std::string &v) { str(k), u32(8), str(v); }
  void kv_u32(const std::string &k, uint32_t v) { str(k), u32(4), u32(v); }
  void kv_str_array(const std::string &k, const std::vector<std::string> &vs) {
    str(k), u32(9), u32(8), u64(vs.size());
    for (const std::string &v : vs) str(v);
  }
  void tensor(const std::string &name, const std::vector<uint64_t> &shape, uint32_t type, uint64_t offset) {
    str(name);
    u32((uint32_t)shape.size());
    for (uint64_t d : shape) u64(d);
    u32(type);
    u64(offset);
  }
  void pad(size_t a) {
    while (b.size() % a) b.push_back(0);
  }
  void write(const std::string &path) const {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) throw Failure{"cannot write " + path};
    std::fwrite(b.data(), 1, b.size(), f);
    std::fclose(f);
  }
};

std::string tmp_path(const std::string &name) {
  return "/tmp/okq_gguf_test_" + std::to_string(getpid()) + "_" + name + ".gguf";
}

// The minimal fixture of the reference test: 4 metadata entries, one F32
// [2, 2] tensor at `offset`, `data_len` payload bytes after alignment.
void write_minimal(const std::string &path, uint64_t offset, size_t data_len) {
  Writer w;
  w.b = {'G', 'G', 'U', 'F'};
  w.u32(3), w.u64(1), w.u64(4);
  w.kv_str("general.architecture", "gemma4");
  w.kv_str("general.name", "tiny synthetic gemma4");
  w.kv_u32("general.alignment", 32);
  w.kv_str_array("tokenizer.ggml.tokens", {"<bos>", "<eos>"});
  w.tensor("blk.0.attn_q.weight", {2, 2}, 0, offset);
  w.pad(32);
  w.b.insert(w.b.end(), data_len, 0);
  w.write(path);
}

InvalidModelError expect_invalid(const Result<GgufManifest> &r, const char *what) {
  if (r.is_ok()) throw Failure{std::string(what) + ": expected InvalidModel, got Ok"};
  const InvalidModelError *m = r.error().as_invalid_model();
  if (!m) throw Failure{std::string(what) + ": expected InvalidModel, got " + r.error().to_string()};
  return *m;
}

bool contains(const std::string &s, const char *sub) { return s.find(sub) != std::string::npos; }

// ---- cpu suite ----------------------------------------------------------------

void parses_minimal_v3_manifest() {
  const std::string p = tmp_path("minimal");
  write_minimal(p, 0, 16);
  GgufManifest m = ok(inspect_gguf(p), "inspect");
  CHECK(m.version == 3 && m.alignment == 32, "version/alignment");
  const GgufMetadataValue *arch = m.metadata_value("general.architecture");
  CHECK(arch && arch->type == GgufMetadataType::String && arch->s == "gemma4", "architecture");
  const GgufMetadataValue *tok = m.metadata_value("tokenizer.ggml.tokens");
  CHECK(tok && tok->type == GgufMetadataType::Array && tok->element_type == GgufMetadataType::String &&
            tok->len == 2,
        "tokens array");
  CHECK(m.tensors.size() == 1, "one tensor");
  const GgufTensorEntry &t = m.tensors[0];
  CHECK(t.name == "blk.0.attn_q.weight" && t.shape == std::vector<uint64_t>({2, 2}) && t.tensor_type == 0, "entry");
  CHECK(t.offset == 0 && t.byte_len && *t.byte_len == 16 && t.file_offset == m.data_start, "offsets");
  CHECK(m.data_start % 32 == 0 && m.file_len == m.data_start + 16, "data section");
  std::remove(p.c_str());
}

void missing_file_is_an_io_error() {
  const std::string p = tmp_path("missing");
  auto r = inspect_gguf(p);
  CHECK(r.is_err() && r.error().as_io(), "Io error");
  CHECK(r.error().as_io()->code == ENOENT && *r.error().as_io()->path == p, "ENOENT with path");
}

void truncated_header_is_invalid_model() {
  const std::string p = tmp_path("truncated");
  Writer w;
  w.b = {'G', 'G', 'U', 'F', 3};
  w.write(p);
  const InvalidModelError e = expect_invalid(inspect_gguf(p), "truncated");
  CHECK(e.field && *e.field == "header" && contains(e.message, "truncated") && *e.path == p, "field/message");
  std::remove(p.c_str());
}

void unsupported_version_is_typed_unsupported() {
  const std::string p = tmp_path("version");
  Writer w;
  w.b = {'G', 'G', 'U', 'F'};
  w.u32(99), w.u64(0), w.u64(0);
  w.write(p);
  auto r = inspect_gguf(p);
  CHECK(r.is_err() && r.error().as_unsupported(), "Unsupported");
  const UnsupportedError &u = *r.error().as_unsupported();
  CHECK(u.feature == "gguf_version" && u.requested && *u.requested == "99", "feature/requested");
  CHECK(u.supported.size() == 1 && u.supported[0] == "3", "supported");
  std::remove(p.c_str());
}

void tensor_past_the_end_is_rejected_before_payload_read() {
  const std::string p = tmp_path("bad_offset");
  write_minimal(p, 64, 16);
  const InvalidModelError e = expect_invalid(inspect_gguf(p), "bad offset");
  CHECK(e.field && *e.field == "blk.0.attn_q.weight", "field is the tensor");
  CHECK(contains(e.message, "exceeds file length") || contains(e.message, "beyond file length"), e.message);
  std::remove(p.c_str());
}

void oversized_metadata_string_is_rejected() {
  const std::string p = tmp_path("oversized");
  Writer w;
  w.b = {'G', 'G', 'U', 'F'};
  w.u32(3), w.u64(0), w.u64(1);
  w.str("general.name");
  w.u32(8);
  w.u64(16ull * 1024 * 1024 + 1);
  w.write(p);
  const InvalidModelError e = expect_invalid(inspect_gguf(p), "oversized");
  CHECK(e.field && *e.field == "metadata string" && contains(e.message, "exceeds max"), e.message);
  std::remove(p.c_str());
}

void unaligned_tensor_offset_is_rejected() {
  const std::string p = tmp_path("unaligned");
  write_minimal(p, 1, 16);
  const InvalidModelError e = expect_invalid(inspect_gguf(p), "unaligned");
  CHECK(e.field && *e.field == "blk.0.attn_q.weight" && contains(e.message, "not aligned"), e.message);
  std::remove(p.c_str());
}

void bad_alignment_and_magic_are_rejected() {
  const std::string p = tmp_path("align");
  Writer w;
  w.b = {'G', 'G', 'U', 'F'};
  w.u32(3), w.u64(0), w.u64(1);
  w.kv_u32("general.alignment", 12);
  w.write(p);
  const InvalidModelError e = expect_invalid(inspect_gguf(p), "alignment 12");
  CHECK(e.field && *e.field == "general.alignment" && contains(e.message, "positive multiple of 8"), e.message);
  Writer m;
  m.b = {'G', 'G', 'U', 'X'};
  m.u32(3), m.u64(0), m.u64(0);
  m.write(p);
  const InvalidModelError e2 = expect_invalid(inspect_gguf(p), "magic");
  CHECK(e2.field && *e2.field == "magic", e2.message);
  std::remove(p.c_str());
}

// What this loader adds: block-quantized byte lengths, range-checked.
void quantized_byte_lengths_are_known_and_range_checked() {
  const std::string p = tmp_path("quant");
  struct T {
    const char *name;
    std::vector<uint64_t> shape;
    uint32_t type;
    uint64_t bytes;
  } ts[] = {{"a.q8_0", {64, 3}, 8, 3 * 2 * 34},
            {"b.q4_k", {512, 5}, 12, 5 * 2 * 144},
            {"c.q6_k", {256, 7}, 14, 7 * 210},
            {"d.q5_k", {256, 2}, 13, 2 * 176},
            {"e.q4_0", {96, 2}, 2, 2 * 3 * 18},
            {"f.q3_k", {512, 1}, 11, 2 * 110},
            {"g.q8_1", {64, 2}, 9, 0}};  // no block layout here: length unknown, as in the reference
  Writer w;
  w.b = {'G', 'G', 'U', 'F'};
  w.u32(3), w.u64(7), w.u64(0);
  uint64_t off = 0;
  for (const T &t : ts) {
    w.tensor(t.name, t.shape, t.type, off);
    off += (t.bytes + 31) / 32 * 32;
  }
  w.pad(32);
  w.b.insert(w.b.end(), off, 0);
  w.write(p);
  GgufManifest m = ok(inspect_gguf(p), "inspect quantized");
  for (size_t i = 0; i < 6; ++i) {
    CHECK(m.tensors[i].byte_len && *m.tensors[i].byte_len == ts[i].bytes, ts[i].name);
    auto b = tensor_byte_len(static_cast<GgmlTensorType>(ts[i].type),
                             {(int64_t)ts[i].shape[0], (int64_t)ts[i].shape[1]});
    CHECK(b.is_ok() && b.value() == ts[i].bytes, "agrees with okq_tensor_bytes");
  }
  CHECK(!m.tensors[6].byte_len, "Q8_1 length unknown");
  // the same file cut short: the last quantized tensor no longer fits
  Writer cut = w;
  cut.b.resize(cut.b.size() - off + ts[0].bytes + 32 + ts[1].bytes);
  cut.write(p);
  const InvalidModelError e = expect_invalid(inspect_gguf(p), "cut");
  CHECK(e.field && *e.field == "c.q6_k" && contains(e.message, "exceeds file length"), e.message);
  // a Q4_K row that is not whole blocks
  Writer bad;
  bad.b = {'G', 'G', 'U', 'F'};
  bad.u32(3), bad.u64(1), bad.u64(0);
  bad.tensor("e.q4_k", {300, 2}, 12, 0);
  bad.pad(32);
  bad.b.insert(bad.b.end(), 4096, 0);
  bad.write(p);
  const InvalidModelError e2 = expect_invalid(inspect_gguf(p), "ragged row");
  CHECK(e2.field && *e2.field == "e.q4_k" && contains(e2.message, "block size 256"), e2.message);
  std::remove(p.c_str());
}

void gemma4_fixture_token_embd_byte_len() {
  // fixtures/metadata/gemma4_e4b_it_q4_k_m_gguf_metadata.json: token_embd.weight
  // [2560, 262144] q4_k -> 262144 rows of 10 super-blocks
  ByteLen b = gguf_byte_len(12, {2560, 262144});
  CHECK(b.error.empty() && b.bytes && *b.bytes == 262144ull * 10 * 144, "token_embd bytes");
}

// ---- gpu suite ------------------------------------------------------------------

void loaded_weights_match_the_file_bit_for_bit_and_run() {
  HipKernelBackend be = ok(HipKernelBackend::create(0), "create");
  const std::string p = tmp_path("gpu");
  struct T {
    const char *name;
    uint32_t type;
    uint64_t ne0, ne1;
    std::vector<uint8_t> q;
  } ts[] = {{"blk.0.attn_q.weight", 12, 4096, 64, {}},
            {"blk.0.ffn_down.weight", 14, 1024, 33, {}},
            {"output.weight", 8, 2048, 17, {}}};
  Writer w;
  w.b = {'G', 'G', 'U', 'F'};
  w.u32(3), w.u64(3), w.u64(1);
  w.kv_str("general.architecture", "llama");
  uint64_t off = 0;
  std::vector<uint64_t> offs;
  for (T &t : ts) {
    std::vector<float> f(t.ne0 * t.ne1);
    okr_fill_normal(900 + t.type, 0, (int64_t)f.size(), 0.02f, f.data());
    const int64_t be_ = t.type == 8 ? 32 : 256, bb = t.type == 8 ? 34 : t.type == 12 ? 144 : 210;
    t.q.resize(f.size() / be_ * bb);
    CHECK(okr_quantize((int)t.type, f.data(), (int64_t)f.size(), t.q.data()) == 0, "quantize");
    w.tensor(t.name, {t.ne0, t.ne1}, t.type, off);
    offs.push_back(off);
    off += (t.q.size() + 31) / 32 * 32;
  }
  w.pad(32);
  const size_t data = w.b.size();
  w.b.resize(data + off, 0);
  for (size_t i = 0; i < 3; ++i) std::memcpy(w.b.data() + data + offs[i], ts[i].q.data(), ts[i].q.size());
  w.write(p);
  GgufManifest m = ok(inspect_gguf(p), "inspect");
  for (const T &t : ts) {
    QuantizedWeight qw = ok(load_quantized_weight(be, p, m, t.name), t.name);
    CHECK(qw.ne0() == t.ne0 && qw.ne1() == t.ne1 && qw.byte_len() == t.q.size(), "shape");
    std::vector<float> want(t.ne0 * t.ne1);
    CHECK(okr_dequantize((int)t.type, t.q.data(), (int64_t)want.size(), want.data()) == 0, "oracle dequant");
    std::vector<float> got = ok(ok(be.dequantize(qw), "dequantize").to_host_owned(), "to_host");
    CHECK(std::memcmp(got.data(), want.data(), want.size() * 4) == 0, "dequantized bits");
    std::vector<float> x(2 * t.ne0);
    okr_fill_normal(77, 0, (int64_t)x.size(), 1.0f, x.data());
    std::vector<float> y(2 * t.ne1), ref(2 * t.ne1);
    auto r = be.linear_out_by_in(x.data(), x.size(), 2, t.ne0, qw, t.ne1, nullptr, 0, y.data(), y.size());
    CHECK(r.is_ok(), r.is_ok() ? "" : r.error().to_string());
    CHECK(okr_linear_q((int)t.type, 0, 1, x.data(), 2, (int64_t)t.ne0, t.q.data(), (int64_t)t.ne1, nullptr,
                       ref.data()) == 0,
          "oracle linear");
    for (size_t i = 0; i < y.size(); ++i) {
      const float d = std::fabs(y[i] - ref[i]);
      CHECK(d <= 1e-3f || d <= 1e-3f * std::fabs(ref[i]), "linear within the reference rule");
    }
  }
  auto missing = load_quantized_weight(be, p, m, "no.such.tensor");
  CHECK(missing.is_err() && missing.error().as_invalid_model(), "missing tensor");
  std::remove(p.c_str());
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
    tests = {{"parses_minimal_v3_manifest", parses_minimal_v3_manifest},
             {"missing_file_is_an_io_error", missing_file_is_an_io_error},
             {"truncated_header_is_invalid_model", truncated_header_is_invalid_model},
             {"unsupported_version_is_typed_unsupported", unsupported_version_is_typed_unsupported},
             {"tensor_past_the_end_is_rejected_before_payload_read",
              tensor_past_the_end_is_rejected_before_payload_read},
             {"oversized_metadata_string_is_rejected", oversized_metadata_string_is_rejected},
             {"unaligned_tensor_offset_is_rejected", unaligned_tensor_offset_is_rejected},
             {"bad_alignment_and_magic_are_rejected", bad_alignment_and_magic_are_rejected},
             {"quantized_byte_lengths_are_known_and_range_checked", quantized_byte_lengths_are_known_and_range_checked},
             {"gemma4_fixture_token_embd_byte_len", gemma4_fixture_token_embd_byte_len}};
  } else if (suite == "gpu") {
    tests = {{"loaded_weights_match_the_file_bit_for_bit_and_run", loaded_weights_match_the_file_bit_for_bit_and_run}};
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
