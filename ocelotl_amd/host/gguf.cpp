// gguf.cpp -- GGUF v3 inspection and tensor payload loading.  The header walk,
// limits and messages follow inspect_gguf (crates/loader/src/gguf_inspect.rs:
// 224-414, reader :422-665, alignment :665-705).
#include "gguf.hpp"

#include <cerrno>
#include <cstring>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

namespace ocelotl {

namespace {

constexpr char kMagic[4] = {'G', 'G', 'U', 'F'};
constexpr uint32_t kVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;
constexpr uint64_t kMaxMetadataEntries = 200000;
constexpr uint64_t kMaxTensors = 2000000;
constexpr uint64_t kMaxMetadataStringBytes = 16ull * 1024 * 1024;
constexpr uint64_t kMaxKeyBytes = 65535;
constexpr uint64_t kMaxTensorNameBytes = 65535;
constexpr uint64_t kMaxArrayElements = 2000000;
constexpr int kMaxArrayDepth = 4;
constexpr uint32_t kMaxTensorDims = 8;

OcelotlError invalid(const std::string &path, std::optional<std::string> field, std::string message) {
  return OcelotlError::invalid_model(path, std::move(field), std::move(message));
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t &out) {
  if (a != 0 && b > UINT64_MAX / a) return false;
  out = a * b;
  return true;
}

// UTF-8 structure check (lead byte, continuation bytes, no truncated
// sequence), as String::from_utf8 requires of metadata strings.
bool valid_utf8(const std::string &s) {
  const size_t n = s.size();
  size_t i = 0;
  while (i < n) {
    const unsigned char c = (unsigned char)s[i];
    size_t extra;
    if (c < 0x80) extra = 0;
    else if ((c >> 5) == 0x6) extra = 1;
    else if ((c >> 4) == 0xE) extra = 2;
    else if ((c >> 3) == 0x1E) extra = 3;
    else return false;
    if (extra && i + extra >= n) return false;
    for (size_t k = 1; k <= extra; ++k)
      if ((((unsigned char)s[i + k]) >> 6) != 0x2) return false;
    i += extra + 1;
  }
  return true;
}

// Sequential reader over the header region (GgufReader, gguf_inspect.rs:422-665).
class Reader {
 public:
  Reader(int fd, std::string path, uint64_t len) : fd_(fd), path_(std::move(path)), len_(len) {}
  uint64_t position() const { return pos_; }

  Result<void> read(void *buf, size_t n) {
    if (pos_ + n > len_) return invalid(path_, std::string("header"), "GGUF header is truncated");
    size_t done = 0;
    while (done < n) {
      const ssize_t r = pread(fd_, static_cast<char *>(buf) + done, n - done, (off_t)(pos_ + done));
      if (r < 0) {
        if (errno == EINTR) continue;
        return OcelotlError::io(path_, errno);
      }
      if (r == 0) return invalid(path_, std::string("header"), "GGUF header is truncated");
      done += (size_t)r;
    }
    pos_ += n;
    return {};
  }

  template <class T>
  Result<T> scalar() {  // little-endian host (x86-64, the only host this library runs on)
    T v{};
    Result<void> r = read(&v, sizeof v);
    if (r.is_err()) return r.error();
    return v;
  }

  Result<void> skip(uint64_t n) {
    uint64_t end;
    if (pos_ > UINT64_MAX - n)
      return invalid(path_, std::string("header"), "GGUF skip length " + std::to_string(n) + " overflows file offset");
    end = pos_ + n;
    if (end > len_)
      return invalid(path_, std::string("header"),
                     "GGUF metadata/tensor-info region is truncated: attempted to seek to " + std::to_string(end) +
                         ", file length is " + std::to_string(len_));
    pos_ = end;
    return {};
  }

  Result<uint64_t> string_len(const std::string &field, uint64_t max_len) {
    auto len = scalar<uint64_t>();
    if (len.is_err()) return len.error();
    if (len.value() > max_len || len.value() > kMaxMetadataStringBytes)
      return invalid(path_, field,
                     "GGUF " + field + " length " + std::to_string(len.value()) + " exceeds max " +
                         std::to_string(max_len));
    return len.value();
  }

  Result<std::string> string(const std::string &field, uint64_t max_len) {
    auto len = string_len(field, max_len);
    if (len.is_err()) return len.error();
    std::string s(len.value(), '\0');
    if (len.value()) {
      Result<void> r = read(&s[0], s.size());
      if (r.is_err()) return r.error();
    }
    if (!valid_utf8(s)) return invalid(path_, field, "GGUF " + field + " is not UTF-8");
    return s;
  }

  Result<GgufMetadataType> value_type(const std::string &field) {
    auto raw = scalar<uint32_t>();
    if (raw.is_err()) return raw.error();
    if (raw.value() > 12)
      return invalid(path_, field, "unknown GGUF metadata value type " + std::to_string(raw.value()));
    return static_cast<GgufMetadataType>(raw.value());
  }

  Result<GgufMetadataValue> value(GgufMetadataType t, int depth) {
    GgufMetadataValue v;
    v.type = t;
    switch (t) {
    case GgufMetadataType::U8: return num<uint8_t>(v, false);
    case GgufMetadataType::I8: return num<int8_t>(v, true);
    case GgufMetadataType::U16: return num<uint16_t>(v, false);
    case GgufMetadataType::I16: return num<int16_t>(v, true);
    case GgufMetadataType::U32: return num<uint32_t>(v, false);
    case GgufMetadataType::I32: return num<int32_t>(v, true);
    case GgufMetadataType::U64: return num<uint64_t>(v, false);
    case GgufMetadataType::I64: return num<int64_t>(v, true);
    case GgufMetadataType::F32: {
      auto x = scalar<float>();
      if (x.is_err()) return x.error();
      v.f = x.value();
      return v;
    }
    case GgufMetadataType::F64: {
      auto x = scalar<double>();
      if (x.is_err()) return x.error();
      v.f = x.value();
      return v;
    }
    case GgufMetadataType::Bool: {
      auto x = scalar<uint8_t>();
      if (x.is_err()) return x.error();
      if (x.value() > 1)
        return invalid(path_, std::string("bool"), "GGUF bool value must be 0 or 1, got " + std::to_string(x.value()));
      v.u = x.value();
      return v;
    }
    case GgufMetadataType::String: {
      auto x = string("metadata string", kMaxMetadataStringBytes);
      if (x.is_err()) return x.error();
      v.s = std::move(x.value());
      return v;
    }
    case GgufMetadataType::Array: {
      auto et = value_type("metadata array");
      if (et.is_err()) return et.error();
      auto len = scalar<uint64_t>();
      if (len.is_err()) return len.error();
      if (len.value() > kMaxArrayElements)
        return invalid(path_, std::string("metadata array"),
                       "GGUF metadata array length " + std::to_string(len.value()) + " exceeds max " +
                           std::to_string(kMaxArrayElements));
      if (depth >= kMaxArrayDepth)
        return invalid(path_, std::string("metadata array"),
                       "GGUF metadata array nesting exceeds max depth " + std::to_string(kMaxArrayDepth));
      for (uint64_t i = 0; i < len.value(); ++i) {
        Result<void> r = skip_value(et.value(), depth + 1);
        if (r.is_err()) return r.error();
      }
      v.element_type = et.value();
      v.len = len.value();
      return v;
    }
    }
    return invalid(path_, std::nullopt, "unreachable metadata type");
  }

 private:
  template <class T>
  Result<GgufMetadataValue> num(GgufMetadataValue v, bool is_signed) {
    auto x = scalar<T>();
    if (x.is_err()) return x.error();
    if (is_signed) v.i = (int64_t)x.value();
    else v.u = (uint64_t)x.value();
    return v;
  }

  Result<void> skip_value(GgufMetadataType t, int depth) {
    switch (t) {
    case GgufMetadataType::U8: case GgufMetadataType::I8: case GgufMetadataType::Bool: return skip(1);
    case GgufMetadataType::U16: case GgufMetadataType::I16: return skip(2);
    case GgufMetadataType::U32: case GgufMetadataType::I32: case GgufMetadataType::F32: return skip(4);
    case GgufMetadataType::U64: case GgufMetadataType::I64: case GgufMetadataType::F64: return skip(8);
    case GgufMetadataType::String: {
      auto len = string_len("metadata string", kMaxMetadataStringBytes);
      if (len.is_err()) return len.error();
      return skip(len.value());
    }
    case GgufMetadataType::Array: {
      if (depth >= kMaxArrayDepth)
        return invalid(path_, std::string("metadata array"),
                       "GGUF metadata array nesting exceeds max depth " + std::to_string(kMaxArrayDepth));
      auto et = value_type("metadata array");
      if (et.is_err()) return et.error();
      auto len = scalar<uint64_t>();
      if (len.is_err()) return len.error();
      if (len.value() > kMaxArrayElements)
        return invalid(path_, std::string("metadata array"),
                       "GGUF metadata array length " + std::to_string(len.value()) + " exceeds max " +
                           std::to_string(kMaxArrayElements));
      for (uint64_t i = 0; i < len.value(); ++i) {
        Result<void> r = skip_value(et.value(), depth + 1);
        if (r.is_err()) return r;
      }
      return {};
    }
    }
    return {};
  }

  int fd_;
  std::string path_;
  uint64_t len_;
  uint64_t pos_ = 0;
};

struct Fd {
  int fd = -1;
  ~Fd() {
    if (fd >= 0) close(fd);
  }
};

Result<uint64_t> alignment_from_metadata(const std::string &path, const std::vector<GgufMetadataEntry> &md) {
  uint64_t a = kDefaultAlignment;
  for (const GgufMetadataEntry &e : md) {
    if (e.key != "general.alignment") continue;
    if (e.value.type == GgufMetadataType::U32 || e.value.type == GgufMetadataType::U64) a = e.value.u;
    else
      return invalid(path, std::string("general.alignment"),
                     "GGUF general.alignment must be uint32 or uint64, got metadata type " +
                         std::to_string((uint32_t)e.value.type));
    break;
  }
  if (a == 0 || a % 8 != 0)
    return invalid(path, std::string("general.alignment"),
                   "GGUF alignment must be a positive multiple of 8, got " + std::to_string(a));
  return a;
}

// Block formats with a known layout: raw id, name, elements and bytes per block.
struct BlockFormat {
  uint32_t type;
  const char *name;
  uint64_t elems, bytes;
};
constexpr BlockFormat kBlockFormats[] = {{2, "Q4_0", 32, 18},   {3, "Q4_1", 32, 20},   {6, "Q5_0", 32, 22},
                                         {7, "Q5_1", 32, 24},   {8, "Q8_0", 32, 34},   {10, "Q2_K", 256, 84},
                                         {11, "Q3_K", 256, 110}, {12, "Q4_K", 256, 144}, {13, "Q5_K", 256, 176},
                                         {14, "Q6_K", 256, 210}};

const BlockFormat *block_format(uint32_t t) {
  for (const BlockFormat &f : kBlockFormats)
    if (f.type == t) return &f;
  return nullptr;
}

const std::vector<std::string> &block_format_names() {
  static const std::vector<std::string> v = {"Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0",
                                             "Q2K",  "Q3K",  "Q4K",  "Q5K",  "Q6K"};
  return v;
}

}  // namespace

const GgufMetadataValue *GgufManifest::metadata_value(const std::string &key) const {
  for (const GgufMetadataEntry &e : metadata)
    if (e.key == key) return &e.value;
  return nullptr;
}

const GgufTensorEntry *GgufManifest::tensor(const std::string &name) const {
  for (const GgufTensorEntry &t : tensors)
    if (t.name == name) return &t;
  return nullptr;
}

ByteLen gguf_byte_len(uint32_t type, const std::vector<uint64_t> &shape) {
  uint64_t count = 1;
  for (uint64_t d : shape)
    if (!mul_ok(count, d, count)) return {std::nullopt, "element count overflows u64"};
  uint64_t elem = 0;
  switch (type) {
  case 0: case 26: elem = 4; break;   // F32, I32
  case 1: case 30: case 25: elem = 2; break;  // F16, BF16, I16
  case 24: elem = 1; break;           // I8
  case 27: case 28: elem = 8; break;  // I64, F64
  default: break;
  }
  uint64_t out;
  if (elem) {
    if (!mul_ok(count, elem, out)) return {std::nullopt, "byte length overflows u64"};
    return {out, ""};
  }
  const BlockFormat *bf = block_format(type);
  if (!bf) return {std::nullopt, ""};  // Q8_1, Q8_K, the IQ and TQ formats: layout not known here
  if (shape.empty() || shape[0] % bf->elems != 0)
    return {std::nullopt, std::string("row of ") + std::to_string(shape.empty() ? 0 : shape[0]) +
                              " elements is not a multiple of the " + bf->name + " block size " +
                              std::to_string(bf->elems)};
  if (!mul_ok(count / bf->elems, bf->bytes, out)) return {std::nullopt, "byte length overflows u64"};
  return {out, ""};
}

Result<GgufManifest> inspect_gguf(const std::string &path) {
  Fd f;
  f.fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (f.fd < 0) return OcelotlError::io(path, errno);
  struct stat st;
  if (fstat(f.fd, &st) != 0) return OcelotlError::io(path, errno);
  GgufManifest m;
  m.file_len = (uint64_t)st.st_size;
  Reader rd(f.fd, path, m.file_len);

  char magic[4];
  Result<void> r = rd.read(magic, 4);
  if (r.is_err()) return r.error();
  if (std::memcmp(magic, kMagic, 4) != 0) {
    char buf[96];
    std::snprintf(buf, sizeof buf, "invalid GGUF magic bytes: [%u, %u, %u, %u]", (unsigned char)magic[0],
                  (unsigned char)magic[1], (unsigned char)magic[2], (unsigned char)magic[3]);
    return invalid(path, std::string("magic"), buf);
  }
  auto version = rd.scalar<uint32_t>();
  if (version.is_err()) return version.error();
  if (version.value() != kVersion)
    return OcelotlError::unsupported("gguf_version", std::to_string(version.value()), {std::to_string(kVersion)});
  m.version = version.value();
  auto tensor_count = rd.scalar<uint64_t>();
  if (tensor_count.is_err()) return tensor_count.error();
  auto metadata_count = rd.scalar<uint64_t>();
  if (metadata_count.is_err()) return metadata_count.error();
  if (tensor_count.value() > kMaxTensors)
    return invalid(path, std::string("tensor_count"),
                   "GGUF tensor_count " + std::to_string(tensor_count.value()) + " exceeds max " +
                       std::to_string(kMaxTensors));
  if (metadata_count.value() > kMaxMetadataEntries)
    return invalid(path, std::string("metadata_kv_count"),
                   "GGUF metadata_kv_count " + std::to_string(metadata_count.value()) + " exceeds max " +
                       std::to_string(kMaxMetadataEntries));

  for (uint64_t i = 0; i < metadata_count.value(); ++i) {
    auto key = rd.string("metadata key", kMaxKeyBytes);
    if (key.is_err()) return key.error();
    auto t = rd.value_type(key.value());
    if (t.is_err()) return t.error();
    auto v = rd.value(t.value(), 0);
    if (v.is_err()) return v.error();
    m.metadata.push_back({std::move(key.value()), std::move(v.value())});
  }
  auto alignment = alignment_from_metadata(path, m.metadata);
  if (alignment.is_err()) return alignment.error();
  m.alignment = alignment.value();

  for (uint64_t i = 0; i < tensor_count.value(); ++i) {
    GgufTensorEntry t;
    auto name = rd.string("tensor name", kMaxTensorNameBytes);
    if (name.is_err()) return name.error();
    t.name = std::move(name.value());
    auto n_dims = rd.scalar<uint32_t>();
    if (n_dims.is_err()) return n_dims.error();
    if (n_dims.value() == 0 || n_dims.value() > kMaxTensorDims)
      return invalid(path, t.name,
                     "GGUF tensor `" + t.name + "` has unsupported dimension count " + std::to_string(n_dims.value()));
    uint64_t count = 1;
    for (uint32_t d = 0; d < n_dims.value(); ++d) {
      auto dim = rd.scalar<uint64_t>();
      if (dim.is_err()) return dim.error();
      if (dim.value() == 0) return invalid(path, t.name, "GGUF tensor `" + t.name + "` has a zero dimension");
      if (!mul_ok(count, dim.value(), count))
        return invalid(path, t.name, "GGUF tensor `" + t.name + "` element count overflows u64");
      t.shape.push_back(dim.value());
    }
    auto type = rd.scalar<uint32_t>();
    if (type.is_err()) return type.error();
    t.tensor_type = type.value();
    auto offset = rd.scalar<uint64_t>();
    if (offset.is_err()) return offset.error();
    t.offset = offset.value();
    if (t.offset % m.alignment != 0)
      return invalid(path, t.name,
                     "GGUF tensor `" + t.name + "` offset " + std::to_string(t.offset) + " is not aligned to " +
                         std::to_string(m.alignment) + " bytes");
    ByteLen bl = gguf_byte_len(t.tensor_type, t.shape);
    if (!bl.error.empty()) return invalid(path, t.name, "GGUF tensor `" + t.name + "` " + bl.error);
    t.byte_len = bl.bytes;
    m.tensors.push_back(std::move(t));
  }

  const uint64_t info_end = rd.position();
  const uint64_t rem = info_end % m.alignment;
  if (rem != 0 && info_end > UINT64_MAX - (m.alignment - rem))
    return invalid(path, std::string("alignment"), "GGUF aligned offset overflows u64");
  m.data_start = rem == 0 ? info_end : info_end + (m.alignment - rem);
  if (m.data_start > m.file_len)
    return invalid(path, std::string("tensor_data"),
                   "GGUF tensor data section starts at " + std::to_string(m.data_start) + ", beyond file length " +
                       std::to_string(m.file_len));
  for (GgufTensorEntry &t : m.tensors) {
    if (t.offset > UINT64_MAX - m.data_start)
      return invalid(path, t.name, "GGUF tensor `" + t.name + "` file offset overflows u64");
    const uint64_t fo = m.data_start + t.offset;
    if (fo > m.file_len)
      return invalid(path, t.name,
                     "GGUF tensor `" + t.name + "` starts at file offset " + std::to_string(fo) +
                         ", beyond file length " + std::to_string(m.file_len));
    if (t.byte_len) {
      if (*t.byte_len > UINT64_MAX - fo)
        return invalid(path, t.name, "GGUF tensor `" + t.name + "` end offset overflows u64");
      const uint64_t end = fo + *t.byte_len;
      if (end > m.file_len)
        return invalid(path, t.name,
                       "GGUF tensor `" + t.name + "` byte range " + std::to_string(fo) + ".." + std::to_string(end) +
                           " exceeds file length " + std::to_string(m.file_len));
    }
    t.file_offset = fo;
  }
  return m;
}

Result<std::vector<uint8_t>> read_tensor_bytes(const std::string &path, const GgufManifest &manifest,
                                               const GgufTensorEntry &entry) {
  if (!entry.byte_len)
    return OcelotlError::unsupported("quantized_tensor_type", std::to_string(entry.tensor_type),
                                     block_format_names());
  (void)manifest;
  Fd f;
  f.fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (f.fd < 0) return OcelotlError::io(path, errno);
  std::vector<uint8_t> buf(*entry.byte_len);
  size_t done = 0;
  while (done < buf.size()) {
    const ssize_t r = pread(f.fd, buf.data() + done, buf.size() - done, (off_t)(entry.file_offset + done));
    if (r < 0) {
      if (errno == EINTR) continue;
      return OcelotlError::io(path, errno);
    }
    if (r == 0)
      return invalid(path, entry.name, "GGUF tensor `" + entry.name + "` payload is truncated");
    done += (size_t)r;
  }
  return buf;
}

Result<QuantizedWeight> load_quantized_weight(const HipKernelBackend &backend, const std::string &path,
                                              const GgufManifest &manifest, const std::string &name) {
  const GgufTensorEntry *t = manifest.tensor(name);
  if (!t) return invalid(path, name, "GGUF tensor `" + name + "` not found");
  if (!block_format(t->tensor_type))
    return OcelotlError::unsupported("quantized_tensor_type", std::to_string(t->tensor_type), block_format_names());
  uint64_t ne1 = 1;
  for (size_t d = 1; d < t->shape.size(); ++d) ne1 *= t->shape[d];  // no overflow: checked by inspect_gguf
  auto bytes = read_tensor_bytes(path, manifest, *t);
  if (bytes.is_err()) return bytes.error();
  return backend.upload_quantized(static_cast<GgmlTensorType>(t->tensor_type), (size_t)t->shape[0], (size_t)ne1,
                                  bytes.value().data(), bytes.value().size());
}

}  // namespace ocelotl
