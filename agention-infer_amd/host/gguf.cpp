// gguf.cpp -- see gguf.h.
#include "gguf.h"

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace gqh {

namespace {

// Block geometry per type: {elements, bytes}; {0, 0} for ids not in the format.
struct Geo {
  uint16_t elems, bytes;
};
constexpr Geo kGeo[34] = {
    {1, 4},    {1, 2},    {32, 18},  {32, 20},  {0, 0},    {0, 0},    {32, 22},  {32, 24},
    {32, 34},  {32, 40},  {256, 256}, {256, 110}, {256, 144}, {256, 176}, {256, 210}, {256, 292},
    {256, 66}, {256, 74}, {256, 98}, {256, 50}, {32, 18},  {256, 110}, {256, 82}, {256, 136},
    {1, 1},    {1, 2},    {1, 4},    {1, 8},    {1, 8},    {256, 56}, {1, 2},    {32, 18},
    {32, 18},  {32, 18},
};
constexpr const char *kNames[34] = {
    "F32",  "F16",  "Q4_0", "Q4_1", nullptr, nullptr, "Q5_0", "Q5_1", "Q8_0", "Q8_1", "Q2_K",
    "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_K", "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ1_S", "IQ4_NL",
    "IQ3_S", "IQ2_S", "IQ4_XS", "I8", "I16", "I32", "I64", "F64", "IQ1_M", "BF16", "Q4_0_4_4",
    "Q4_0_4_8", "Q4_0_8_8",
};

std::string fmt(const char *f, unsigned long long v) {
  char buf[160];
  std::snprintf(buf, sizeof buf, f, v);
  return buf;
}

// Bounds-checked little-endian reader over the file image.
class Reader {
 public:
  Reader(const uint8_t *p, size_t n) : p_(p), n_(n) {}
  size_t pos() const { return pos_; }
  const uint8_t *take(size_t k) {
    if (n_ - pos_ < k) throw GgufError(GgufError::Kind::UnexpectedEof,
                                       fmt("unexpected end of input at byte %llu", pos_), pos_);
    const uint8_t *r = p_ + pos_;
    pos_ += k;
    return r;
  }
  template <class T>
  T le() {
    const uint8_t *b = take(sizeof(T));
    uint64_t v = 0;
    for (size_t i = 0; i < sizeof(T); i++) v |= (uint64_t)b[i] << (8 * i);
    T out;
    if constexpr (sizeof(T) == 8) {
      std::memcpy(&out, &v, 8);
    } else {
      const uint32_t w = (uint32_t)v;
      if constexpr (sizeof(T) == 4) std::memcpy(&out, &w, 4);
      else if constexpr (sizeof(T) == 2) { const uint16_t h = (uint16_t)v; std::memcpy(&out, &h, 2); }
      else { const uint8_t c = (uint8_t)v; std::memcpy(&out, &c, 1); }
    }
    return out;
  }
  std::string str() {
    const uint64_t len = le<uint64_t>();
    if (len > n_ - pos_)
      throw GgufError(GgufError::Kind::UnexpectedEof,
                      fmt("unexpected end of input at byte %llu", pos_), pos_);
    const size_t at = pos_;
    const uint8_t *b = take((size_t)len);
    if (!valid_utf8(b, (size_t)len))
      throw GgufError(GgufError::Kind::InvalidString, fmt("invalid string at byte offset %llu", at), at);
    return std::string((const char *)b, (size_t)len);
  }

 private:
  static bool valid_utf8(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
      const uint8_t c = s[i];
      int extra;
      uint32_t cp;
      if (c < 0x80) { i++; continue; }
      if ((c & 0xE0) == 0xC0) { extra = 1; cp = c & 0x1F; }
      else if ((c & 0xF0) == 0xE0) { extra = 2; cp = c & 0x0F; }
      else if ((c & 0xF8) == 0xF0) { extra = 3; cp = c & 0x07; }
      else return false;
      if (n - i <= (size_t)extra) return false;
      for (int k = 1; k <= extra; k++) {
        if ((s[i + k] & 0xC0) != 0x80) return false;
        cp = (cp << 6) | (s[i + k] & 0x3F);
      }
      // overlong forms, surrogates and values past U+10FFFF are not UTF-8
      static const uint32_t kMin[4] = {0, 0x80, 0x800, 0x10000};
      if (cp < kMin[extra] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
      i += extra + 1;
    }
    return true;
  }
  const uint8_t *p_;
  size_t n_, pos_ = 0;
};

bool scalar_type(uint32_t t) { return t <= 12 && t != 9; }

MetadataValue read_value(Reader &r, uint32_t t) {
  MetadataValue v;
  if (t > 12) throw GgufError(GgufError::Kind::UnknownMetadataType,
                              fmt("unknown metadata value type: %llu", t), t);
  v.type = (MetaType)t;
  switch (v.type) {
  case MetaType::U8: v.u = r.le<uint8_t>(); break;
  case MetaType::I8: v.i = r.le<int8_t>(); break;
  case MetaType::U16: v.u = r.le<uint16_t>(); break;
  case MetaType::I16: v.i = r.le<int16_t>(); break;
  case MetaType::U32: v.u = r.le<uint32_t>(); break;
  case MetaType::I32: v.i = r.le<int32_t>(); break;
  case MetaType::F32: v.f = r.le<float>(); break;
  case MetaType::Bool: v.b = r.le<uint8_t>() != 0; break;
  case MetaType::String: v.s = r.str(); break;
  case MetaType::U64: v.u = r.le<uint64_t>(); break;
  case MetaType::I64: v.i = r.le<int64_t>(); break;
  case MetaType::F64: v.f = r.le<double>(); break;
  case MetaType::Array: {
    const uint32_t et = r.le<uint32_t>();
    if (!scalar_type(et))  // arrays of arrays are not part of the format
      throw GgufError(GgufError::Kind::UnknownMetadataType,
                      fmt("unknown metadata value type: %llu", et), et);
    v.elem = (MetaType)et;
    const uint64_t count = r.le<uint64_t>();
    // every element takes at least one byte: a count past the input is an EOF
    if (count > (uint64_t)SIZE_MAX / 2)
      throw GgufError(GgufError::Kind::UnexpectedEof,
                      fmt("unexpected end of input at byte %llu", r.pos()), r.pos());
    for (uint64_t k = 0; k < count; k++) v.items.push_back(read_value(r, et));
    break;
  }
  }
  return v;
}

}  // namespace

GgmlType ggml_type_from_u32(uint32_t v) {
  if (v >= 34 || !kNames[v])
    throw GgufError(GgufError::Kind::UnknownTensorType, fmt("unknown tensor GGML type: %llu", v), v);
  return (GgmlType)v;
}
size_t block_size(GgmlType t) { return kGeo[(uint32_t)t].elems; }
size_t block_bytes(GgmlType t) { return kGeo[(uint32_t)t].bytes; }
size_t type_size(GgmlType t, size_t n) {
  const size_t bs = block_size(t);
  return (n + bs - 1) / bs * block_bytes(t);
}
const char *type_name(GgmlType t) { return kNames[(uint32_t)t]; }

std::optional<uint64_t> MetadataValue::as_u64() const {
  switch (type) {
  case MetaType::U8: case MetaType::U16: case MetaType::U32: case MetaType::U64: return u;
  default: return std::nullopt;
  }
}
std::optional<int64_t> MetadataValue::as_i64() const {
  switch (type) {
  case MetaType::U8: case MetaType::U16: case MetaType::U32: case MetaType::U64: return (int64_t)u;
  case MetaType::I8: case MetaType::I16: case MetaType::I32: case MetaType::I64: return i;
  default: return std::nullopt;
  }
}
std::optional<float> MetadataValue::as_f32() const {
  if (type == MetaType::F32 || type == MetaType::F64) return (float)f;
  return std::nullopt;
}
std::optional<bool> MetadataValue::as_bool() const {
  if (type == MetaType::Bool) return b;
  return std::nullopt;
}
std::optional<std::string_view> MetadataValue::as_str() const {
  if (type == MetaType::String) return std::string_view(s);
  return std::nullopt;
}
const std::vector<MetadataValue> *MetadataValue::as_array() const {
  return type == MetaType::Array ? &items : nullptr;
}
std::string MetadataValue::display_value() const {
  static const char *kElem[13] = {"U8", "I8", "U16", "I16", "U32", "I32", "Float32", "Bool",
                                  "String", "Array", "U64", "I64", "Float64"};
  char buf[96];
  switch (type) {
  case MetaType::U8: case MetaType::U16: case MetaType::U32: case MetaType::U64:
    return std::to_string(u);
  case MetaType::I8: case MetaType::I16: case MetaType::I32: case MetaType::I64:
    return std::to_string(i);
  case MetaType::F32: case MetaType::F64:
    std::snprintf(buf, sizeof buf, "%.6f", f);
    return buf;
  case MetaType::Bool: return b ? "true" : "false";
  case MetaType::String: return s;
  case MetaType::Array:
    std::snprintf(buf, sizeof buf, "Array(%s, %zu items)", kElem[(int)elem], items.size());
    return buf;
  }
  return "";
}

size_t TensorInfo::n_elements() const {
  // parse() rejects shapes whose product overflows; saturate for tensors
  // built by other means
  size_t n = 1;
  for (uint64_t d : dims)
    if (__builtin_mul_overflow(n, (size_t)d, &n)) return SIZE_MAX;
  return n;
}
std::string TensorInfo::shape_str() const {
  std::string s = "[";
  for (size_t k = 0; k < dims.size(); k++) s += (k ? ", " : "") + std::to_string(dims[k]);
  return s + "]";
}

const MetadataValue *GgufFile::get(std::string_view key) const {
  auto it = metadata.find(std::string(key));
  return it == metadata.end() ? nullptr : &it->second;
}
std::optional<std::string_view> GgufFile::get_string(std::string_view key) const {
  const MetadataValue *v = get(key);
  return v ? v->as_str() : std::nullopt;
}
std::optional<uint64_t> GgufFile::get_u64(std::string_view key) const {
  const MetadataValue *v = get(key);
  return v ? v->as_u64() : std::nullopt;
}
std::optional<float> GgufFile::get_f32(std::string_view key) const {
  const MetadataValue *v = get(key);
  return v ? v->as_f32() : std::nullopt;
}
std::optional<bool> GgufFile::get_bool(std::string_view key) const {
  const MetadataValue *v = get(key);
  return v ? v->as_bool() : std::nullopt;
}
std::optional<std::vector<std::string_view>> GgufFile::get_str_array(std::string_view key) const {
  const MetadataValue *v = get(key);
  if (!v || !v->as_array()) return std::nullopt;
  std::vector<std::string_view> out;
  for (const MetadataValue &e : v->items) {
    auto s = e.as_str();
    if (!s) return std::nullopt;
    out.push_back(*s);
  }
  return out;
}
std::optional<std::vector<int64_t>> GgufFile::get_i64_array(std::string_view key) const {
  const MetadataValue *v = get(key);
  if (!v || !v->as_array()) return std::nullopt;
  std::vector<int64_t> out;
  for (const MetadataValue &e : v->items) {
    auto x = e.as_i64();
    if (!x) return std::nullopt;
    out.push_back(*x);
  }
  return out;
}
uint64_t GgufFile::total_tensor_bytes() const {
  uint64_t n = 0;
  for (const TensorInfo &t : tensors) n += t.byte_size();
  return n;
}
const TensorInfo *GgufFile::find(std::string_view tensor_name) const {
  for (const TensorInfo &t : tensors)
    if (t.name == tensor_name) return &t;
  return nullptr;
}

GgufFile parse(const uint8_t *data, size_t len) {
  Reader r(data, len);
  const uint8_t *magic = r.take(4);
  if (std::memcmp(magic, "GGUF", 4) != 0)
    throw GgufError(GgufError::Kind::InvalidMagic, "invalid GGUF magic bytes");
  GgufFile f;
  f.version = r.le<uint32_t>();
  if (f.version < 2 || f.version > 3)
    throw GgufError(GgufError::Kind::UnsupportedVersion,
                    fmt("unsupported GGUF version: %llu", f.version), f.version);
  f.tensor_count = r.le<uint64_t>();
  const uint64_t n_kv = r.le<uint64_t>();
  for (uint64_t k = 0; k < n_kv; k++) {
    std::string key = r.str();
    const uint32_t t = r.le<uint32_t>();
    f.metadata[std::move(key)] = read_value(r, t);  // a repeated key keeps the last value
  }
  for (uint64_t k = 0; k < f.tensor_count; k++) {
    TensorInfo t;
    t.name = r.str();
    t.n_dims = r.le<uint32_t>();
    if (t.n_dims > (len - r.pos()) / 8)  // each dim is 8 bytes
      throw GgufError(GgufError::Kind::UnexpectedEof,
                      fmt("unexpected end of input at byte %llu", r.pos()), r.pos());
    uint64_t prod = 1;
    bool wraps = false;
    for (uint32_t d = 0; d < t.n_dims; d++) {
      t.dims.push_back(r.le<uint64_t>());
      wraps |= __builtin_mul_overflow(prod, t.dims.back(), &prod);
    }
    // An element count past 2^64 cannot be backed by the input (the
    // reference's dims.product() would wrap and index the wrong bytes).
    if (wraps)
      throw GgufError(GgufError::Kind::UnexpectedEof,
                      fmt("unexpected end of input at byte %llu", r.pos()) + " (tensor " + t.name +
                          ": element count overflows)",
                      r.pos());
    t.ggml_type = ggml_type_from_u32(r.le<uint32_t>());
    t.byte_offset = r.le<uint64_t>();
    f.tensors.push_back(std::move(t));
  }
  f.data_offset = ((uint64_t)r.pos() + 31) & ~(uint64_t)31;
  return f;
}

Mmap::Mmap(const std::string &path) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0)
    throw GgufError(GgufError::Kind::Io, "I/O error: " + path + ": " + std::strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    ::close(fd);
    throw GgufError(GgufError::Kind::Io, "I/O error: " + path + ": " + std::strerror(e));
  }
  size_ = (size_t)st.st_size;
  if (size_ > 0) {
    void *p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      const int e = errno;
      ::close(fd);
      throw GgufError(GgufError::Kind::Io, "I/O error: " + path + ": " + std::strerror(e));
    }
    data_ = (const uint8_t *)p;
  }
  ::close(fd);
}
Mmap::Mmap(Mmap &&o) noexcept : data_(o.data_), size_(o.size_) {
  o.data_ = nullptr;
  o.size_ = 0;
}
Mmap &Mmap::operator=(Mmap &&o) noexcept {
  if (this != &o) {
    if (data_) munmap((void *)data_, size_);
    data_ = o.data_;
    size_ = o.size_;
    o.data_ = nullptr;
    o.size_ = 0;
  }
  return *this;
}
Mmap::~Mmap() {
  if (data_) munmap((void *)data_, size_);
}

std::pair<GgufFile, Mmap> load(const std::string &path) {
  Mmap m(path);
  GgufFile f = parse(m.data(), m.size());
  return {std::move(f), std::move(m)};
}

std::optional<std::pair<size_t, size_t>> parse_split_index(std::string_view name) {
  constexpr std::string_view ext = ".gguf";
  if (name.size() < ext.size() || name.substr(name.size() - ext.size()) != ext) return std::nullopt;
  name.remove_suffix(ext.size());
  const size_t of = name.rfind("-of-");
  if (of == std::string_view::npos) return std::nullopt;
  const std::string_view total = name.substr(of + 4), head = name.substr(0, of);
  const size_t dash = head.rfind('-');
  if (dash == std::string_view::npos) return std::nullopt;
  const std::string_view index = head.substr(dash + 1);
  auto num = [](std::string_view s) -> std::optional<size_t> {
    if (s.empty() || s.size() > 18) return std::nullopt;
    size_t v = 0;
    for (char c : s) {
      if (c < '0' || c > '9') return std::nullopt;
      v = v * 10 + (size_t)(c - '0');
    }
    return v;
  };
  auto i = num(index), t = num(total);
  if (!i || !t) return std::nullopt;
  return std::make_pair(*i, *t);
}

std::pair<GgufFile, MultiFileMmap> MultiFileMmap::load(const std::string &first) {
  auto [f, m0] = gqh::load(first);
  MultiFileMmap mm;
  const size_t slash = first.rfind('/');
  const std::string dir = slash == std::string::npos ? "" : first.substr(0, slash + 1);
  const std::string base = slash == std::string::npos ? first : first.substr(slash + 1);
  const size_t total = parse_split_index(base).value_or(std::make_pair(size_t(1), size_t(1))).second;
  uint64_t at = m0.size();
  mm.maps_.emplace_back(std::move(m0), 0);
  char from[32], to[32];
  std::snprintf(from, sizeof from, "-00001-of-%05zu", total);
  for (size_t k = 2; k <= total; k++) {
    std::snprintf(to, sizeof to, "-%05zu-of-%05zu", k, total);
    std::string name = base;
    const size_t p = name.find(from);
    if (p == std::string::npos)
      throw GgufError(GgufError::Kind::MultiFileMismatch,
                      "multi-file mismatch: " + base + " is not part 1 of " + std::to_string(total));
    name.replace(p, std::strlen(from), to);
    Mmap m(dir + name);
    const uint64_t sz = m.size();
    mm.maps_.emplace_back(std::move(m), at);
    at += sz;
  }
  return {std::move(f), std::move(mm)};
}

const uint8_t *MultiFileMmap::slice(uint64_t offset, size_t len) const {
  for (const auto &[m, start] : maps_)
    if (start <= offset && offset + len <= start + m.size()) return m.data() + (offset - start);
  return nullptr;
}

const uint8_t *tensor_data(const GgufFile &f, const Mmap &m, const TensorInfo &t) {
  const uint64_t at = f.data_offset + t.byte_offset, n = t.byte_size();
  if (at > m.size() || n > m.size() - at)
    throw GgufError(GgufError::Kind::UnexpectedEof,
                    fmt("unexpected end of input at byte %llu", m.size()), m.size());
  return m.data() + at;
}

}  // namespace gqh
