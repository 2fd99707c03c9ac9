// gguf.h -- GGUF container parsing and memory-mapped loading (host C++).
//
// Mirrors the reference's parser and loader for the hot path's data format:
// parser::parse (src/parser.rs:9-66), loader::load / parse_split_index /
// MultiFileMmap (src/loader.rs:14-86), and the types they produce
// (GgmlType, MetadataValue, TensorInfo, GgufFile: src/types.rs).  Errors are
// thrown as GgufError with the reference's kinds and messages
// (src/error.rs:4-42).  Tensor bytes are never copied here: they are viewed
// in the mapping and handed to gq_upload once (see hip_backend.h).
#pragma once
#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>
#include <utility>
#include <vector>

namespace gqh {

class GgufError : public std::runtime_error {
 public:
  enum class Kind {
    InvalidMagic,
    UnsupportedVersion,
    UnexpectedEof,
    UnknownMetadataType,
    UnknownTensorType,
    InvalidString,
    MissingMetadata,
    WrongMetadataType,
    UnsupportedArchitecture,
    MultiFileMismatch,
    Io,
    BackendError,
  };
  GgufError(Kind k, std::string msg, uint64_t value = 0)
      : std::runtime_error(std::move(msg)), kind_(k), value_(value) {}
  Kind kind() const { return kind_; }
  uint64_t value() const { return value_; }  // the version / byte offset / type id, if any

 private:
  Kind kind_;
  uint64_t value_;
};

// GGML tensor types (ids as in the file format).
enum class GgmlType : uint32_t {
  F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q8_1 = 9,
  Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15,
  IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18, IQ1_S = 19, IQ4_NL = 20, IQ3_S = 21, IQ2_S = 22,
  IQ4_XS = 23, I8 = 24, I16 = 25, I32 = 26, I64 = 27, F64 = 28, IQ1_M = 29, BF16 = 30,
  Q4_0_4_4 = 31, Q4_0_4_8 = 32, Q4_0_8_8 = 33,
};
GgmlType ggml_type_from_u32(uint32_t v);  // throws UnknownTensorType
size_t block_size(GgmlType t);             // elements per block
size_t block_bytes(GgmlType t);            // bytes per block
size_t type_size(GgmlType t, size_t n);    // bytes of n elements (whole blocks)
const char *type_name(GgmlType t);

// Metadata value types (ids as in the file format; 9 = array).
enum class MetaType : uint32_t {
  U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, Bool = 7, String = 8, Array = 9,
  U64 = 10, I64 = 11, F64 = 12,
};

struct MetadataValue {
  MetaType type = MetaType::U8;
  MetaType elem = MetaType::U8;  // arrays: element type
  uint64_t u = 0;                // unsigned integers
  int64_t i = 0;                 // signed integers
  double f = 0.0;                // F32 (widened) and F64
  bool b = false;
  std::string s;
  std::vector<MetadataValue> items;  // arrays

  uint32_t type_id() const { return (uint32_t)type; }
  std::optional<uint64_t> as_u64() const;  // unsigned kinds only
  std::optional<int64_t> as_i64() const;   // every integer kind
  std::optional<float> as_f32() const;     // F32 and F64
  std::optional<bool> as_bool() const;
  std::optional<std::string_view> as_str() const;
  const std::vector<MetadataValue> *as_array() const;
  std::string display_value() const;
};

struct TensorInfo {
  std::string name;
  uint32_t n_dims = 0;
  std::vector<uint64_t> dims;  // dims[0] is the fastest (in_dim of a weight)
  GgmlType ggml_type = GgmlType::F32;
  uint64_t byte_offset = 0;  // from the data section start

  size_t n_elements() const;
  size_t byte_size() const { return type_size(ggml_type, n_elements()); }
  std::string shape_str() const;
};

struct GgufFile {
  uint32_t version = 0;
  uint64_t tensor_count = 0;
  std::unordered_map<std::string, MetadataValue> metadata;
  std::vector<TensorInfo> tensors;
  uint64_t data_offset = 0;  // 32-byte aligned start of the tensor data

  const MetadataValue *get(std::string_view key) const;
  std::optional<std::string_view> get_string(std::string_view key) const;
  std::optional<uint64_t> get_u64(std::string_view key) const;
  std::optional<float> get_f32(std::string_view key) const;
  std::optional<bool> get_bool(std::string_view key) const;
  std::optional<std::vector<std::string_view>> get_str_array(std::string_view key) const;
  std::optional<std::vector<int64_t>> get_i64_array(std::string_view key) const;
  std::optional<std::string_view> architecture() const { return get_string("general.architecture"); }
  std::optional<std::string_view> name() const { return get_string("general.name"); }
  uint64_t total_tensor_bytes() const;
  const TensorInfo *find(std::string_view tensor_name) const;
};

// Parse a GGUF image held in memory (versions 2 and 3).  No I/O.
GgufFile parse(const uint8_t *data, size_t len);

// A read-only private mapping of a whole file (moved, not copied).
class Mmap {
 public:
  Mmap() = default;
  explicit Mmap(const std::string &path);  // throws Io
  Mmap(Mmap &&o) noexcept;
  Mmap &operator=(Mmap &&o) noexcept;
  Mmap(const Mmap &) = delete;
  Mmap &operator=(const Mmap &) = delete;
  ~Mmap();
  const uint8_t *data() const { return data_; }
  size_t size() const { return size_; }

 private:
  const uint8_t *data_ = nullptr;
  size_t size_ = 0;
};

// Map and parse one file.
std::pair<GgufFile, Mmap> load(const std::string &path);

// "name-00002-of-00005.gguf" -> (2, 5), 1-based; nullopt for other names.
std::optional<std::pair<size_t, size_t>> parse_split_index(std::string_view file_name);

// The files of a split model: only the first holds the header; tensor
// offsets run on through the following files.
class MultiFileMmap {
 public:
  static std::pair<GgufFile, MultiFileMmap> load(const std::string &first_file_path);
  // Bytes [offset, offset + len) of the concatenated files, if they lie in
  // one file; nullptr otherwise.
  const uint8_t *slice(uint64_t offset, size_t len) const;
  size_t file_count() const { return maps_.size(); }

 private:
  std::vector<std::pair<Mmap, uint64_t>> maps_;  // (mapping, first byte's global offset)
};

// The bytes of a tensor in a single mapped file (checked against its size).
const uint8_t *tensor_data(const GgufFile &f, const Mmap &m, const TensorInfo &t);

}  // namespace gqh
