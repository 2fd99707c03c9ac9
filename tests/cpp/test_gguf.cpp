// C++ API of the host GGUF code (agention-infer_amd/host/gguf.h), run by
// tests/test_host_cpp.py.  Exit 0 = all checks passed.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../agention-infer_amd/host/gguf.h"

using namespace gqh;
static int failures = 0;
#define CHECK(c)                                                          \
  do {                                                                    \
    if (!(c)) {                                                           \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #c); \
      failures++;                                                         \
    }                                                                     \
  } while (0)

struct Buf {
  std::vector<uint8_t> b;
  template <class T> void le(T v) {
    uint8_t t[sizeof(T)];
    std::memcpy(t, &v, sizeof(T));
    b.insert(b.end(), t, t + sizeof(T));
  }
  void str(const std::string &s) {
    le<uint64_t>(s.size());
    b.insert(b.end(), s.begin(), s.end());
  }
  void head(uint32_t version, uint64_t nt, uint64_t nkv) {
    b.insert(b.end(), {'G', 'G', 'U', 'F'});
    le(version);
    le(nt);
    le(nkv);
  }
};

template <class F>
static GgufError::Kind kind_of(F &&f) {
  try {
    f();
  } catch (const GgufError &e) {
    return e.kind();
  }
  return GgufError::Kind::BackendError;  // "no error" marker for the checks below
}

int main() {
  // block geometry (src/types.rs block_size / block_bytes / type_size)
  CHECK(type_size(GgmlType::Q4_K, 3584) == 14 * 144);
  CHECK(type_size(GgmlType::Q6_K, 18944) == 74 * 210);
  CHECK(type_size(GgmlType::Q8_0, 2048) == 64 * 34);
  CHECK(type_size(GgmlType::IQ3_XXS, 3072) == 12 * 98);
  CHECK(type_size(GgmlType::F16, 7) == 14 && type_size(GgmlType::Q8_K, 256) == 292);
  CHECK(std::strcmp(type_name(GgmlType::Q5_K), "Q5_K") == 0);
  CHECK(kind_of([] { ggml_type_from_u32(5); }) == GgufError::Kind::UnknownTensorType);
  CHECK(kind_of([] { ggml_type_from_u32(34); }) == GgufError::Kind::UnknownTensorType);

  // a file with metadata of several kinds and two tensors
  Buf f;
  f.head(3, 2, 5);
  f.str("general.architecture"); f.le<uint32_t>(8); f.str("qwen2");
  f.str("general.name"); f.le<uint32_t>(8); f.str("tiny");
  f.str("qwen2.context_length"); f.le<uint32_t>(4); f.le<uint32_t>(32768);
  f.str("qwen2.rope.freq_base"); f.le<uint32_t>(6); f.le<float>(1e6f);
  f.str("tokenizer.ggml.tokens"); f.le<uint32_t>(9); f.le<uint32_t>(8); f.le<uint64_t>(2);
  f.str("<s>"); f.str("hi");
  f.str("blk.0.ffn_down.weight"); f.le<uint32_t>(2); f.le<uint64_t>(512); f.le<uint64_t>(3);
  f.le<uint32_t>(14); f.le<uint64_t>(0);
  f.str("norm"); f.le<uint32_t>(1); f.le<uint64_t>(8); f.le<uint32_t>(0); f.le<uint64_t>(1280);
  const size_t head_len = f.b.size();
  GgufFile g = parse(f.b.data(), f.b.size());
  CHECK(g.version == 3 && g.tensor_count == 2 && g.metadata.size() == 5);
  CHECK(g.data_offset == (head_len + 31) / 32 * 32);
  CHECK(g.architecture() && *g.architecture() == "qwen2" && g.name() && *g.name() == "tiny");
  CHECK(g.get_u64("qwen2.context_length").value_or(0) == 32768);
  CHECK(g.get_f32("qwen2.rope.freq_base").value_or(0.f) == 1e6f);
  CHECK(!g.get_u64("general.name") && !g.get("absent"));
  auto toks = g.get_str_array("tokenizer.ggml.tokens");
  CHECK(toks && toks->size() == 2 && (*toks)[1] == "hi");
  CHECK(!g.get_i64_array("tokenizer.ggml.tokens"));
  CHECK(g.get("tokenizer.ggml.tokens")->display_value() == "Array(String, 2 items)");
  CHECK(g.get("qwen2.rope.freq_base")->display_value() == "1000000.000000");
  const TensorInfo *down = g.find("blk.0.ffn_down.weight");
  CHECK(down && down->ggml_type == GgmlType::Q6_K && down->n_elements() == 1536);
  CHECK(down->byte_size() == 6 * 210 && down->shape_str() == "[512, 3]");
  CHECK(g.total_tensor_bytes() == 6 * 210 + 32 && !g.find("missing"));

  // errors: truncations, version, magic
  for (size_t n = 0; n + 1 < head_len; n += 7)
    CHECK(kind_of([&] { parse(f.b.data(), n); }) == GgufError::Kind::UnexpectedEof);
  Buf v1;
  v1.head(1, 0, 0);
  CHECK(kind_of([&] { parse(v1.b.data(), v1.b.size()); }) == GgufError::Kind::UnsupportedVersion);
  std::vector<uint8_t> zeros(24, 0);
  CHECK(kind_of([&] { parse(zeros.data(), zeros.size()); }) == GgufError::Kind::InvalidMagic);
  try {
    parse(zeros.data(), zeros.size());
  } catch (const GgufError &e) {
    CHECK(std::string(e.what()) == "invalid GGUF magic bytes");
  }

  // load() + tensor_data() through a real mapping
  f.b.resize(g.data_offset + 1280 + 32, 0);
  for (size_t k = 0; k < 6 * 210; k++) f.b[g.data_offset + k] = (uint8_t)(k * 7 + 1);
  const char *path = "test_gguf_cpp.tmp.gguf";
  FILE *fp = std::fopen(path, "wb");
  std::fwrite(f.b.data(), 1, f.b.size(), fp);
  std::fclose(fp);
  {
    auto [gf, m] = load(path);
    CHECK(m.size() == f.b.size());
    const uint8_t *p = tensor_data(gf, m, *gf.find("blk.0.ffn_down.weight"));
    CHECK(p[0] == 1 && p[1] == 8 && p[6 * 210 - 1] == (uint8_t)((6 * 210 - 1) * 7 + 1));
    Mmap moved = std::move(m);
    CHECK(moved.size() == f.b.size() && m.data() == nullptr);
    TensorInfo past = *gf.find("norm");
    past.byte_offset = 1 << 20;
    CHECK(kind_of([&] { tensor_data(gf, moved, past); }) == GgufError::Kind::UnexpectedEof);
  }
  std::remove(path);
  CHECK(kind_of([] { load("no/such/file.gguf"); }) == GgufError::Kind::Io);

  CHECK(parse_split_index("a-00002-of-00003.gguf") == std::make_pair(size_t(2), size_t(3)));
  CHECK(!parse_split_index("a-0000x-of-00003.gguf") && !parse_split_index("a.gguf"));

  if (failures) std::fprintf(stderr, "%d check(s) failed\n", failures);
  else std::printf("all checks passed\n");
  return failures ? 1 : 0;
}
