// ModelConfig::from_gguf (agention-infer_amd/host/model.h) on the CPU, with the
// reference's rules (src/model/mod.rs:212-272).  Run by tests/test_host_cpp.py.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../agention-infer_amd/host/model.h"

using namespace gqh;
static int failures = 0;
#define CHECK(c)                                                                 \
  do {                                                                           \
    if (!(c)) {                                                                  \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #c); \
      failures++;                                                                \
    }                                                                            \
  } while (0)

namespace {
MetadataValue u(uint64_t v) {
  MetadataValue m;
  m.type = MetaType::U32;
  m.u = v;
  return m;
}
MetadataValue fl(float v) {
  MetadataValue m;
  m.type = MetaType::F32;
  m.f = v;
  return m;
}
MetadataValue s(const char *v) {
  MetadataValue m;
  m.type = MetaType::String;
  m.s = v;
  return m;
}
MetadataValue arr_i32(std::vector<int64_t> xs) {
  MetadataValue m;
  m.type = MetaType::Array;
  m.elem = MetaType::I32;
  for (int64_t x : xs) {
    MetadataValue e;
    e.type = MetaType::I32;
    e.i = x;
    m.items.push_back(e);
  }
  return m;
}
TensorInfo tensor(const char *name, std::vector<uint64_t> dims) {
  TensorInfo t;
  t.name = name;
  t.n_dims = (uint32_t)dims.size();
  t.dims = dims;
  t.ggml_type = GgmlType::Q4_K;
  return t;
}
}  // namespace

int main() {
  GgufFile f;
  f.metadata.emplace("general.architecture", s("qwen2"));
  f.metadata.emplace("qwen2.attention.head_count", u(28));
  f.metadata.emplace("qwen2.embedding_length", u(3584));
  f.tensors.push_back(tensor("token_embd.weight", {3584, 152064}));
  ModelConfig c = ModelConfig::from_gguf(f);
  CHECK(c.architecture == "qwen2" && c.head_count == 28 && c.embedding_length == 3584);
  CHECK(c.head_dim == 128);               // embedding_length / head_count
  CHECK(c.head_count_kv == 28);           // defaults to head_count
  CHECK(c.vocab_size == 152064);          // token_embd's outer dim
  CHECK(c.context_length == 4096 && c.block_count == 32 && c.feed_forward_length == 0);
  CHECK(c.rope_freq_base == 10000.f && c.layer_norm_rms_epsilon == 1e-5f);
  CHECK(!c.rope_scaling_type && !c.rope_scaling_factor);

  f.metadata.emplace("qwen2.attention.key_length", u(64));
  f.metadata.emplace("qwen2.attention.head_count_kv", arr_i32({0, 4, 0, 8, 2}));
  f.metadata.emplace("qwen2.rope.freq_base", fl(1e6f));
  f.metadata.emplace("qwen2.rope.scaling.type", s("linear"));
  f.metadata.emplace("qwen2.rope.scaling.factor", fl(2.f));
  f.metadata.emplace("qwen2.attention.layer_norm_rms_epsilon", fl(1e-6f));
  f.metadata.emplace("qwen2.context_length", u(32768));
  f.metadata.emplace("qwen2.block_count", u(28));
  f.metadata.emplace("qwen2.feed_forward_length", u(18944));
  c = ModelConfig::from_gguf(f);
  CHECK(c.head_dim == 64);                // attention.key_length wins
  CHECK(c.head_count_kv == 8);            // the largest per-layer entry
  CHECK(c.rope_freq_base == 1e6f && c.layer_norm_rms_epsilon == 1e-6f);
  CHECK(c.rope_scaling_type && *c.rope_scaling_type == "linear" && *c.rope_scaling_factor == 2.f);
  CHECK(c.context_length == 32768 && c.block_count == 28 && c.feed_forward_length == 18944);
  CHECK(c.gqa_group_size() == 3);

  // a 1-D token_embd gives dims[0]; missing keys are MissingMetadata
  GgufFile g;
  g.metadata.emplace("general.architecture", s("llama"));
  g.metadata.emplace("llama.attention.head_count", u(4));
  g.metadata.emplace("llama.embedding_length", u(256));
  g.tensors.push_back(tensor("token_embd.weight", {777}));
  CHECK(ModelConfig::from_gguf(g).vocab_size == 777);
  for (const char *drop : {"general.architecture", "llama.attention.head_count", "llama.embedding_length"}) {
    GgufFile h = g;
    h.metadata.erase(drop);
    try {
      ModelConfig::from_gguf(h);
      CHECK(!"expected MissingMetadata");
    } catch (const GgufError &e) {
      CHECK(e.kind() == GgufError::Kind::MissingMetadata);
      CHECK(std::strstr(e.what(), drop) != nullptr);
    }
  }
  GgufFile h = g;
  h.tensors.clear();
  try {
    ModelConfig::from_gguf(h);
    CHECK(!"expected MissingMetadata");
  } catch (const GgufError &e) {
    CHECK(std::strstr(e.what(), "token_embd.weight") != nullptr);
  }

  // F32 / F16 tensors dequantize on the host
  TensorInfo t16 = tensor("n", {4});
  t16.ggml_type = GgmlType::F16;
  const uint16_t h16[4] = {0x3c00, 0xc000, 0x0001, 0x7bff};  // 1, -2, 2^-24, 65504
  std::vector<float> v = dequant_tensor(t16, (const uint8_t *)h16);
  CHECK(v.size() == 4 && v[0] == 1.f && v[1] == -2.f && v[2] == 5.9604644775390625e-8f && v[3] == 65504.f);
  TensorInfo t32 = tensor("n", {2});
  t32.ggml_type = GgmlType::F32;
  const float f32[2] = {0.5f, -3.25f};
  v = dequant_tensor(t32, (const uint8_t *)f32);
  CHECK(v.size() == 2 && v[0] == 0.5f && v[1] == -3.25f);

  if (failures) std::fprintf(stderr, "%d check(s) failed\n", failures);
  else std::printf("all checks passed\n");
  return failures ? 1 : 0;
}
