// model.h -- a dense Llama/Qwen2-style decoder loaded from a GGUF file onto
// the GPU and decoded there (gq_model_*, include/gq.h).
//
// ModelConfig::from_gguf follows ModelConfig::from_gguf (src/model/mod.rs:
// 212-272): the architecture prefix, head_dim from attention.key_length or
// embedding_length / head_count, head_count_kv as a scalar or the largest
// entry of a per-layer array, vocab from token_embd.weight's outer dim, and
// the same defaults.  ResidentModel::load follows LlamaModel::new's layer
// discovery (src/model/llama/mod.rs:130-300: blk.N.* names, output_norm or
// token_embd_norm, lm_head tied to token_embd when output.weight is absent)
// and pre_upload_gpu (src/model/llama/gpu_resident.rs:69-229: every matmul
// weight uploaded once, in ascending file order, the mapped pages released
// behind the upload).  The GPU-resident decode covers the Attention mixer
// without QK-norm and unscaled (or linear factor 1) RoPE; a file holding
// another mixer (ShortConv, GatedAttention, GatedDeltaNet), QK-norm weights
// or RoPE scaling is refused with BackendError naming what is missing.
#pragma once
#include <cstdint>
#include <functional>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "gguf.h"
#include "hip_backend.h"

namespace gqh {

struct ModelConfig {
  std::string architecture;
  uint64_t context_length = 4096, embedding_length = 0, block_count = 32, head_count = 0,
           head_count_kv = 0, head_dim = 0, feed_forward_length = 0, vocab_size = 0;
  float rope_freq_base = 10000.f;
  std::optional<std::string> rope_scaling_type;
  std::optional<float> rope_scaling_factor;
  float layer_norm_rms_epsilon = 1e-5f;

  static ModelConfig from_gguf(const GgufFile &f);  // throws MissingMetadata
  uint64_t gqa_group_size() const { return head_count / head_count_kv; }
};

// The bytes of a tensor (size t.byte_size()), and an optional hint that a
// tensor's bytes will not be read again (for file mappings).
using TensorBytes = std::function<const uint8_t *(const TensorInfo &)>;
using ReleaseBytes = std::function<void(const uint8_t *, size_t)>;

// A 1-D tensor (norm weight) or the rows of a 2-D tensor as f32: F32 and F16
// are converted on the host; quantized types go through the GPU dequant
// (gq_dequant_rows_host), which is bit-identical to the CPU dequant.
std::vector<float> dequant_tensor(const TensorInfo &t, const uint8_t *bytes);

class ResidentModel {
 public:
  // ctx: positions of the KV cache (0: the file's context_length);
  // max_tokens: tokens one generate() call may produce.
  static std::unique_ptr<ResidentModel> load(const GgufFile &f, const TensorBytes &bytes,
                                             int ctx = 0, int max_tokens = 4096,
                                             const ReleaseBytes &release = nullptr);
  ~ResidentModel();
  ResidentModel(const ResidentModel &) = delete;
  ResidentModel &operator=(const ResidentModel &) = delete;

  const ModelConfig &config() const { return cfg_; }
  int ctx() const { return ctx_; }
  gq_model *handle() const { return model_; }
  size_t device_weight_bytes() const;

  int decode(int token, int pos, float *logits = nullptr);  // returns the greedy next token
  void generate(int token, int pos, int n_steps, int *tokens);

 private:
  ResidentModel() = default;
  ModelConfig cfg_;
  int ctx_ = 0;
  std::vector<GpuWeight> weights_;  // outlive model_
  gq_model *model_ = nullptr;
};

}  // namespace gqh
