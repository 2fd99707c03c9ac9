// model.cpp -- see model.h.
#include <climits>
#include "model.h"

#include <algorithm>
#include <cstring>
#include <map>

namespace gqh {
namespace {

[[noreturn]] void missing(const std::string &what) {
  throw GgufError(GgufError::Kind::MissingMetadata, "missing required metadata key: " + what);
}
[[noreturn]] void unsupported(const std::string &what) {
  throw GgufError(GgufError::Kind::BackendError,
                  "backend error: the GPU-resident decode does not cover " + what);
}
void check(int rc) {
  if (rc) throw GgufError(GgufError::Kind::BackendError, std::string("backend error: ") + gq_last_error());
}

// IEEE 754 binary16 -> binary32 (exact: every f16 is an f32).
float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  uint32_t bits;
  if (e == 0x1f) {
    bits = sign | 0x7f800000u | (m << 13);  // inf / nan
  } else if (e) {
    bits = sign | ((e + 112) << 23) | (m << 13);
  } else if (!m) {
    bits = sign;
  } else {  // subnormal: m * 2^-24, normalised
    int s = 0;
    uint32_t mm = m;
    while (!(mm & 0x400)) {
      mm <<= 1;
      s++;
    }
    bits = sign | ((uint32_t)(113 - s) << 23) | ((mm & 0x3ff) << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint64_t outer(const TensorInfo &t) {
  uint64_t n = 1;
  for (size_t i = 1; i < t.dims.size(); i++) n *= t.dims[i];
  return n;
}

}  // namespace

ModelConfig ModelConfig::from_gguf(const GgufFile &f) {
  ModelConfig c;
  auto arch = f.get_string("general.architecture");
  if (!arch) missing("general.architecture");
  c.architecture = std::string(*arch);
  auto key = [&](const char *field) { return c.architecture + "." + field; };
  auto hc = f.get_u64(key("attention.head_count"));
  if (!hc) missing(key("attention.head_count"));
  auto el = f.get_u64(key("embedding_length"));
  if (!el) missing(key("embedding_length"));
  c.head_count = *hc;
  c.embedding_length = *el;
  if (c.head_count == 0) missing(key("attention.head_count") + " (zero)");
  c.head_dim = f.get_u64(key("attention.key_length")).value_or(c.embedding_length / c.head_count);
  if (auto kv = f.get_u64(key("attention.head_count_kv"))) {
    c.head_count_kv = *kv;
  } else if (auto arr = f.get_i64_array(key("attention.head_count_kv"))) {
    int64_t mx = 0;
    for (int64_t v : *arr) mx = std::max(mx, v);
    c.head_count_kv = mx > 0 ? (uint64_t)mx : c.head_count;
  } else {
    c.head_count_kv = c.head_count;
  }
  const TensorInfo *embd = f.find("token_embd.weight");
  if (!embd) missing("token_embd.weight tensor");
  c.vocab_size = embd->n_dims >= 2 ? embd->dims[1] : embd->dims[0];
  c.context_length = f.get_u64(key("context_length")).value_or(4096);
  c.block_count = f.get_u64(key("block_count")).value_or(32);
  c.feed_forward_length = f.get_u64(key("feed_forward_length")).value_or(0);
  c.rope_freq_base = f.get_f32(key("rope.freq_base")).value_or(10000.f);
  if (auto s = f.get_string(key("rope.scaling.type"))) c.rope_scaling_type = std::string(*s);
  c.rope_scaling_factor = f.get_f32(key("rope.scaling.factor"));
  c.layer_norm_rms_epsilon = f.get_f32(key("attention.layer_norm_rms_epsilon")).value_or(1e-5f);
  return c;
}

std::vector<float> dequant_tensor(const TensorInfo &t, const uint8_t *bytes) {
  const size_t n = t.n_elements();
  std::vector<float> out(n);
  if (t.ggml_type == GgmlType::F32) {
    std::memcpy(out.data(), bytes, n * 4);
  } else if (t.ggml_type == GgmlType::F16) {
    for (size_t i = 0; i < n; i++) {
      uint16_t h;
      std::memcpy(&h, bytes + 2 * i, 2);
      out[i] = f16_to_f32(h);
    }
  } else if (gpu_dequant_type(t.ggml_type)) {
    const size_t in_dim = t.dims.empty() ? 0 : t.dims[0], rows = outer(t);
    if (!n) return out;
    if (in_dim > (size_t)INT_MAX || rows > (size_t)INT_MAX)
      throw GgufError(GgufError::Kind::BackendError,
                      "backend error: dequant: tensor " + t.name + " shape " + t.shape_str() +
                          " exceeds the backend's 2^31-1 rows/columns");
    gq_weight *w = nullptr;
    check(gq_upload((int)t.ggml_type, bytes, t.byte_size(), (int)in_dim, (int)rows, &w));
    GpuWeight hold(w);
    check(gq_dequant_rows_host(w, 0, (int)rows, out.data()));
  } else {
    throw GgufError(GgufError::Kind::BackendError,
                    std::string("backend error: dequant not implemented for ") + type_name(t.ggml_type));
  }
  return out;
}

std::unique_ptr<ResidentModel> ResidentModel::load(const GgufFile &f, const TensorBytes &bytes,
                                                   int ctx, int max_tokens,
                                                   const ReleaseBytes &release) {
  std::unique_ptr<ResidentModel> m(new ResidentModel());
  ModelConfig &c = m->cfg_ = ModelConfig::from_gguf(f);
  const std::string &st = c.rope_scaling_type.value_or("none");
  const bool unscaled = st.empty() || st == "none" ||
                        (st == "linear" && c.rope_scaling_factor.value_or(1.f) == 1.f);
  if (!unscaled) unsupported("RoPE scaling type " + st);
  auto need = [&](const std::string &name) -> const TensorInfo & {
    const TensorInfo *t = f.find(name);
    if (!t) missing("tensor " + name);
    return *t;
  };

  // Layer discovery (names as LlamaModel::new).
  const int L = (int)c.block_count;
  const uint64_t q_dim = c.head_count * c.head_dim;
  std::vector<std::string> names;  // matmul weights: 7 per layer, then lm_head
  for (int i = 0; i < L; i++) {
    const std::string b = "blk." + std::to_string(i) + ".";
    if (f.find(b + "shortconv.conv.weight")) unsupported("layer " + std::to_string(i) + "'s ShortConv mixer");
    if (f.find(b + "ssm_alpha.weight")) unsupported("layer " + std::to_string(i) + "'s GatedDeltaNet mixer");
    const TensorInfo &wq = need(b + "attn_q.weight");
    if (outer(wq) == 2 * q_dim) unsupported("layer " + std::to_string(i) + "'s GatedAttention mixer");
    if (f.find(b + "attn_q_norm.weight") || f.find(b + "attn_k_norm.weight"))
      unsupported("layer " + std::to_string(i) + "'s QK-norm");
    for (const char *s : {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"})
      names.push_back(b + s + ".weight");
  }
  const TensorInfo &embd = need("token_embd.weight");
  const bool tied = !f.find("output.weight");
  names.push_back(tied ? "token_embd.weight" : "output.weight");
  std::string out_norm = f.find("output_norm.weight") ? "output_norm.weight" : "token_embd_norm.weight";
  if (!f.find(out_norm)) missing("output_norm.weight or token_embd_norm.weight");

  // Upload in ascending file order; the pages behind are released.
  std::vector<const TensorInfo *> order;
  for (const std::string &n : names) {
    const TensorInfo &t = need(n);
    if (t.n_dims != 2 || !gpu_dequant_type(t.ggml_type))
      unsupported("tensor " + n + " (" + type_name(t.ggml_type) + ", " + t.shape_str() +
                  "): matmul weights must be 2-D Q8_0/Q4_K/Q5_K/Q6_K/IQ3_XXS");
    order.push_back(&t);
  }
  std::sort(order.begin(), order.end(),
            [](const TensorInfo *a, const TensorInfo *b) { return a->byte_offset < b->byte_offset; });
  order.erase(std::unique(order.begin(), order.end()), order.end());
  std::map<std::string, const gq_weight *> up;
  const HipBackend be;
  m->weights_.reserve(order.size());
  for (const TensorInfo *t : order) {
    const uint8_t *p = bytes(*t);
    m->weights_.push_back(be.upload_weight(t->ggml_type, p, t->byte_size(), (size_t)t->dims[0]));
    up[t->name] = m->weights_.back().get();
    if (release && !(tied && t == &embd)) release(p, t->byte_size());
  }

  // Norms and the f32 embedding table (copied to the device by gq_model_create).
  std::vector<std::vector<float>> an(L), fn(L);
  std::vector<const float *> anp(L), fnp(L);
  for (int i = 0; i < L; i++) {
    const std::string b = "blk." + std::to_string(i) + ".";
    an[i] = dequant_tensor(need(b + "attn_norm.weight"), bytes(need(b + "attn_norm.weight")));
    const std::string fnn = f.find(b + "ffn_norm.weight") ? b + "ffn_norm.weight" : b + "post_attention_norm.weight";
    fn[i] = dequant_tensor(need(fnn), bytes(need(fnn)));
    if (an[i].size() != c.embedding_length || fn[i].size() != c.embedding_length)
      unsupported("layer " + std::to_string(i) + "'s norm width");
    anp[i] = an[i].data();
    fnp[i] = fn[i].data();
  }
  const std::vector<float> onorm = dequant_tensor(need(out_norm), bytes(need(out_norm)));
  if (onorm.size() != c.embedding_length) unsupported(out_norm + "'s width");
  std::vector<float> table;
  if (tied) {
    table.resize(embd.n_elements());
    check(gq_dequant_rows_host(up["token_embd.weight"], 0, (int)outer(embd), table.data()));
    if (release) release(bytes(embd), embd.byte_size());
  } else {
    table = dequant_tensor(embd, bytes(embd));
    if (release) release(bytes(embd), embd.byte_size());
  }
  if (embd.dims[0] != c.embedding_length) unsupported("token_embd.weight of width " + std::to_string(embd.dims[0]));

  std::vector<const gq_weight *> w[7];
  for (int i = 0; i < L; i++)
    for (int k = 0; k < 7; k++) w[k].push_back(up[names[7 * i + k]]);
  const TensorInfo &gate0 = need("blk.0.ffn_gate.weight");
  m->ctx_ = ctx > 0 ? ctx : (int)std::min<uint64_t>(c.context_length, 65536);
  gq_model_desc d{};
  d.n_layers = L;
  d.hidden = (int)c.embedding_length;
  d.n_heads = (int)c.head_count;
  d.n_kv_heads = (int)c.head_count_kv;
  d.head_dim = (int)c.head_dim;
  d.ffn = (int)(c.feed_forward_length ? c.feed_forward_length : outer(gate0));
  d.vocab = (int)c.vocab_size;
  d.ctx = m->ctx_;
  d.max_tokens = max_tokens;
  d.eps = c.layer_norm_rms_epsilon;
  d.theta = c.rope_freq_base;
  d.wq = w[0].data(), d.wk = w[1].data(), d.wv = w[2].data(), d.wo = w[3].data();
  d.wgate = w[4].data(), d.wup = w[5].data(), d.wdown = w[6].data();
  d.lm_head = up[names.back()];
  d.attn_norm = anp.data();
  d.ffn_norm = fnp.data();
  d.output_norm = onorm.data();
  d.embd = table.data();
  check(gq_model_create(&d, &m->model_));  // checks every weight's shape
  return m;
}

ResidentModel::~ResidentModel() {
  if (model_) gq_model_free(model_);
}

size_t ResidentModel::device_weight_bytes() const {
  size_t n = 0;
  for (const GpuWeight &w : weights_) n += w.device_bytes();
  return n;
}

int ResidentModel::decode(int token, int pos, float *logits) {
  int next = -1;
  check(gq_model_decode(model_, token, pos, logits, &next));
  return next;
}

void ResidentModel::generate(int token, int pos, int n_steps, int *tokens) {
  check(gq_model_generate(model_, token, pos, n_steps, tokens, nullptr));
}

}  // namespace gqh
