// gqh_capi.cpp -- the C ABI of include/gq_host.h over gguf.h / hip_backend.h.
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/gq_host.h"
#include "gguf.h"
#include "hip_backend.h"
#include "model.h"

#include <sys/mman.h>
#include <unistd.h>

struct gqh_model {
  std::unique_ptr<gqh::ResidentModel> m;
};

struct gqh_gguf {
  gqh::GgufFile file;
  gqh::MultiFileMmap maps;          // opened from a path
  std::vector<uint8_t> owned;       // parsed from a caller's buffer
  const uint8_t *single = nullptr;  // the one image, when not split
  size_t single_len = 0;
};

namespace {
thread_local std::string g_err;

int code(const gqh::GgufError &e) {
  using K = gqh::GgufError::Kind;
  switch (e.kind()) {
  case K::InvalidMagic: return GQH_EINVALID_MAGIC;
  case K::UnsupportedVersion: return GQH_EVERSION;
  case K::UnexpectedEof: return GQH_EEOF;
  case K::UnknownMetadataType: return GQH_EMETA_TYPE;
  case K::UnknownTensorType: return GQH_ETENSOR_TYPE;
  case K::InvalidString: return GQH_ESTRING;
  case K::MissingMetadata: return GQH_EMISSING;
  case K::WrongMetadataType: return GQH_EWRONG_TYPE;
  case K::MultiFileMismatch: return GQH_EMULTIFILE;
  case K::Io: return GQH_EIO;
  case K::BackendError: return GQH_EBACKEND;
  default: return GQH_EINVAL;
  }
}
int fail(int c, std::string msg) {
  g_err = std::move(msg);
  return c;
}
template <class F>
int guard(F &&f) {
  try {
    return f();
  } catch (const gqh::GgufError &e) {
    return fail(code(e), e.what());
  } catch (const std::exception &e) {
    return fail(GQH_EINVAL, e.what());
  }
}
const gqh::MetadataValue *meta(const gqh_gguf *f, const char *key, int &rc) {
  if (!f || !key) {
    rc = fail(GQH_EINVAL, "null argument");
    return nullptr;
  }
  const gqh::MetadataValue *v = f->file.get(key);
  if (!v) rc = fail(GQH_EMISSING, std::string("missing required metadata key: ") + key);
  return v;
}
int wrong(const char *key, const char *want) {
  return fail(GQH_EWRONG_TYPE, std::string("wrong type for metadata key ") + key + ": expected " + want);
}
// The image holding the tensor data of t (single buffer or one of the parts).
const uint8_t *tensor_bytes(const gqh_gguf *f, const gqh::TensorInfo &t) {
  const uint64_t at = f->file.data_offset + t.byte_offset;
  const size_t n = t.byte_size();
  if (f->single) {
    if (at > f->single_len || n > f->single_len - at)
      throw gqh::GgufError(gqh::GgufError::Kind::UnexpectedEof,
                           "unexpected end of input at byte " + std::to_string(f->single_len),
                           f->single_len);
    return f->single + at;
  }
  const uint8_t *p = f->maps.slice(at, n);
  if (!p)
    throw gqh::GgufError(gqh::GgufError::Kind::UnexpectedEof,
                         "unexpected end of input: tensor " + t.name + " lies outside the files", at);
  return p;
}
}  // namespace

extern "C" {

const char *gqh_last_error(void) { return g_err.c_str(); }

int gqh_gguf_open(const char *path, gqh_gguf **out) {
  if (!path || !out) return fail(GQH_EINVAL, "null argument");
  *out = nullptr;
  return guard([&]() -> int {
    auto [file, maps] = gqh::MultiFileMmap::load(path);
    auto h = std::make_unique<gqh_gguf>();
    h->file = std::move(file);
    h->maps = std::move(maps);
    *out = h.release();
    return GQH_OK;
  });
}

int gqh_gguf_parse(const void *data, size_t len, gqh_gguf **out) {
  if ((!data && len) || !out) return fail(GQH_EINVAL, "null argument");
  *out = nullptr;
  return guard([&]() -> int {
    auto h = std::make_unique<gqh_gguf>();
    h->owned.assign((const uint8_t *)data, (const uint8_t *)data + len);
    h->file = gqh::parse(h->owned.data(), h->owned.size());
    h->single = h->owned.data();
    h->single_len = h->owned.size();
    *out = h.release();
    return GQH_OK;
  });
}

int gqh_gguf_close(gqh_gguf *f) {
  delete f;
  return GQH_OK;
}

int gqh_gguf_header(const gqh_gguf *f, uint32_t *version, uint64_t *tensor_count,
                    uint64_t *metadata_count, uint64_t *data_offset) {
  if (!f) return fail(GQH_EINVAL, "null file");
  if (version) *version = f->file.version;
  if (tensor_count) *tensor_count = f->file.tensor_count;
  if (metadata_count) *metadata_count = f->file.metadata.size();
  if (data_offset) *data_offset = f->file.data_offset;
  return GQH_OK;
}

int gqh_gguf_tensor(const gqh_gguf *f, uint64_t i, const char **name, uint32_t *n_dims,
                    uint64_t *dims, uint32_t *ggml_type, uint64_t *byte_offset, uint64_t *nbytes) {
  if (!f || i >= f->file.tensors.size()) return fail(GQH_EINVAL, "tensor index out of range");
  const gqh::TensorInfo &t = f->file.tensors[i];
  if (name) *name = t.name.c_str();
  if (n_dims) *n_dims = t.n_dims;
  if (dims)
    for (size_t k = 0; k < t.dims.size() && k < 8; k++) dims[k] = t.dims[k];
  if (ggml_type) *ggml_type = (uint32_t)t.ggml_type;
  if (byte_offset) *byte_offset = t.byte_offset;
  if (nbytes) *nbytes = t.byte_size();
  return GQH_OK;
}

int gqh_gguf_find_tensor(const gqh_gguf *f, const char *name, uint64_t *index) {
  if (!f || !name || !index) return fail(GQH_EINVAL, "null argument");
  for (size_t k = 0; k < f->file.tensors.size(); k++)
    if (f->file.tensors[k].name == name) {
      *index = k;
      return GQH_OK;
    }
  return fail(GQH_EMISSING, std::string("no tensor named ") + name);
}

int gqh_gguf_tensor_data(const gqh_gguf *f, uint64_t i, const void **data, size_t *nbytes) {
  if (!f || !data || i >= f->file.tensors.size()) return fail(GQH_EINVAL, "bad argument");
  return guard([&]() -> int {
    const gqh::TensorInfo &t = f->file.tensors[i];
    *data = tensor_bytes(f, t);
    if (nbytes) *nbytes = t.byte_size();
    return GQH_OK;
  });
}

int gqh_gguf_meta_type(const gqh_gguf *f, const char *key, uint32_t *type_id) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  if (type_id) *type_id = v->type_id();
  return GQH_OK;
}
int gqh_gguf_meta_u64(const gqh_gguf *f, const char *key, uint64_t *out) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  auto x = v->as_u64();
  if (!x) return wrong(key, "unsigned integer");
  if (out) *out = *x;
  return GQH_OK;
}
int gqh_gguf_meta_i64(const gqh_gguf *f, const char *key, int64_t *out) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  auto x = v->as_i64();
  if (!x) return wrong(key, "integer");
  if (out) *out = *x;
  return GQH_OK;
}
int gqh_gguf_meta_f32(const gqh_gguf *f, const char *key, float *out) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  auto x = v->as_f32();
  if (!x) return wrong(key, "float");
  if (out) *out = *x;
  return GQH_OK;
}
int gqh_gguf_meta_bool(const gqh_gguf *f, const char *key, int *out) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  auto x = v->as_bool();
  if (!x) return wrong(key, "bool");
  if (out) *out = *x ? 1 : 0;
  return GQH_OK;
}
int gqh_gguf_meta_str(const gqh_gguf *f, const char *key, const char **out, size_t *len) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  if (v->type != gqh::MetaType::String) return wrong(key, "string");
  if (out) *out = v->s.c_str();
  if (len) *len = v->s.size();
  return GQH_OK;
}
int gqh_gguf_meta_array(const gqh_gguf *f, const char *key, uint32_t *elem_type, uint64_t *count) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  if (v->type != gqh::MetaType::Array) return wrong(key, "array");
  if (elem_type) *elem_type = (uint32_t)v->elem;
  if (count) *count = v->items.size();
  return GQH_OK;
}
int gqh_gguf_meta_array_i64(const gqh_gguf *f, const char *key, uint64_t k, int64_t *out) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  if (v->type != gqh::MetaType::Array) return wrong(key, "array");
  if (k >= v->items.size()) return fail(GQH_EINVAL, "array index out of range");
  auto x = v->items[k].as_i64();
  if (!x) return wrong(key, "integer array");
  if (out) *out = *x;
  return GQH_OK;
}
int gqh_gguf_meta_array_str(const gqh_gguf *f, const char *key, uint64_t k, const char **out,
                            size_t *len) {
  int rc = GQH_OK;
  const gqh::MetadataValue *v = meta(f, key, rc);
  if (!v) return rc;
  if (v->type != gqh::MetaType::Array) return wrong(key, "array");
  if (k >= v->items.size()) return fail(GQH_EINVAL, "array index out of range");
  if (v->items[k].type != gqh::MetaType::String) return wrong(key, "string array");
  if (out) *out = v->items[k].s.c_str();
  if (len) *len = v->items[k].s.size();
  return GQH_OK;
}

int gqh_parse_split_index(const char *file_name, uint64_t *index, uint64_t *total) {
  if (!file_name) return fail(GQH_EINVAL, "null argument");
  auto r = gqh::parse_split_index(file_name);
  if (!r) return fail(GQH_EMISSING, std::string("not a split file name: ") + file_name);
  if (index) *index = r->first;
  if (total) *total = r->second;
  return GQH_OK;
}

int gqh_gguf_upload(const gqh_gguf *f, const char *name, gq_weight **out) {
  if (!f || !name || !out) return fail(GQH_EINVAL, "null argument");
  *out = nullptr;
  return guard([&]() -> int {
    const gqh::TensorInfo *t = f->file.find(name);
    if (!t) return fail(GQH_EMISSING, std::string("no tensor named ") + name);
    const gqh::HipBackend be;
    if (t->n_dims != 2 || !gqh::gpu_dequant_type(t->ggml_type))
      return fail(GQH_EBACKEND, std::string("backend error: tensor ") + name + " (" +
                                    gqh::type_name(t->ggml_type) + ", " + t->shape_str() +
                                    ") is not a weight this backend multiplies");
    const uint8_t *p = tensor_bytes(f, *t);
    *out = be.upload_weight(t->ggml_type, p, t->byte_size(), (size_t)t->dims[0]).release();
    return GQH_OK;
  });
}

int gqh_model_load(const gqh_gguf *f, int ctx, int max_tokens, gqh_model **out) {
  if (!f || !out) return fail(GQH_EINVAL, "null argument");
  *out = nullptr;
  if (ctx < 0 || max_tokens <= 0) return fail(GQH_EINVAL, "ctx must be >= 0 and max_tokens > 0");
  return guard([&]() -> int {
    auto bytes = [f](const gqh::TensorInfo &t) { return tensor_bytes(f, t); };
    // Pages of a file mapping that the upload has consumed go back to the
    // page cache's control (a private read-only mapping re-reads on access).
    gqh::ReleaseBytes release;
    if (!f->single) {
      release = [](const uint8_t *p, size_t n) {
        const uintptr_t pg = (uintptr_t)sysconf(_SC_PAGESIZE);
        const uintptr_t a = ((uintptr_t)p + pg - 1) & ~(pg - 1), b = ((uintptr_t)p + n) & ~(pg - 1);
        if (b > a) (void)madvise((void *)a, b - a, MADV_DONTNEED);
      };
    }
    auto h = std::make_unique<gqh_model>();
    h->m = gqh::ResidentModel::load(f->file, bytes, ctx, max_tokens, release);
    *out = h.release();
    return GQH_OK;
  });
}

int gqh_model_free(gqh_model *m) {
  delete m;
  return GQH_OK;
}

int gqh_model_config_get(const gqh_model *m, gqh_model_config *cfg) {
  if (!m || !cfg) return fail(GQH_EINVAL, "null argument");
  const gqh::ModelConfig &c = m->m->config();
  std::memset(cfg, 0, sizeof(*cfg));
  cfg->context_length = c.context_length;
  cfg->embedding_length = c.embedding_length;
  cfg->block_count = c.block_count;
  cfg->head_count = c.head_count;
  cfg->head_count_kv = c.head_count_kv;
  cfg->head_dim = c.head_dim;
  cfg->feed_forward_length = c.feed_forward_length;
  cfg->vocab_size = c.vocab_size;
  cfg->rope_freq_base = c.rope_freq_base;
  cfg->layer_norm_rms_epsilon = c.layer_norm_rms_epsilon;
  cfg->ctx = m->m->ctx();
  std::strncpy(cfg->architecture, c.architecture.c_str(), sizeof(cfg->architecture) - 1);
  return GQH_OK;
}

int gqh_model_handle(const gqh_model *m, gq_model **out) {
  if (!m || !out) return fail(GQH_EINVAL, "null argument");
  *out = m->m->handle();
  return GQH_OK;
}

}  // extern "C"
