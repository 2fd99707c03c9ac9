/* gq_host.h -- C ABI of the host library libgq_host.so: GGUF files opened,
 * parsed and mapped once, their weight tensors uploaded to libgq (gq.h).
 *
 * Entry points replace the reference's loader path for the hot path's data
 * format: parser::parse (src/parser.rs:9-66), loader::load and the split
 * loader MultiFileMmap (src/loader.rs:14-86), the GgufFile accessors
 * (src/types.rs: get_*, tensors) and the one-time weight upload of
 * pre_upload_gpu (src/model/llama/gpu_resident.rs:69-229).  The C++ API
 * behind it is agention-infer_amd/host/{gguf,hip_backend}.h.
 *
 * Every call returns 0 or a negative GQH_E* code (the reference's GgufError
 * kinds); gqh_last_error() gives the message of the calling thread's last
 * failure. */
#ifndef GQ_HOST_H
#define GQ_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "gq.h"

#ifdef __cplusplus
extern "C" {
#endif

enum {
  GQH_OK = 0,
  GQH_EINVALID_MAGIC = -101,      /* GgufError::InvalidMagic */
  GQH_EVERSION = -102,            /* UnsupportedVersion */
  GQH_EEOF = -103,                /* UnexpectedEof */
  GQH_EMETA_TYPE = -104,          /* UnknownMetadataType */
  GQH_ETENSOR_TYPE = -105,        /* UnknownTensorType */
  GQH_ESTRING = -106,             /* InvalidString */
  GQH_EMISSING = -107,            /* MissingMetadata (also: no such key / tensor) */
  GQH_EWRONG_TYPE = -108,         /* WrongMetadataType */
  GQH_EMULTIFILE = -110,          /* MultiFileMismatch */
  GQH_EIO = -111,                 /* Io */
  GQH_EBACKEND = -112,            /* BackendError */
  GQH_EINVAL = -113               /* a null or out-of-range argument */
};

typedef struct gqh_gguf gqh_gguf; /* a parsed, mapped GGUF file (or split set) */

const char *gqh_last_error(void);

/* loader::load / MultiFileMmap::load: a name of the form
 * "x-00001-of-0000N.gguf" opens all N parts. */
int gqh_gguf_open(const char *path, gqh_gguf **out);
/* parser::parse over a caller's buffer (copied). */
int gqh_gguf_parse(const void *data, size_t len, gqh_gguf **out);
int gqh_gguf_close(gqh_gguf *f);

int gqh_gguf_header(const gqh_gguf *f, uint32_t *version, uint64_t *tensor_count,
                    uint64_t *metadata_count, uint64_t *data_offset);

/* Tensor i: name (valid while f is open), dims[0..n_dims) (n_dims <= 8
 * copied), GGML type id, byte offset from the data section, byte size. */
int gqh_gguf_tensor(const gqh_gguf *f, uint64_t i, const char **name, uint32_t *n_dims,
                    uint64_t *dims, uint32_t *ggml_type, uint64_t *byte_offset, uint64_t *nbytes);
int gqh_gguf_find_tensor(const gqh_gguf *f, const char *name, uint64_t *index);
/* The tensor's bytes in the mapping (valid while f is open). */
int gqh_gguf_tensor_data(const gqh_gguf *f, uint64_t i, const void **data, size_t *nbytes);

/* Metadata by key (GgufFile::get_u64 / as_i64 / get_f32 / get_string / get_bool);
 * GQH_EMISSING if absent, GQH_EWRONG_TYPE if of another kind. */
int gqh_gguf_meta_type(const gqh_gguf *f, const char *key, uint32_t *type_id);
int gqh_gguf_meta_u64(const gqh_gguf *f, const char *key, uint64_t *v);
int gqh_gguf_meta_i64(const gqh_gguf *f, const char *key, int64_t *v);
int gqh_gguf_meta_f32(const gqh_gguf *f, const char *key, float *v);
int gqh_gguf_meta_bool(const gqh_gguf *f, const char *key, int *v);
int gqh_gguf_meta_str(const gqh_gguf *f, const char *key, const char **v, size_t *len);
/* Arrays: element count and type; element k as integer / string. */
int gqh_gguf_meta_array(const gqh_gguf *f, const char *key, uint32_t *elem_type, uint64_t *count);
int gqh_gguf_meta_array_i64(const gqh_gguf *f, const char *key, uint64_t k, int64_t *v);
int gqh_gguf_meta_array_str(const gqh_gguf *f, const char *key, uint64_t k, const char **v,
                            size_t *len);

/* "x-00002-of-00005.gguf" -> 2, 5 (loader::parse_split_index); GQH_EMISSING
 * for other names. */
int gqh_parse_split_index(const char *file_name, uint64_t *index, uint64_t *total);

/* Upload a 2-D weight tensor once (HipBackend::upload_tensor): dims [in_dim,
 * out_dim], type Q8_0/Q4_K/Q5_K/Q6_K/IQ3_XXS.  Free with gq_weight_free. */
int gqh_gguf_upload(const gqh_gguf *f, const char *name, gq_weight **out);

/* ---- A dense decoder from a GGUF file, resident on the GPU ------------
 * LlamaModel::new (src/model/llama/mod.rs:130-300) with ModelConfig::
 * from_gguf (src/model/mod.rs:212-272) and pre_upload_gpu (src/model/llama/
 * gpu_resident.rs:69-229): every matmul weight uploaded once in file order,
 * norms and the embedding table dequantized, then gq_model_create.  ctx = 0
 * takes the file's context_length (at most 65536).  Files whose layers use
 * another mixer, QK-norm or RoPE scaling fail with GQH_EBACKEND naming what
 * the GPU-resident decode does not cover. The file may be closed after. */
typedef struct gqh_model gqh_model;
typedef struct {
  uint64_t context_length, embedding_length, block_count, head_count, head_count_kv, head_dim,
      feed_forward_length, vocab_size;
  float rope_freq_base, layer_norm_rms_epsilon;
  int ctx;                /* KV cache positions allocated */
  char architecture[64];  /* NUL-terminated, truncated */
} gqh_model_config;

int gqh_model_load(const gqh_gguf *f, int ctx, int max_tokens, gqh_model **out);
int gqh_model_free(gqh_model *m);
int gqh_model_config_get(const gqh_model *m, gqh_model_config *cfg);
/* The gq_model (include/gq.h) for gq_model_decode / _generate / _kv_*;
 * owned by m. */
int gqh_model_handle(const gqh_model *m, gq_model **out);

#ifdef __cplusplus
}
#endif
#endif
