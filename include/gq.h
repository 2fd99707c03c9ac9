/*
 * gq.h -- C ABI of libgq.so, the MI355X (gfx950) quantized dequant-matmul
 * backend for gguf-rs.
 *
 * Every entry point returns 0 on success or a negative GQ_E* code; the
 * message for the last failure on the calling thread is gq_last_error()
 * (mirrors GgufError::BackendError(String), src/error.rs:4-42).
 * Pointers named *_dev are device pointers; *_host are host pointers.
 * `stream` is a hipStream_t (NULL = the default stream).
 * Launch entry points (gq_matvec, gq_gemm, ...) are asynchronous on
 * `stream`; the *_host entry points are synchronous.
 */
#ifndef GQ_H
#define GQ_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GQ_OK 0
#define GQ_EINVAL (-1)   /* bad argument / shape mismatch */
#define GQ_EDTYPE (-2)   /* unsupported dtype ("unsupported dtype {other}") */
#define GQ_ESHORT (-3)   /* buffer too short ("need N bytes, have M") */
#define GQ_EHIP (-4)     /* HIP runtime error */
#define GQ_ENOMEM (-5)   /* device allocation failed */
#define GQ_ENODEV (-6)   /* no gfx950 device / not initialised */

/* GgmlType ids, the on-disk tensor type ids (src/types.rs:9-46). */
#define GQ_TYPE_F16 1
#define GQ_TYPE_Q8_0 8
#define GQ_TYPE_Q4_K 12
#define GQ_TYPE_Q5_K 13
#define GQ_TYPE_Q6_K 14
#define GQ_TYPE_IQ3_XXS 18

/* gq_gemm modes (batched prefill). */
#define GQ_GEMM_BF16 0  /* weight tiles dequantized to bf16 in LDS, bf16 MFMA */
#define GQ_GEMM_INT8 1  /* activations packed per-32 to Q8, int8 MFMA      */

typedef struct gq_weight gq_weight;

/* Select and initialise device `device` (BackendPreference::Hip arm of
 * create_backend, src/ops/backend_select.rs:72-83, which is a CPU-fallback
 * stub in the reference).  Fails with GQ_ENODEV if it is not a gfx950. */
int gq_init(int device);

/* Backend::name (src/ops/mod.rs:101): returns "hip". */
const char *gq_backend_name(void);

/* Message of the last failing call on this thread ("" if none). */
const char *gq_last_error(void);

/* GgmlType::type_size (src/types.rs:164-168): bytes of one row of n
 * elements; 0 for an unknown dtype. */
size_t gq_type_size(int dtype, size_t n);

/* WgpuBackend::upload_weight (src/ops/wgpu_backend/mod.rs:61-92): copy a
 * whole tensor (out_dim rows of type_size(in_dim) bytes, ggml block order)
 * to the device once and keep it resident, re-laid-out for the kernels.
 * All-zero blocks are valid (warmup, src/ops/backend_select.rs:133-139). */
int gq_upload(int dtype, const void *w_host, size_t nbytes, int in_dim, int out_dim,
              gq_weight **out);

/* Same, from bytes already on the device (ggml block order). */
int gq_upload_device(int dtype, const void *w_dev, size_t nbytes, int in_dim, int out_dim,
                     gq_weight **out);

/* Drop a handle (GpuWeightHandle's Drop). */
int gq_weight_free(gq_weight *w);

/* GpuWeightHandle::shape / out_dim (src/ops/wgpu_backend/mod.rs:914-922). */
int gq_weight_shape(const gq_weight *w, int *dtype, int *in_dim, int *out_dim);

/* Device bytes held by the handle (equals the ggml tensor size). */
size_t gq_weight_bytes(const gq_weight *w);

/* launch_only / launch_only_f32out (src/ops/wgpu_backend/resident.rs:13-69)
 * with the arithmetic of WeightMap::matmul_into (src/model/mod.rs:362-403):
 * y_dev[out_dim] = W . x_dev[in_dim], fp32 in and out, no readback.  Q5_K
 * weights take matmul_into's route: x quantized to Q8_K, then
 * dot_q5_k_q8k per row (mod.rs:381-394); every other type the float dot. */
int gq_matvec(const gq_weight *w, const float *x_dev, float *y_dev, void *stream);

/* matmul_dequant_qkv / _multi / _ffn (src/ops/wgpu_backend/mod.rs:702-854):
 * several weights sharing one input, one launch.  All weights must have
 * the same in_dim; y_dev[i] receives out_dim(w[i]) floats.  The arithmetic
 * is gq_matvec's per weight: Q5_K weights take matmul_into's Q8_K route
 * (mod.rs:381-394), unlike the wgpu kernels' float dequant-dot. */
int gq_matvec_multi(const gq_weight *const *w, int count, const float *x_dev,
                    float *const *y_dev, void *stream);

/* matmul_dequant_preloaded (src/ops/wgpu_backend/mod.rs:642-696):
 * host x in, host out, synchronous.  The float dot of every type, Q5_K
 * included (Backend::matmul_dequant's dot_row). */
int gq_matmul_dequant_preloaded(const gq_weight *w, const float *x_host, float *out_host);

/* Backend::matmul_dequant (src/ops/mod.rs:105, cpu_backend.rs:38-65):
 * w_host is the whole tensor (out_dim rows of type_size(in_dim) bytes);
 * out_host[out_dim] is overwritten.  Uploads, runs, reads back.  The float
 * dot (dot_row) of every type, Q5_K included. */
int gq_matmul_dequant_host(int dtype, const void *w_host, size_t nbytes, const float *x_host,
                           size_t in_dim, float *out_host, size_t out_dim);

/* quant::dequant_row (src/quant/mod.rs:25-45) for rows [row0, row0+nrows):
 * out_dev[nrows][in_dim] f32, bit-identical to the CPU dequant. */
int gq_dequant_rows(const gq_weight *w, int row0, int nrows, float *out_dev, void *stream);
/* The same into host memory, synchronous (WeightMap::dequant_tensor /
 * dequant_row, src/model/mod.rs:307-349): out_host[nrows][in_dim]. */
int gq_dequant_rows_host(const gq_weight *w, int row0, int nrows, float *out_host);

/* launch_only_batch (src/ops/wgpu_backend/resident.rs:76-104) and the
 * prefill path of WeightMap::matmul_batch_into (src/model/mod.rs:414-464):
 * X_dev [n][in_dim] fp32 token-major -> Y_dev [n][out_dim] fp32.
 * mode GQ_GEMM_BF16 (Q4_K, Q5_K, Q6_K or Q8_0 weights; each dequantized as
 * dequant_row does, then rounded to bf16) or GQ_GEMM_INT8 (Q4_K weights).
 * The first call on a weight builds its GEMM copy (per-stage records) and
 * synchronizes the stream once.  The packed-X workspace is the stream's own
 * (as gq_moe_ffn's).  Under HIP graph capture a call is accepted only if
 * that first call was made before and the stream's workspace already holds
 * the call's bytes; otherwise it fails with GQ_EINVAL and records nothing.
 * Workspaces are never freed while the process runs, so a captured graph
 * stays valid when later, larger calls grow the stream's workspace. */
int gq_gemm(const gq_weight *w, const float *X_dev, int n, float *Y_dev, int mode, void *stream);

/* Per-32 Q8 activation pack used by GQ_GEMM_INT8, identical to
 * KvDtype::Q8_0::pack (src/model/mod.rs:574-583): scale_dev[n/32] f16
 * bits, q_dev[n] int8 (n a multiple of 32). */
int gq_quantize_q8_32(const float *x_dev, int n, uint16_t *scale_dev, int8_t *q_dev,
                      void *stream);

/* quantize_row_q8_k (src/quant/q8_k.rs:49-91) of x_dev[n]: per 256-element
 * block d_dev[nb] (f32), qs_dev[nb*256] (int8, zero past n) and
 * bsums_dev[nb*16] (int16), nb = ceil(n / 256); bit-identical to the
 * reference.  This is the input quantization gq_matvec applies for Q5_K. */
int gq_quantize_row_q8k(const float *x_dev, int n, float *d_dev, int8_t *qs_dev,
                        int16_t *bsums_dev, void *stream);

/* IQ3_XXS codebook (256 entries, 4 magnitude bytes each).  The reference
 * has no IQ3_XXS implementation (src/quant/mod.rs:7,38-41) and the library
 * does not ship ggml's iq3xxs_grid: IQ3_XXS uploads fail with GQ_EDTYPE
 * until the caller installs a codebook.  NULL installs a built-in test
 * codebook (a fixed hash over ggml's magnitude alphabet) for synthetic
 * weights; it cannot decode a real IQ3_XXS tensor. */
int gq_set_iq3xxs_grid(const uint32_t *grid_host);
int gq_get_iq3xxs_grid(uint32_t *grid_host);

/* A stacked expert tensor as GGUF stores it (ffn_{gate,up,down}_exps,
 * [n_experts][rows_per_expert][in_dim], docs/08-moe-routing.md:36-46):
 * like gq_upload, with tiles that never straddle two experts. */
int gq_upload_experts(int dtype, const void *w_host, size_t nbytes, int in_dim,
                      int rows_per_expert, int n_experts, gq_weight **out);

/* MoE FFN for T tokens (docs/08-moe-routing.md:24-30; the reference has no
 * MoE forward pass, docs/roadmap/00-parity-roadmap.md:40):
 *   ids[t], w[t] = top_k of softmax(logits[t]) (ties: lower expert index;
 *                  weights are the full-softmax probabilities),
 *   out[t] = sum_s w[t][s] * down_e(silu(gate_e x_t) * up_e x_t),
 * SwiGLU as ffn_gate_up (src/model/llama/cpu_path.rs:200-232); each expert
 * matvec is matmul_into's (src/model/mod.rs:362-403): for Q5_K experts the
 * gate, up and down matvecs all take the Q8_K route (quantize_row_q8_k of
 * the input, dot_q5_k_q8k), not ffn_gate_up's float dot_row.  The
 * reference has no MoE, so that choice is not pinned to a reference output.  gate/up:
 * [n_experts][f][h], down: [n_experts][h][f], uploaded with
 * gq_upload_experts.  logits_dev [T][n_experts], x_dev/out_dev [T][h];
 * ids_dev/w_dev ([T][top_k]) receive the routing if non-NULL; top_k <= 64.
 * The workspace (T * top_k * (4 * f + 8) + 1024 bytes) is the stream's own,
 * allocated on first use and grown on demand, shared with gq_gemm's calls
 * on that stream and held until the process ends; under graph capture it
 * cannot grow (GQ_EINVAL; see gq_gemm, or use gq_moe_ffn_noalloc). */
int gq_moe_ffn(const gq_weight *gate, const gq_weight *up, const gq_weight *down, int n_experts,
               const float *logits_dev, int T, int top_k, const float *x_dev, float *out_dev,
               int *ids_dev, float *w_dev, void *stream);

/* gq_moe_ffn without any allocation: no counterpart in the reference; for
 * callers that cannot allocate (code under HIP graph capture, serving
 * loops).  The workspace (T * top_k * (4 * f + 8) + 1024 bytes) lives in a
 * static device array of GQ_MOE_NOALLOC_MAX_BYTES per GPU, held until the
 * process ends; larger shapes fail with GQ_EINVAL.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads) race.  Results equal gq_moe_ffn's. */
#define GQ_MOE_NOALLOC_MAX_BYTES (4 << 20)
int gq_moe_ffn_noalloc(const gq_weight *gate, const gq_weight *up, const gq_weight *down,
                       int n_experts, const float *logits_dev, int T, int top_k, const float *x_dev,
                       float *out_dev, int *ids_dev, float *w_dev, void *stream);

/* ---- GPU-resident decode of a dense Llama/Qwen2-style decoder ----------
 * The reference's run_gpu_resident (src/model/llama/gpu_resident.rs:427-697)
 * with the arithmetic of LlamaModel::run (src/model/llama/cpu_path.rs:
 * 695-818): embedding row, per layer RMSNorm -> q/k/v -> RoPE (NEOX) ->
 * f16 KV cache (KvDtype::F16) -> attention -> o -> residual -> RMSNorm ->
 * SwiGLU FFN -> residual, final RMSNorm, output head, greedy argmax
 * (sampler.rs:120-131).  Weight handles stay owned by the caller and must
 * outlive the model; norms and the f32 embedding are copied to the device. */
typedef struct gq_model gq_model;
typedef struct {
  int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, ctx, max_tokens;
  float eps, theta;
  const gq_weight *const *wq, *const *wk, *const *wv, *const *wo;  /* [n_layers] */
  const gq_weight *const *wgate, *const *wup, *const *wdown;       /* [n_layers] */
  const gq_weight *lm_head;
  const float *const *attn_norm, *const *ffn_norm;  /* host [n_layers][hidden] */
  const float *output_norm;                         /* host [hidden] */
  const float *embd;                                /* host [vocab][hidden] */
  /* KV cache type (KvDtype, src/model/mod.rs:530-603): 0 (or GQ_TYPE_F16)
   * f16 rows, GQ_TYPE_Q8_0 Q8_0 blocks (kv_dim a multiple of 32). */
  int kv_dtype;
} gq_model_desc;

int gq_model_create(const gq_model_desc *desc, gq_model **out);
int gq_model_free(gq_model *m);

/* Fill / read back KV cache rows [0, n_pos) of a layer, e.g. a prefilled
 * context (KvCache::write_range, src/model/mod.rs:671-680), in the cache's
 * KvDtype byte format: F16 rows of kv_dim f16 (uint16), Q8_0 rows of
 * kv_dim / 32 blocks of 34 bytes (f16 scale, 32 int8). */
int gq_model_kv_upload(gq_model *m, int layer, const void *k_host, const void *v_host, int n_pos);
int gq_model_kv_download(gq_model *m, int layer, void *k_host, void *v_host, int n_pos);

/* One decode step (Model::forward, src/model/llama/mod.rs:336-363): token at
 * position pos; logits_host[vocab] (may be NULL) and the greedy next token. */
int gq_model_decode(gq_model *m, int token, int pos, float *logits_host, int *next_token);

/* Batched prefill (LlamaModel::run_batch, src/model/llama/cpu_path.rs:834-991):
 * tokens_host[n] at positions pos .. pos + n - 1 through every layer, in
 * passes of up to 512 tokens; K/V of every position into the cache;
 * logits_host[vocab] (may be NULL) and the greedy next token (may be NULL)
 * of the last position.  Projection GEMMs run in bf16 (weights: bf16 of the
 * exact dequant; activations: bf16), everything else in fp32.  Needs Q4_K,
 * Q5_K, Q6_K or Q8_0 projection weights; the first call builds their GEMM
 * copies.  With a Q8_0 KV cache (KvDtype::Q8_0) the prompt rows are packed
 * as the decode step packs them and the attention reads every row unpacked
 * (code * scale), rounded to f16 for its MFMA operands.
 * Synchronous on `stream`. */
int gq_model_prefill(gq_model *m, const int *tokens_host, int n, int pos, float *logits_host,
                     int *next_token, void *stream);

/* n_steps greedy steps from (token, pos) (runner::greedy_run decode loop,
 * src/runner.rs:67-135): each step is one replay of a captured HIP graph;
 * the argmax feeds the next step on the device.  tokens_host[n_steps]
 * receives the generated tokens (synchronous when non-NULL). */
int gq_model_generate(gq_model *m, int token, int pos, int n_steps, int *tokens_host,
                      void *stream);

/* Wait for all work on `stream`. */
int gq_sync(void *stream);

#ifdef __cplusplus
}
#endif
#endif
