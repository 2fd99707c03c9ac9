/*
 * gq_oracle.h -- CPU restatement of gguf-rs's quantized dequant-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the
 * timed CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (libgq.so) never links
 * or calls it.
 *
 * Every function restates one reference function (Rust crate gguf-rs,
 * /root/reference/src/...) with the same arithmetic order, compiled with
 * -ffp-contract=off so that no a*b+c is fused (Rust never contracts).
 *
 * Return codes: 0 = ok, GQO_ESHORT = buffer too short ("need N bytes"),
 * GQO_EDTYPE = unsupported dtype, GQO_ERANGE = row out of range.
 */
#ifndef GQ_ORACLE_H
#define GQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GQO_ESHORT (-1)
#define GQO_EDTYPE (-2)
#define GQO_ERANGE (-3)

/* GgmlType ids (types.rs:9-46). */
enum { GQO_F32 = 0, GQO_F16 = 1, GQO_Q8_0 = 8, GQO_Q4_K = 12, GQO_Q5_K = 13,
       GQO_Q6_K = 14, GQO_Q8_K = 15, GQO_IQ3_XXS = 18, GQO_BF16 = 30 };

size_t gqo_block_size(int dtype);              /* types.rs:88-123 */
size_t gqo_block_bytes(int dtype);             /* types.rs:126-161 */
size_t gqo_type_size(int dtype, size_t n);     /* types.rs:164-168 */

float    gqo_f16_to_f32(uint16_t h);           /* half::f16::to_f32 (exact) */
uint16_t gqo_f32_to_f16(float f);              /* half::f16::from_f32 (RNE) */

/* Per-format dequant of n elements from `data` (nbytes long). */
int gqo_dequant_q8_0(const uint8_t *data, size_t nbytes, size_t n, float *out);
int gqo_dequant_q4_k(const uint8_t *data, size_t nbytes, size_t n, float *out);
int gqo_dequant_q5_k(const uint8_t *data, size_t nbytes, size_t n, float *out);
int gqo_dequant_q6_k(const uint8_t *data, size_t nbytes, size_t n, float *out);
int gqo_dequant_iq3_xxs(const uint8_t *data, size_t nbytes, size_t n, float *out);
int gqo_dequant(int dtype, const uint8_t *data, size_t nbytes, size_t n, float *out);

/* Fused dequant+dot of one row with x[n]. */
int gqo_dot_q8_0(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res);
int gqo_dot_q4_k(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res);
int gqo_dot_q5_k(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res);
int gqo_dot_q6_k(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res);
int gqo_dot_iq3_xxs(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res);
int gqo_dot_row(int dtype, const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res);

/* Q4_K sub-block scale/min unpack (q4_k.rs:26-35). */
void gqo_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);

/* Q8_K activation quantizer (q8_k.rs:49-91): d[nblk], qs[nblk*256], bsums[nblk*16]. */
void gqo_quantize_row_q8_k(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums);
int  gqo_dot_q5_k_q8k(const uint8_t *data, size_t nbytes, size_t n, const float *d,
                      const int8_t *qs, const int16_t *bsums, float *res);

/* Per-32 Q8 activation pack (KvDtype::Q8_0::pack, model/mod.rs:574-583):
 * scale_f16[n/32], q[n] (int8).  Used for the int8 prefill GEMM. */
void gqo_quantize_q8_32(const float *x, size_t n, uint16_t *scale_f16, int8_t *q);

/* IQ3_XXS codebook in use (256 x uint32, 4 magnitude bytes each). */
void gqo_set_iq3xxs_grid(const uint32_t *grid);
void gqo_get_iq3xxs_grid(uint32_t *grid);

/* WeightMap::matmul_into (model/mod.rs:362-403): out[r] = dot_row(W, r, x),
 * rows partitioned over nthreads (0 = hardware concurrency); for Q5_K x is
 * quantized to Q8_K once and every row runs dot_q5_k_q8k (mod.rs:381-394). */
int gqo_matmul_into(int dtype, const uint8_t *w, size_t nbytes, const float *x, size_t in_dim,
                    float *out, size_t out_dim, int nthreads);

/* out[r] = quant::dot_row(W, r, x) for every type (the float dot, also for
 * Q5_K), row-parallel: ffn_gate_up's per-row dots (cpu_path.rs:222-229). */
int gqo_matmul_rows(int dtype, const uint8_t *w, size_t nbytes, const float *x, size_t in_dim,
                    float *out, size_t out_dim, int nthreads);

/* CpuBackend::matmul_dequant (cpu_backend.rs:38-65): serial row loop. */
int gqo_matmul_dequant(int dtype, const uint8_t *w, size_t nbytes, const float *x, size_t in_dim,
                       float *out, size_t out_dim);

/* WeightMap::matmul_batch_into (model/mod.rs:414-464): X [batch][in_dim]
 * token-major -> Y [batch][out_dim] token-major; dequant each row once,
 * sequential f32 sum per token. */
int gqo_matmul_batch_into(int dtype, const uint8_t *w, size_t nbytes, const float *x,
                          size_t in_dim, size_t batch, float *out, size_t out_dim, int nthreads);

/* Same, over rows [r0, r1) only, writing rowmajor[r - r0][batch]. */
int gqo_matmul_batch_rows(int dtype, const uint8_t *w, size_t nbytes, const float *x,
                          size_t in_dim, size_t batch, size_t r0, size_t r1, float *rowmajor);

/* MoE routing (docs/08-moe-routing.md:24-30: probs = softmax(scores),
 * top_k_indices = argtop_k(probs, k)): for each of T tokens, ids[t][k] are
 * the k largest logits (ties: lower expert index first) and w[t][k] their
 * softmax probabilities over all E experts (not renormalised). */
void gqo_moe_route(const float *logits, int T, int E, int k, int *ids, float *w);

/* MoE FFN (docs/08-moe-routing.md:24-30) with the dense SwiGLU of
 * ffn_gate_up (model/llama/cpu_path.rs:200-232):
 *   out[t] = sum_s w[t][s] * down_e(silu(gate_e x_t) * up_e x_t),  e = ids[t][s].
 * gate/up: E stacked [F][H] matrices, down: E stacked [H][F] matrices, all
 * of `dtype`.  Slots are accumulated in order s = 0..k-1. */
int gqo_moe_ffn(int dtype, const uint8_t *gate, const uint8_t *up, const uint8_t *down, int E,
                int H, int F, const float *x, int T, int k, const int *ids, const float *w,
                float *out, int nthreads);

/* A dense Llama/Qwen2-style decoder (the Attention mixer of LlamaModel) for
 * the decode restatement.  Weights are ggml bytes (rows of type_size(K));
 * norms and the embedding are f32; the KV cache is f16 bits
 * [layer][ctx][n_kv_heads * head_dim] (KvDtype::F16, model/mod.rs:567-603). */
typedef struct {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, ctx;
    float eps, theta;
    int attn_type, gate_up_type, down_type, head_type;
    const float *embd;                /* [vocab][hidden] */
    const float *output_norm;         /* [hidden] */
    const uint8_t *lm_head;
    const float *const *attn_norm;    /* [n_layers] -> [hidden] */
    const float *const *ffn_norm;
    const uint8_t *const *wq, *const *wk, *const *wv, *const *wo;
    const uint8_t *const *wgate, *const *wup, *const *wdown;
    uint16_t *const *kcache, *const *vcache;
    /* Optional per-tensor types [n_layers][7] in the order wq, wk, wv, wo,
     * wgate, wup, wdown (a GGUF file types each tensor on its own, as
     * matmul_into dispatches per tensor, model/mod.rs:358-380); NULL: the
     * uniform attn/gate_up/down types above. */
    const int *layer_types;
    /* KvDtype (model/mod.rs:540-603): 0 = F16 (kcache/vcache rows of kv_dim
     * f16), 1 = Q8_0 (rows of kv_dim/32 blocks of 34 bytes: f16 scale, 32
     * int8; kcache/vcache point to those bytes). */
    int kv_q8;
} gqo_model;

/* LlamaModel::run (model/llama/cpu_path.rs:695-818) for the Attention
 * mixer: embedding row, per layer rms_norm_into (:67-74) -> q/k/v matmuls ->
 * rope (:99-133, NEOX pairs d <-> d + head_dim/2) -> KvCache::write /
 * read_up_to (model/mod.rs:657-702, f16) -> attention_into (:141-194) -> wo
 * -> residual -> rms_norm -> ffn_gate_up (:200-232) -> down -> residual;
 * final norm and lm head.  logits[vocab]. */
int gqo_decode_step(const gqo_model *m, int token, int pos, float *logits, int nthreads);

/* argmax, first maximum wins (sampler.rs:120-131). */
size_t gqo_argmax(const float *xs, size_t n);

#ifdef __cplusplus
}
#endif
#endif
