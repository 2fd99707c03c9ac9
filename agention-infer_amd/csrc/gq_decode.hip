// gq_decode.hip -- the non-matmul kernels of a GPU-resident decode step for
// a dense Llama/Qwen2-style decoder (the reference's run_gpu_resident,
// src/model/llama/gpu_resident.rs:427-697, restating the arithmetic of
// LlamaModel::run, src/model/llama/cpu_path.rs:695-818).
//
// Step state (token, position, step counter) lives in device memory so that
// a captured HIP graph of one step can be replayed for every greedy step:
// the argmax kernel writes the next token and advances the position.
#include "gq_device.h"
#include "gq_internal.h"

namespace gq {

// Block-wide sum for 1024 threads (16 waves).
__device__ __forceinline__ float block_sum_1024(float v, float *red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  if (threadIdx.x < 64) {
    s = threadIdx.x < 16 ? red[threadIdx.x] : 0.f;
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (threadIdx.x == 0) red[16] = s;
  }
  __syncthreads();
  s = red[16];
  __syncthreads();
  return s;
}

// x = embd[token]  (the embedding row lookup, cpu_path.rs:705-707).
__global__ void k_embed(const float *embd, const DecodeState *st, float *x, int h) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < h) x[i] = embd[(long)st->token * h + i];
}

// Optional residual add (x += r), then out = w * x / rms(x)
// (rms_norm_into, cpu_path.rs:67-74).  One 1024-thread block.
__global__ __launch_bounds__(1024) void k_add_rmsnorm(float *x, const float *r, const float *w,
                                                      float *out, int h, float eps) {
  __shared__ float red[17];
  float ss = 0.f;
  for (int i = threadIdx.x; i < h; i += 1024) {
    float v = x[i];
    if (r) {
      v += r[i];
      x[i] = v;
    }
    ss += v * v;
  }
  ss = block_sum_1024(ss, red);
  const float rms = sqrtf(ss / (float)h + eps);
  for (int i = threadIdx.x; i < h; i += 1024) out[i] = w[i] * x[i] / rms;
}

// RoPE on q and k at the current position (NEOX pairs d <-> d + hd/2,
// freq = pos / theta^(2d/hd), cpu_path.rs:99-133), then k and v stored as
// f16 (round to nearest even, KvDtype::F16::pack) into the cache row.
// Grid: n_heads + n_kv_heads blocks of hd/2 threads.
__global__ void k_rope_kv(float *q, const float *k, const float *v, uint16_t *kc, uint16_t *vc,
                          const DecodeState *st, int n_heads, int n_kv, int hd, float theta) {
  const int hb = blockIdx.x, d = threadIdx.x, half = hd / 2;
  const int pos = st->pos;
  const float freq = (float)pos * 1.0f / powf(theta, 2.0f * (float)d / (float)hd);
  const float sn = sinf(freq), cs = cosf(freq);
  if (hb < n_heads) {
    float *p = q + (long)hb * hd;
    const float x0 = p[d], x1 = p[d + half];
    p[d] = x0 * cs - x1 * sn;
    p[d + half] = x0 * sn + x1 * cs;
  } else {
    const int h = hb - n_heads;
    const long kvd = (long)n_kv * hd;
    const float *pk = k + (long)h * hd;
    const float x0 = pk[d], x1 = pk[d + half];
    const float y0 = x0 * cs - x1 * sn, y1 = x0 * sn + x1 * cs;
    uint16_t *kr = kc + (long)pos * kvd + (long)h * hd;
    uint16_t *vr = vc + (long)pos * kvd + (long)h * hd;
    kr[d] = __half_as_ushort(__float2half_rn(y0));
    kr[d + half] = __half_as_ushort(__float2half_rn(y1));
    vr[d] = __half_as_ushort(__float2half_rn(v[(long)h * hd + d]));
    vr[d + half] = __half_as_ushort(__float2half_rn(v[(long)h * hd + d + half]));
  }
}

// Attention, split over position chunks (flash-decode): block (h, c) scores
// positions [c*ATT_CHUNK, ...) of head h against its KV head h / group,
// writing m = max score, l = sum exp(s - m), o = sum exp(s - m) v.
// Scores are q.k / sqrt(hd) as attention_into (cpu_path.rs:141-194).
constexpr int ATT_CHUNK = 256;

__global__ __launch_bounds__(256) void k_attn_partial(const float *q, const uint16_t *kc,
                                                      const uint16_t *vc, const DecodeState *st,
                                                      int n_heads, int group, int hd, int kvd,
                                                      float *part) {
  __shared__ float qs[256];
  __shared__ float sc[ATT_CHUNK];
  __shared__ float red[8];
  __shared__ float ohalf[2][256];
  const int h = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
  const int n = st->pos + 1;
  const int t0 = c * ATT_CHUNK;
  const int kh = h / group;
  float *out = part + ((long)h * gridDim.y + c) * (2 + hd);
  if (t0 >= n) {  // chunk past the current length: neutral partial
    if (tid == 0) {
      out[0] = -INFINITY;
      out[1] = 0.f;
    }
    if (tid < hd) out[2 + tid] = 0.f;
    return;
  }
  if (tid < hd) qs[tid] = q[(long)h * hd + tid];
  __syncthreads();
  const int t = t0 + tid;
  float s = -INFINITY;
  if (t < n) {
    const uint16_t *kr = kc + (long)t * kvd + (long)kh * hd;
    float dot = 0.f;
    for (int d = 0; d < hd; d += 8) {
      const uint4 raw = *(const uint4 *)(kr + d);
      const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        dot += qs[d + 2 * j] * h2f(w4[j]);
        dot += qs[d + 2 * j + 1] * h2f(w4[j] >> 16);
      }
    }
    s = dot / sqrtf((float)hd);
  }
  // block max
  float m = s;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float p = t < n ? expf(s - m) : 0.f;
  sc[tid] = p;
  float l = p;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
  __syncthreads();
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = l;
  __syncthreads();
  l = red[4] + red[5] + red[6] + red[7];
  // o[d] = sum_t p_t v_t[d]: threads (d, half) take alternate positions
  const int d = tid % 128, hv = tid / 128;
  const int tn = min(ATT_CHUNK, n - t0);
  float o = 0.f;
  if (d < hd)
    for (int j = hv; j < tn; j += 2)
      o += sc[j] * h2f(vc[(long)(t0 + j) * kvd + (long)kh * hd + d]);
  ohalf[hv][d] = o;
  __syncthreads();
  if (tid < hd) out[2 + tid] = ohalf[0][tid] + ohalf[1][tid];
  if (tid == 0) {
    out[0] = m;
    out[1] = l;
  }
}

// Combine the chunks of each head: out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M).
__global__ void k_attn_combine(const float *part, int nchunks, int hd, float *att) {
  const int h = blockIdx.x, d = threadIdx.x;
  const float *ph = part + (long)h * nchunks * (2 + hd);
  float M = -INFINITY;
  for (int c = 0; c < nchunks; c++) M = fmaxf(M, ph[c * (2 + hd)]);
  float L = 0.f, o = 0.f;
  for (int c = 0; c < nchunks; c++) {
    const float *pc = ph + c * (2 + hd);
    if (pc[0] == -INFINITY) continue;
    const float f = expf(pc[0] - M);
    L += pc[1] * f;
    o += pc[2 + d] * f;
  }
  if (d < hd) att[(long)h * hd + d] = o / L;
}

// Greedy argmax (first maximum wins, sampler.rs:120-131); records the token,
// makes it the next input and advances the position.  One 1024-thread block.
__global__ __launch_bounds__(1024) void k_argmax_next(const float *logits, int n, DecodeState *st,
                                                      int *tokens, int max_tokens) {
  __shared__ float bv_s[16];
  __shared__ int bi_s[16];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += 1024) {
    const float v = logits[i];
    if (v > bv) {  // i increases per thread: strict > keeps the first
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bv_s[w] = bv;
    bi_s[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = bv_s[0];
    int idx = bi_s[0];
    for (int j = 1; j < 16; j++)
      if (bv_s[j] > v || (bv_s[j] == v && bi_s[j] < idx)) { v = bv_s[j]; idx = bi_s[j]; }
    if (idx == 0x7fffffff) idx = 0;  // all -inf / NaN: index 0, as argmax's initial best
    if (tokens && st->step < max_tokens) tokens[st->step] = idx;
    st->token = idx;
    st->pos += 1;
    st->step += 1;
  }
}

// Start a decode sequence: token and position from the host, step 0.
__global__ void k_set_state(DecodeState *st, int token, int pos) {
  if (threadIdx.x == 0) *st = DecodeState{token, pos, 0, 0};
}

// ------------------------------------------------------------------ host
hipError_t launch_set_state(DecodeState *st, int token, int pos, hipStream_t s) {
  hipLaunchKernelGGL(k_set_state, dim3(1), dim3(64), 0, s, st, token, pos);
  return hipGetLastError();
}

hipError_t launch_decode_step(const DecodeLaunch &m, hipStream_t s) {
  const int H = m.hidden, hd = m.head_dim, nh = m.n_heads, nkv = m.n_kv_heads;
  const int kvd = nkv * hd;
  hipLaunchKernelGGL(k_embed, dim3((H + 255) / 256), dim3(256), 0, s, m.embd, m.state, m.x, H);
  for (int L = 0; L < m.n_layers; L++) {
    // attention block (the previous layer's FFN residual is added here)
    hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(1024), 0, s, m.x, L ? m.proj : nullptr,
                       m.attn_norm[L], m.xn, H, m.eps);
    const gq_weight *qkv[3] = {m.wq[L], m.wk[L], m.wv[L]};
    float *qkv_out[3] = {m.q, m.k, m.v};
    hipError_t e = matvec_launch(qkv, 3, m.xn, nullptr, nullptr, qkv_out, s);
    if (e != hipSuccess) return e;
    uint16_t *kc = m.kcache + (long)L * m.ctx * kvd, *vc = m.vcache + (long)L * m.ctx * kvd;
    hipLaunchKernelGGL(k_rope_kv, dim3(nh + nkv), dim3(hd / 2), 0, s, m.q, m.k, m.v, kc, vc,
                       m.state, nh, nkv, hd, m.theta);
    hipLaunchKernelGGL(k_attn_partial, dim3(nh, m.att_chunks), dim3(256), 0, s, m.q, kc, vc,
                       m.state, nh, nh / nkv, hd, kvd, m.att_part);
    hipLaunchKernelGGL(k_attn_combine, dim3(nh), dim3(hd), 0, s, m.att_part, m.att_chunks, hd,
                       m.att);
    const gq_weight *wo[1] = {m.wo[L]};
    float *proj[1] = {m.proj};
    if ((e = matvec_launch(wo, 1, m.att, nullptr, nullptr, proj, s)) != hipSuccess) return e;
    // FFN block
    hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(1024), 0, s, m.x, m.proj, m.ffn_norm[L],
                       m.xn, H, m.eps);
    const gq_weight *gu[2] = {m.wgate[L], m.wup[L]};
    float *gu_out[2] = {m.g, m.u};
    if ((e = matvec_launch(gu, 2, m.xn, nullptr, nullptr, gu_out, s)) != hipSuccess) return e;
    const gq_weight *wd[1] = {m.wdown[L]};
    if ((e = matvec_launch(wd, 1, nullptr, m.g, m.u, proj, s)) != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(1024), 0, s, m.x, m.proj, m.output_norm, m.xn,
                     H, m.eps);
  const gq_weight *hw[1] = {m.lm_head};
  float *lo[1] = {m.logits};
  hipError_t e = matvec_launch(hw, 1, m.xn, nullptr, nullptr, lo, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_argmax_next, dim3(1), dim3(1024), 0, s, m.logits, m.vocab, m.state,
                     m.tokens, m.max_tokens);
  return hipGetLastError();
}

}  // namespace gq
