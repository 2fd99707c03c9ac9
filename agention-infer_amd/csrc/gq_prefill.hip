// gq_prefill.hip -- batched prefill of a dense Llama/Qwen2-style decoder:
// n prompt tokens at positions pos0 .. pos0 + n - 1 through every layer in
// one pass, K/V written to the cache for every position, logits of the last
// position (LlamaModel::run_batch, src/model/llama/cpu_path.rs:834-991).
//
// Per layer (as run_batch, with the projections on the bf16 GEMM):
//   xn = RMSNorm(x) * attn_norm      -> bf16 MFMA fragments (k_norm_to_frag)
//   q, k, v = xn . Wq/Wk/Wv          (one GEMM launch, K split)
//   RoPE of q and k, f16 K/V rows into the cache (k_rope_kv)
//   att = causal attention of every query over the cache (k_attn_prefill,
//         written as the o GEMM's bf16 X fragments)
//   x += att . Wo                    (GEMM, K split, accumulating reduction)
//   xn = RMSNorm(x) * ffn_norm; g, u = xn . Wgate/Wup
//   x += (silu(g) * u) . Wdown       (k_swiglu_to_frag, GEMM)
// then the output head on RMSNorm(x[n - 1]) (the decode matvec).
// The GEMM operands are bf16 (weights: bf16 of the exact dequant;
// activations: bf16 of the fp32 values), accumulation fp32; everything
// else is fp32 as on the CPU path.
#include <algorithm>

#include "gq_device.h"
#include "gq_internal.h"

namespace gq {

typedef _Float16 pf16x8_t __attribute__((ext_vector_type(8)));
typedef float pf32x4_t __attribute__((ext_vector_type(4)));

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Position of elements (t, c .. c + 7) (c % 8 == 0) in the GEMM's X
// fragments: fragment (t / 16, c / 32) of 64 lanes x 8 bf16, lane
// t % 16 + 16 * ((c % 32) / 8).
__device__ __forceinline__ long frag_slot(int t, int c, int ksteps) {
  return (((long)(t >> 4) * ksteps + (c >> 5)) * 64 + (t & 15) + 16 * ((c & 31) >> 3)) * 8;
}

__device__ __forceinline__ void put_frag8(uint16_t *xb, long slot, const float (&v)[8]) {
  const uint4 o = make_uint4(bf16_bits(v[0]) | (bf16_bits(v[1]) << 16),
                             bf16_bits(v[2]) | (bf16_bits(v[3]) << 16),
                             bf16_bits(v[4]) | (bf16_bits(v[5]) << 16),
                             bf16_bits(v[6]) | (bf16_bits(v[7]) << 16));
  *(uint4 *)(xb + slot) = o;
}

__device__ __forceinline__ float block_sum256(float v, float *red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return s;
}

// x[t] = embd[tokens[t]] (the embedding rows, fp32 on the device).
__global__ void k_embed_rows(const float *embd, const int *tokens, int H, float *x) {
  const int t = blockIdx.x;
  const float *src = embd + (long)tokens[t] * H;
  for (int i = threadIdx.x; i < H; i += blockDim.x) x[(long)t * H + i] = src[i];
}

// Fragments of RMSNorm(x[t]) * w (rms_norm_into, cpu_path.rs:67-74:
// w * x / sqrt(sum(x^2) / H + eps)) for tokens t < n, zeros for n <= t <
// npad and for columns past H.  One block (256 threads) per token; a
// thread keeps its groups of 8 values in registers across the reduction
// (H <= NORM_GROUPS * 8 * 256, H % 8 == 0 for the vector loads).
constexpr int NORM_GROUPS = 4;
// With ksplit > 0 the preceding accumulating GEMM left its K-split
// partials part[s][t][c] (s < ksplit) unreduced: x[t] += part[0][t] +
// part[1][t] + ... (in that order, as k_gemm_reduce) is done here, and the
// new row is stored back to x.
__global__ __launch_bounds__(256) void k_norm_to_frag(float *__restrict__ x, const float *__restrict__ w, int n,
                                                      int H, int kpad, float eps, uint16_t *__restrict__ xb,
                                                      const float *__restrict__ part, int ksplit) {
  __shared__ float red[4];
  const int t = blockIdx.x, ksteps = kpad / 32;
  float *xt = x + (long)t * H;
  float v[NORM_GROUPS][8];
  bool in[NORM_GROUPS];
  // every group's row loads first, then each split's partials for all
  // groups (loads in flight together, not one group's chain after another)
#pragma unroll
  for (int j = 0; j < NORM_GROUPS; j++) {
    const int c = 8 * (threadIdx.x + 256 * j);
    in[j] = t < n && c < H;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (in[j]) {
      a = *(const float4 *)(xt + c);
      b = *(const float4 *)(xt + c + 4);
    }
    v[j][0] = a.x; v[j][1] = a.y; v[j][2] = a.z; v[j][3] = a.w;
    v[j][4] = b.x; v[j][5] = b.y; v[j][6] = b.z; v[j][7] = b.w;
  }
  if (ksplit > 0) {
    const long cnt = (long)n * H;
    for (int k = 0; k < ksplit; k++) {
#pragma unroll
      for (int j = 0; j < NORM_GROUPS; j++) {
        if (!in[j]) continue;
        const float *pp = part + k * cnt + (long)t * H + 8 * (threadIdx.x + 256 * j);
        const float4 pa = *(const float4 *)pp, pb = *(const float4 *)(pp + 4);
        v[j][0] += pa.x; v[j][1] += pa.y; v[j][2] += pa.z; v[j][3] += pa.w;
        v[j][4] += pb.x; v[j][5] += pb.y; v[j][6] += pb.z; v[j][7] += pb.w;
      }
    }
#pragma unroll
    for (int j = 0; j < NORM_GROUPS; j++) {
      if (!in[j]) continue;
      const int c = 8 * (threadIdx.x + 256 * j);
      *(float4 *)(xt + c) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
      *(float4 *)(xt + c + 4) = make_float4(v[j][4], v[j][5], v[j][6], v[j][7]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NORM_GROUPS; j++)
#pragma unroll
    for (int e = 0; e < 8; e++) ss += v[j][e] * v[j][e];
  ss = block_sum256(ss, red);
  const float rms = sqrtf(ss / (float)H + eps);
#pragma unroll
  for (int j = 0; j < NORM_GROUPS; j++) {
    const int c = 8 * (threadIdx.x + 256 * j);
    if (c >= kpad) continue;
    float o[8];
    if (t < n && c < H) {
      const float4 a = *(const float4 *)(w + c), b = *(const float4 *)(w + c + 4);
      const float wv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = wv[e] * v[j][e] / rms;
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = 0.f;
    }
    put_frag8(xb, frag_slot(t, c, ksteps), o);
  }
}

// Fragments of silu(g) * u (ffn_gate_up, cpu_path.rs:225-227), g and u
// [n][F] (F % 8 == 0); zeros past n and F.  A wave writes one whole
// fragment (16 tokens x 32 columns, 1 KiB contiguous): lane l converts
// token 16 nt + l % 16, columns 32 ks + 8 (l / 16) .. + 8.
__global__ __launch_bounds__(256) void k_swiglu_to_frag(const float *g, const float *u, int n, int F,
                                                        int npad, int kpad, uint16_t *xb) {
  const int ksteps = kpad / 32, lane = threadIdx.x & 63;
  const long f = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (f >= (long)(npad / 16) * ksteps) return;
  const int nt = (int)(f / ksteps), ks = (int)(f % ksteps);
  const int t = 16 * nt + (lane & 15), c = 32 * ks + 8 * (lane >> 4);
  float v[8];
  if (t < n && c < F) {
    const float *gp = g + (long)t * F + c, *up = u + (long)t * F + c;
    const float4 g0 = *(const float4 *)gp, g1 = *(const float4 *)(gp + 4);
    const float4 u0 = *(const float4 *)up, u1 = *(const float4 *)(up + 4);
    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = gv[e] / (1.0f + expf(-gv[e])) * uv[e];
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = 0.f;
  }
  put_frag8(xb, frag_slot(t, c, ksteps), v);
}

// NEOX RoPE (cpu_path.rs:99-133, angle pos / theta^(2i/hd)) of q [n][nh*hd]
// and k [n][nkv*hd] in place for positions pos0 + t, and the f16 K/V rows
// (KvDtype::F16::pack, round to nearest even) into the cache.  One block
// per token.
__global__ __launch_bounds__(256) void k_rope_kv(float *q, float *k, const float *v, uint16_t *kc,
                                                 uint16_t *vc, int pos0, int nh, int nkv, int hd,
                                                 const float *rope_den) {
  __shared__ float sn[64], cs[64];
  const int t = blockIdx.x, pos = pos0 + t, half = hd / 2, kvd = nkv * hd;
  for (int i = threadIdx.x; i < half; i += 256) {
    float s, c;
    sincosf((float)pos / rope_den[i], &s, &c);
    sn[i] = s;
    cs[i] = c;
  }
  __syncthreads();
  for (int o = threadIdx.x; o < (nh + nkv) * half; o += 256) {
    const int hh = o / half, i = o % half;
    float *p = hh < nh ? q + (long)t * nh * hd + (long)hh * hd : k + (long)t * kvd + (long)(hh - nh) * hd;
    const float x0 = p[i], x1 = p[i + half];
    p[i] = x0 * cs[i] - x1 * sn[i];
    p[i + half] = x0 * sn[i] + x1 * cs[i];
  }
  __syncthreads();
  for (int o = threadIdx.x; o < kvd; o += 256) {
    kc[(long)pos * kvd + o] = __half_as_ushort(__float2half_rn(k[(long)t * kvd + o]));
    vc[(long)pos * kvd + o] = __half_as_ushort(__float2half_rn(v[(long)t * kvd + o]));
  }
}

// The same for the Q8_0 KV cache (KvDtype::Q8_0, src/model/mod.rs:574-583):
// the rotated k and v rows packed per 32 values exactly as the decode step
// packs them (scale = max|x| / 127 stored as f16, 1 for an all-zero block;
// codes = round(x / scale) clamped to [-127, 127]) into the int8 codes
// kc / vc [ctx][kvd] and the f16 scales ksc / vsc [ctx][kvd / 32].  32
// consecutive threads hold one block (kvd is a multiple of 32).
__global__ __launch_bounds__(256) void k_rope_kv_q8(float *q, float *k, const float *v, int8_t *kc,
                                                    int8_t *vc, uint16_t *ksc, uint16_t *vsc, int pos0,
                                                    int nh, int nkv, int hd, const float *rope_den) {
  __shared__ float sn[64], cs[64];
  const int t = blockIdx.x, pos = pos0 + t, half = hd / 2, kvd = nkv * hd;
  for (int i = threadIdx.x; i < half; i += 256) {
    float s, c;
    sincosf((float)pos / rope_den[i], &s, &c);
    sn[i] = s;
    cs[i] = c;
  }
  __syncthreads();
  for (int o = threadIdx.x; o < (nh + nkv) * half; o += 256) {
    const int hh = o / half, i = o % half;
    float *p = hh < nh ? q + (long)t * nh * hd + (long)hh * hd : k + (long)t * kvd + (long)(hh - nh) * hd;
    const float x0 = p[i], x1 = p[i + half];
    p[i] = x0 * cs[i] - x1 * sn[i];
    p[i + half] = x0 * sn[i] + x1 * cs[i];
  }
  __syncthreads();
  const int nbr = kvd / 32;
  for (int o0 = 0; o0 < kvd; o0 += 256) {  // (uniform trip count: the shuffles see whole blocks)
    const int o = o0 + (int)threadIdx.x;
    const bool live = o < kvd;
    const float kv = live ? k[(long)t * kvd + o] : 0.f, vv = live ? v[(long)t * kvd + o] : 0.f;
    float km = fabsf(kv), vm = fabsf(vv);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
      km = fmaxf(km, __shfl_xor(km, off, 32));
      vm = fmaxf(vm, __shfl_xor(vm, off, 32));
    }
    const float kscale = km > 0.f ? km / 127.0f : 1.0f, vscale = vm > 0.f ? vm / 127.0f : 1.0f;
    if (live) {
      kc[(long)pos * kvd + o] = (int8_t)fminf(fmaxf(roundf(kv / kscale), -127.f), 127.f);
      vc[(long)pos * kvd + o] = (int8_t)fminf(fmaxf(roundf(vv / vscale), -127.f), 127.f);
      if ((o & 31) == 0) {
        ksc[(long)pos * nbr + o / 32] = __half_as_ushort(__float2half_rn(kscale));
        vsc[(long)pos * nbr + o / 32] = __half_as_ushort(__float2half_rn(vscale));
      }
    }
  }
}

// KvDtype::Q8_0::unpack (src/model/mod.rs:595-602) of rows [0, npos) of one
// layer, code * f16 scale in fp32, rounded to f16 for the prefill
// attention's f16 operands: kf / vf [npos][kvd].
__global__ __launch_bounds__(256) void k_kv_q8_to_f16(const int8_t *kc, const int8_t *vc,
                                                      const uint16_t *ksc, const uint16_t *vsc,
                                                      long total, int kvd, uint16_t *kf, uint16_t *vf) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const long row = i / kvd, b = (i % kvd) / 32;
  const long sb = row * (kvd / 32) + b;
  kf[i] = __half_as_ushort(__float2half_rn((float)kc[i] * __half2float(__ushort_as_half(ksc[sb]))));
  vf[i] = __half_as_ushort(__float2half_rn((float)vc[i] * __half2float(__ushort_as_half(vsc[sb]))));
}

// Max / sum of x over the 4 lane groups (lanes 16 apart) of a wave, the
// same value in every lane (gfx950 lane swaps; each combination is
// symmetric, so every lane computes the identical bits).
__device__ __forceinline__ float lane_groups_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float lane_groups_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

constexpr int PF_Q = 64;  // queries per block
typedef short pf16x4s_t __attribute__((ext_vector_type(4)));
typedef short pf16x8s_t __attribute__((ext_vector_type(8)));
typedef uint32_t pu32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t pu32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void pf_lds_t;

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const pf_lds_t *)p;
}
// LDS reads as asm: K/V arrive by direct-to-LDS loads, and the compiler
// would drain all of those (vmcnt(0)) before any LDS read it emits itself.
// The results are not ready until lds_wait(), which takes them as in/out
// operands so that nothing uses them earlier.
__device__ __forceinline__ pu32x4_t lds_b128(uint32_t a) {
  pu32x4_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a) : "memory");
  return v;
}
// ds_read_b64_tr_b16: within each 16 lanes, the 4 halves lane r reads are
// elements 4r .. 4r+3 of a 64-element list; lane r receives elements r,
// r+16, r+32, r+48 of it.  With lane r pointing at row k0 + r/4, columns
// d0 + 4 (r % 4) of a row-major tile, lane r gets column d0 + r of rows
// k0 .. k0+3.
__device__ __forceinline__ pu32x2_t lds_tr16(uint32_t a) {
  pu32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(a) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void lds_wait(pu32x4_t (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; i++) asm volatile("" : "+v"(v[i]));
}
template <int N>
__device__ __forceinline__ void lds_wait(pu32x2_t (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; i++) asm volatile("" : "+v"(v[i]));
}
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// K / V tile of 64 keys in LDS: row-major, HD/8 blocks of 16 B per row,
// block b of row r stored at block b ^ (r % (HD/8)) (the reads of a
// fragment then spread over the banks).
template <int HD>
__device__ __forceinline__ uint32_t kv_slot(int row, int blk) {
  constexpr int NB = HD / 8;
  return (uint32_t)(row * NB + (blk ^ (row & (NB - 1)))) * 16u;
}

// Causal attention of queries t = 0 .. n-1 (position pos0 + t, head h)
// over cache rows 0 .. pos0 + t (attention_into, cpu_path.rs:141-194:
// scores q.k / sqrt(hd), softmax, weighted sum of V), flash-style: block
// (64-query tile, head h), 8 waves: 4 of 16 queries for each half of the
// 64-key chunks (even / odd), merged at the end.  K and V go straight
// from memory to LDS (global_load_lds_dwordx4, no registers;
// two buffers, the next chunk loading while this one is used), one
// barrier per chunk.
// Both products run transposed on v_mfma_f32_16x16x32_f16 so that no
// operand needs a shuffle or an LDS round trip:
//   S^T = K . q^T   A = K rows from LDS, B = q (registers): a lane holds 4
//                   keys (4 (lane/16) + i of each 16-key tile) of query
//                   lane % 16, so the online softmax of its query is its
//                   own 16 values plus two lane swaps across the groups;
//   O^T = V^T . P^T B = the lane's own probabilities (the depth runs over
//                   the keys in the order the S^T layout holds them: slot
//                   8 g + j is key 16 t0 + 4 g + j, j < 4, and 16 t1 + 4 g +
//                   j - 4 otherwise), A = V^T in that key order, read from
//                   the row-major V by the gfx950 transpose load
//                   ds_read_b64_tr_b16.
// O^T puts one query per lane too, so the rescale by exp2(m_old - m_new)
// is per lane.  K and V are f16 already; q (scaled by a power of two) and
// the probabilities are split into f16 hi + lo parts, so the products are
// exact in fp32.  The softmax runs in base 2 (scores scaled by log2 e).
template <int HD>
__global__ __launch_bounds__(512) void k_attn_prefill(const float *q, const uint16_t *kc,
                                                      const uint16_t *vc, int pos0, int n, int nh,
                                                      int group, uint16_t *xb) {
  constexpr int KS = HD / 32, DT = HD / 16;
  constexpr int NB = HD / 8;                 // 16-byte blocks per K/V row
  constexpr int TILE = 64 * HD * 2;          // bytes of one K or V tile
  constexpr int NDMA = 64 * NB / 256;        // 16-byte loads per thread per tile (4 waves)
  // [key half][buffer][K, V]: waves 0-3 take the even chunks, waves 4-7
  // the odd ones, each half with its own two buffers.
  __shared__ __align__(16) uint8_t kvs[2][2][2][TILE];
  __shared__ float red[8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g4 = 4 * (lane >> 4);
  const int half = wave >> 2, wq = wave & 3;  // key half, query wave
  // Block b -> (query tile, query head): the group's heads of one (tile,
  // KV head) item G sit 8 blocks apart, i.e. on one XCD (consecutive blocks
  // go to consecutive XCDs), so they share the K/V chunks in one L2.
  const int nkv = nh / group, nqt = (n + PF_Q - 1) / PF_Q;
  const int bx = blockIdx.x % 8, bk = blockIdx.x / 8;
  const int G = 8 * (bk / group) + bx, gi = bk % group;
  if (G >= nqt * nkv) return;
  const int kh = G % nkv, qt0 = (G / nkv) * PF_Q, h = kh * group + gi;
  const int kvd = nkv * HD;
  const uint16_t *kbase = kc + (long)kh * HD, *vbase = vc + (long)kh * HD;

  const int tlast = min(qt0 + PF_Q, n) - 1;
  const int kend = pos0 + tlast + 1;  // keys [0, kend)
  const int nch = (kend + 63) / 64;
  // Chunk c (of this wave's half, c % 2 == half) into buffer (c / 2) & 1:
  // load j of query wave wq fills the 64 slots s = 64 (NDMA wq + j) + lane,
  // slot s = row s / NB, stored block s % NB (global block (s % NB) ^
  // (row % NB)); rows past kend - 1 repeat it.
  auto dma = [&](int c) {
    uint8_t *kt = kvs[half][(c >> 1) & 1][0], *vt = kvs[half][(c >> 1) & 1][1];
#pragma unroll
    for (int j = 0; j < NDMA; j++) {
      const int sb = 64 * (NDMA * wq + j), sl = sb + lane;
      const int row = sl / NB, blk = (sl % NB) ^ (row & (NB - 1));
      const long r = min(64 * c + row, kend - 1);
      __builtin_amdgcn_global_load_lds(kbase + r * kvd + 8 * blk, (pf_lds_t *)(kt + 16 * sb), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vbase + r * kvd + 8 * blk, (pf_lds_t *)(vt + 16 * sb), 16, 0, 0);
    }
  };
  if (half < nch) dma(half);

  // q fragments (the B operand of S^T): lane column = query qt0 + 16 wq +
  // lane % 16, dims 8 (lane / 16) + 32 ks .. + 8.
  const int tq = qt0 + 16 * wq + (lane & 15);
  float qv[KS][8];
  float qm = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ks++) {
    const float *src = q + (long)tq * nh * HD + (long)h * HD + 8 * (lane >> 4) + 32 * ks;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      qv[ks][e] = tq < n ? src[e] : 0.f;
      qm = fmaxf(qm, fabsf(qv[ks][e]));
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) qm = fmaxf(qm, __shfl_xor(qm, off, 64));
  if (lane == 0) red[wave] = qm;
  __syncthreads();
  qm = red[0];
#pragma unroll
  for (int w = 1; w < 8; w++) qm = fmaxf(qm, red[w]);
  int ex = 0;
  (void)frexpf(qm, &ex);
  const float qscale = qm > 0.f ? ldexpf(1.0f, 10 - ex) : 1.0f;
  // scores in base-2 units: s2 = (q.k / sqrt(hd)) * log2(e), so that
  // exp(s - m) = exp2(s2 - m2)
  const float s2scale = (1.0f / qscale) / sqrtf((float)HD) * 1.4426950408889634f;
  pf16x8_t qhi[KS], qlo[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ks++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float x = qv[ks][e] * qscale;
      const _Float16 hi = (_Float16)x;
      qhi[ks][e] = hi;
      qlo[ks][e] = (_Float16)(x - (float)hi);
    }

  float mrow = -INFINITY, lrow = 0.f;  // of query tq over this half's keys
  pf32x4_t O[DT];                      // O^T: dims 16 d + 4 (lane / 16) + i of query tq
#pragma unroll
  for (int d = 0; d < DT; d++) O[d] = pf32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int cp = 0; cp < nch; cp += 2) {  // chunk pairs: both halves meet at every barrier
    const int c = cp + half;
    const uint32_t kt = lds_addr(kvs[half][(c >> 1) & 1][0]), vt = lds_addr(kvs[half][(c >> 1) & 1][1]);
    vm_wait_all();     // this wave's loads of chunk c
    __syncthreads();   // everyone's; and the chunks before are no longer read
    if (c + 2 < nch) dma(c + 2);
    if (c >= nch) continue;

    // S^T of 64 keys (4 tiles) x this wave's 16 queries
    float sv[4][4];
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
      pu32x4_t kf[KS];
      const int row = 16 * ct + (lane & 15);
#pragma unroll
      for (int ks = 0; ks < KS; ks++) kf[ks] = lds_b128(kt + kv_slot<HD>(row, (lane >> 4) + 4 * ks));
      lds_wait(kf);
      pf32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ks++) {
        const pf16x8_t a = __builtin_bit_cast(pf16x8_t, kf[ks]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qhi[ks], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qlo[ks], acc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int key = 64 * c + 16 * ct + g4 + i;
        // queries past n stay finite (discarded); past the causal limit: -inf
        sv[ct][i] = tq >= n ? 0.f : key > pos0 + tq ? -INFINITY : acc[i] * s2scale;
      }
    }
    // online softmax of query tq: its 64 scores are 16 per lane group
    float mx = sv[0][0];
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
#pragma unroll
      for (int i = 0; i < 4; i++) mx = fmaxf(mx, sv[ct][i]);
    mx = lane_groups_max(mx);
    // (a chunk wholly past a query's causal limit leaves mx = -inf: the
    // state is unchanged; chunk 0 is in every query's range)
    const float mnew = fmaxf(mrow, mx);
    const float alpha = mnew == -INFINITY ? 1.f : exp2f(mrow - mnew);
    float ps = 0.f;
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        sv[ct][i] = mnew == -INFINITY ? 0.f : exp2f(sv[ct][i] - mnew);
        ps += sv[ct][i];
      }
    lrow = lrow * alpha + lane_groups_sum(ps);
    mrow = mnew;
#pragma unroll
    for (int d = 0; d < DT; d++)
#pragma unroll
      for (int i = 0; i < 4; i++) O[d][i] *= alpha;
    // O^T += V^T . P^T over the chunk's keys, 2 depth steps of 32
    const int r = lane & 15;
#pragma unroll
    for (int st = 0; st < 2; st++) {
      const int t0 = 2 * st, t1 = 2 * st + 1;
      pf16x8_t bh, bl;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const _Float16 h0 = (_Float16)sv[t0][i], h1 = (_Float16)sv[t1][i];
        bh[i] = h0;
        bh[4 + i] = h1;
        bl[i] = (_Float16)(sv[t0][i] - (float)h0);
        bl[4 + i] = (_Float16)(sv[t1][i] - (float)h1);
      }
      // lane r: rows k0 + r/4, 8 bytes at column 16 d + 4 (r % 4)
      pu32x2_t vf[2 * DT];
#pragma unroll
      for (int d = 0; d < DT; d++)
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
          const int row = 16 * (tt ? t1 : t0) + g4 + (r >> 2);
          const int col = 16 * d + 4 * (r & 3);
          vf[2 * d + tt] = lds_tr16(vt + kv_slot<HD>(row, col >> 3) + 2 * (col & 7));
        }
      lds_wait(vf);
#pragma unroll
      for (int d = 0; d < DT; d++) {
        const pu32x4_t a4 = {vf[2 * d].x, vf[2 * d].y, vf[2 * d + 1].x, vf[2 * d + 1].y};
        const pf16x8_t a = __builtin_bit_cast(pf16x8_t, a4);
        O[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh, O[d], 0, 0, 0);
        O[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl, O[d], 0, 0, 0);
      }
    }
  }
  // Merge the odd half into the even one: M = max(m0, m1),
  // O = O0 e^(m0 - M) + O1 e^(m1 - M), l likewise (the K/V buffers are free
  // once every wave has passed the barrier).
  __syncthreads();
  float *xch = (float *)&kvs[0][0][0][0];  // [query wave][lane][2 + 4 DT]
  constexpr int XW = 2 + 4 * DT;
  if (half == 1) {
    float *p = xch + (wq * 64 + lane) * XW;
    p[0] = mrow;
    p[1] = lrow;
#pragma unroll
    for (int d = 0; d < DT; d++)
#pragma unroll
      for (int i = 0; i < 4; i++) p[2 + 4 * d + i] = O[d][i];
  }
  __syncthreads();
  // The output goes straight into the o GEMM's bf16 X fragments (row tq,
  // columns h HD + 16 d + 4 (lane / 16) + i): lane groups 0 and 2 take the
  // 4 values of groups 1 and 3 (lane swap) and store 8 columns each.
  if (half == 0) {
    const float *p = xch + (wq * 64 + lane) * XW;
    const float m1 = p[0], l1 = p[1];
    const float M = fmaxf(mrow, m1);  // mrow is finite: chunk 0 is in this half
    const float f0 = exp2f(mrow - M), f1 = m1 == -INFINITY ? 0.f : exp2f(m1 - M);
    const float L = lrow * f0 + l1 * f1;
    const int ksteps = nh * HD / 32;
#pragma unroll
    for (int d = 0; d < DT; d++) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float o = (O[d][i] * f0 + p[2 + 4 * d + i] * f1) / L;
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(o), __float_as_uint(o), false, false);
        v[i] = __uint_as_float(r[0]);      // this group's (even) value
        v[4 + i] = __uint_as_float(r[1]);  // the odd group's
      }
      if (((lane >> 4) & 1) == 0 && tq < n)
        put_frag8(xb, frag_slot(tq, h * HD + 16 * d + 8 * (lane >> 5), ksteps), v);
    }
  }
}

// ------------------------------------------------------------------ host
static int round_up(int v, int m) { return (v + m - 1) / m * m; }

// The largest K-split partial buffer of any launch of a pass of up to nmax
// tokens.  Passes of up to 256 tokens use taller row tiles (fewer tiles, a
// larger split), so both tile regimes are sized at their largest batch.
size_t prefill_part_floats(const DecodeLaunch &m, int nmax, int num_cus) {
  size_t best = 0;
  for (int nn : {std::min(nmax, 256), nmax})
  for (int L = 0; L < m.n_layers; L++) {
    const int nmax = nn;
    const gq_weight *qkv[3] = {m.wq[L], m.wk[L], m.wv[L]};
    for (int i = 0; i < 3; i++) best = std::max(best, gemm_part_floats(&qkv[i], 1, nmax, num_cus, false));
    if (qkv[0]->L.dtype == qkv[1]->L.dtype && qkv[1]->L.dtype == qkv[2]->L.dtype)
      best = std::max(best, gemm_part_floats(qkv, 3, nmax, num_cus, false));
    best = std::max(best, gemm_part_floats(&m.wo[L], 1, nmax, num_cus, true));
    const gq_weight *gu[2] = {m.wgate[L], m.wup[L]};
    best = std::max(best, gemm_part_floats(gu, 2, nmax, num_cus, false));
    best = std::max(best, gemm_part_floats(&m.wdown[L], 1, nmax, num_cus, true));
  }
  return best;
}

// One pass of n <= PREFILL_MAX tokens (tokens_dev) at positions pos0 ..
// pos0 + n - 1; logits of the last position into m.logits.
hipError_t launch_prefill(const DecodeLaunch &m, const PrefillBufs &b, const int *tokens_dev, int n,
                          int pos0, int num_cus, hipStream_t s) {
  if (n < 1 || n > PREFILL_MAX) return hipErrorInvalidValue;
  const int H = m.hidden, hd = m.head_dim, nh = m.n_heads, nkv = m.n_kv_heads;
  const int kvd = nkv * hd, qd = nh * hd, F = m.ffn, group = nh / nkv;
  const int npad = round_up(n, GEMM_NPAD);
  hipError_t e;
  hipLaunchKernelGGL(k_embed_rows, dim3(n), dim3(256), 0, s, m.embd, tokens_dev, H, b.x);
  int pending = 0;  // K split of partials left for the next norm to add into x
  for (int L = 0; L < m.n_layers; L++) {
    hipLaunchKernelGGL(k_norm_to_frag, dim3(npad), dim3(256), 0, s, b.x, m.attn_norm[L], n, H,
                       round_up(H, 256), m.eps, b.xb, b.part, pending);
    pending = 0;
    // q, k, v: one launch per distinct dtype (attn_v is Q6_K in some files)
    const gq_weight *qkv[3] = {m.wq[L], m.wk[L], m.wv[L]};
    float *outs[3] = {b.q, b.k, b.v};
    bool done[3] = {false, false, false};
    for (int i = 0; i < 3; i++) {
      if (done[i]) continue;
      const gq_weight *grp[3];
      float *gout[3];
      int c = 0;
      for (int j = i; j < 3; j++)
        if (!done[j] && qkv[j]->L.dtype == qkv[i]->L.dtype) {
          grp[c] = qkv[j];
          gout[c++] = outs[j];
          done[j] = true;
        }
      if ((e = launch_gemm_bf16(grp, gout, c, b.xb, n, b.part, false, num_cus, s)) != hipSuccess) return e;
    }
    uint16_t *kc, *vc;  // the f16 K/V rows the attention reads
    if (m.kv_q8) {
      // pack the new rows into the Q8_0 cache, then attend over the
      // unpacked rows of every position, the new ones included (run_batch
      // writes the cache and reads it back, cpu_path.rs:904-906)
      int8_t *kq = (int8_t *)m.kcache + (long)L * m.ctx * kvd, *vq = (int8_t *)m.vcache + (long)L * m.ctx * kvd;
      uint16_t *ks = m.kscale + (long)L * m.ctx * (kvd / 32), *vs = m.vscale + (long)L * m.ctx * (kvd / 32);
      hipLaunchKernelGGL(k_rope_kv_q8, dim3(n), dim3(256), 0, s, b.q, b.k, b.v, kq, vq, ks, vs, pos0,
                         nh, nkv, hd, m.rope_den);
      const long total = (long)(pos0 + n) * kvd;
      hipLaunchKernelGGL(k_kv_q8_to_f16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, kq, vq,
                         ks, vs, total, kvd, b.kf, b.vf);
      kc = b.kf;
      vc = b.vf;
    } else {
      kc = m.kcache + (long)L * m.ctx * kvd;
      vc = m.vcache + (long)L * m.ctx * kvd;
      hipLaunchKernelGGL(k_rope_kv, dim3(n), dim3(256), 0, s, b.q, b.k, b.v, kc, vc, pos0, nh, nkv, hd,
                         m.rope_den);
    }
    const int items = (n + PF_Q - 1) / PF_Q * nkv;  // (query tile, KV head)
    const dim3 ag(8 * group * ((items + 7) / 8));
    if (hd == 128)
      hipLaunchKernelGGL(k_attn_prefill<128>, ag, dim3(512), 0, s, b.q, kc, vc, pos0, n, nh, group, b.xb);
    else
      hipLaunchKernelGGL(k_attn_prefill<64>, ag, dim3(512), 0, s, b.q, kc, vc, pos0, n, nh, group, b.xb);
    float *xo[1] = {b.x};
    if ((e = launch_gemm_bf16(&m.wo[L], xo, 1, b.xb, n, b.part, true, num_cus, s, &pending)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(k_norm_to_frag, dim3(npad), dim3(256), 0, s, b.x, m.ffn_norm[L], n, H,
                       round_up(H, 256), m.eps, b.xb, b.part, pending);
    pending = 0;
    // h = silu(gate . xn) * (up . xn) as the down GEMM's X: in the gate/up
    // GEMM's epilogue (into xh: other blocks are still reading xb), or,
    // for batches on the ring kernel and mixed gate/up types, g and u
    // then k_swiglu_to_frag
    const uint16_t *hx = b.xh;
    e = launch_gemm_bf16_swiglu(m.wgate[L], m.wup[L], b.xb, n, b.xh, num_cus, s);
    if (e == hipErrorNotSupported) {
      const gq_weight *gu[2] = {m.wgate[L], m.wup[L]};
      float *guo[2] = {b.g, b.u};
      if ((e = launch_gemm_bf16(gu, guo, 2, b.xb, n, b.part, false, num_cus, s)) != hipSuccess) return e;
      const int kpf = round_up(F, 256);
      hipLaunchKernelGGL(k_swiglu_to_frag, dim3((int)(((long)npad / 16 * (kpf / 32) + 3) / 4)), dim3(256), 0,
                         s, b.g, b.u, n, F, npad, kpf, b.xb);
      hx = b.xb;
    } else if (e != hipSuccess) {
      return e;
    }
    // (the next layer's norm does the reduction; the head reads x itself)
    if ((e = launch_gemm_bf16(&m.wdown[L], xo, 1, hx, n, b.part, true, num_cus, s,
                              L + 1 < m.n_layers ? &pending : nullptr)) != hipSuccess)
      return e;
  }
  // logits of RMSNorm(x[n - 1]) (the decode head matvec)
  MvIn hin;
  hin.src = MV_NORM;
  hin.x = b.x + (long)(n - 1) * H;
  hin.nw = m.output_norm;
  hin.eps = m.eps;
  hin.q8k = true;  // the head: matmul_into (cpu_path.rs:815)
  float *lo[1] = {m.logits};
  return matvec_launch(&m.lm_head, 1, hin, lo, s);
}

}  // namespace gq
