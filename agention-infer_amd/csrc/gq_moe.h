// gq_moe.h -- device pieces shared by the MoE kernels (the v_dot4 ones in
// gq_matvec.hip and the MFMA ones in gq_mvq.hip): in-kernel routing of one
// (token, slot) pair and the staged input of the down projection.
#pragma once
#include <hip/hip_runtime.h>

#include "gq_device.h"
#include "gq_internal.h"
#include "gq_xsrc.h"

namespace gq {

// Routing of pair p = (token p / top_k, slot p % top_k) inside a block of
// NTH threads (every thread calls it; it holds __syncthreads): rank the
// token's logits (rank(i) = #{o : l_o > l_i or (l_o == l_i and o < i)}, so
// ties go to the lower index, like k_moe_route) and return the expert of
// rank p % top_k.  With store, thread 0 also writes ids[p] and the softmax
// weight w[p] over all experts (top-k selection and weights of
// docs/08-moe-routing.md:24-30).  n_experts <= MOE_ROUTE_MAX.
template <int NTH>
__device__ __forceinline__ int moe_route_pair(const MoeArgs &a, int p, bool store) {
  constexpr int NW = NTH / 64;
  __shared__ __align__(16) float lv[MOE_ROUTE_MAX];
  __shared__ __align__(16) unsigned long long key[MOE_ROUTE_MAX];
  __shared__ int prank[4][MOE_ROUTE_MAX / 4];
  __shared__ float rmax[NW], rsum[NW];
  __shared__ int eid_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tok = p / a.top_k, slot = p - tok * a.top_k;
  const int E = a.n_experts;
  const float *lg = a.logits + (long)tok * E;
  // Logits padded with -inf to a multiple of 16.  "o beats i" (l_o > l_i,
  // or l_o == l_i and o < i) is one integer compare of 64-bit keys: the
  // logit's bits mapped to an ordered integer (-0 taken as +0, so the two
  // tie) above 4095 - index.  A NaN logit beats nothing (key 0) and, like
  // the float compares it stands for, is beaten by nothing (rank 0).
  const int E16 = (E + 15) & ~15;
  if (tid == 0) eid_s = 0;  // (NaN logits can leave a rank unused)
  float mx = -INFINITY;
  for (int i = tid; i < E16; i += NTH) {
    const float l = i < E ? lg[i] : -INFINITY;
    lv[i] = l;
    mx = fmaxf(mx, l);
    const uint32_t u = __float_as_uint(l + 0.0f);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    key[i] = l != l ? 0ull : ((unsigned long long)ord << 12) | (uint32_t)(4095 - i);
  }
  __syncthreads();
  // With nq E16 threads or more (nq = 4 or 2), thread (q, i) counts over
  // part q of o.
  const int nq = 4 * E16 <= NTH ? 4 : 2 * E16 <= NTH ? 2 : 1, span = E16 / nq;
  for (int t = tid; t < nq * E16; t += NTH) {
    const int i = t % E16, q = t / E16;
    const unsigned long long me = key[i];
    int rank = 0;
#pragma unroll 4
    for (int o = q * span; o < (q + 1) * span; o += 2) {
      const ulonglong2 ov = *(const ulonglong2 *)&key[o];
      rank += ov.x > me;
      rank += ov.y > me;
    }
    if (me == 0ull) rank = 0;  // NaN
    if (nq > 1) prank[q][i] = rank;
    else if (i < E && rank == slot) eid_s = i;
  }
  if (nq > 1) {
    __syncthreads();
    for (int i = tid; i < E; i += NTH) {
      int r = 0;
      for (int q = 0; q < nq; q++) r += prank[q][i];
      if (r == slot) eid_s = i;
    }
  }
  if (store) {  // softmax over all experts
    mx = wave_max(mx);
    if (lane == 0) rmax[wave] = mx;
    __syncthreads();
    mx = rmax[0];
    for (int w = 1; w < NW; w++) mx = fmaxf(mx, rmax[w]);
    float sum = 0.f;
    for (int i = tid; i < E; i += NTH) sum += expf(lv[i] - mx);
    sum = wave_sum(sum);
    if (lane == 0) rsum[wave] = sum;
  }
  __syncthreads();
  const int e = __builtin_amdgcn_readfirstlane(eid_s);
  if (store && tid == 0) {
    float sum = 0.f;
    for (int w = 0; w < NW; w++) sum += rsum[w];
    a.ids[p] = e;
    a.w[p] = expf(lv[e] - mx) / sum;
  }
  return e;
}

// The top_k inputs h_(t, s) of a token, one after another, each padded to
// span elements: element e is element e % span of slot e / span (zero past
// f).
template <bool K4>
struct XSlots {
  const float *h;  // [pairs][f]
  int f, span, top_k, p0;
  struct Raw { float v[16]; };
  __device__ __forceinline__ int first(int e0) const {  // element index in its slot
    const int s = min(e0 / span, top_k - 1), i0 = e0 - s * span;
    return i0 < span ? i0 : span;
  }
  __device__ __forceinline__ void issue(int e0, Raw &r) const {
    const int s = min(e0 / span, top_k - 1);
    load_raw16<K4>(h + (long)(p0 + s) * f, f, first(e0), r.v);
  }
  __device__ __forceinline__ void make(const Raw &r, int e0, float (&xv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = r.v[i];
    mask16(f, first(e0), xv);
  }
  __device__ __forceinline__ void pre_barrier(float *) const {}
  __device__ __forceinline__ float scale(const float *) const { return 1.f; }
};

}  // namespace gq
