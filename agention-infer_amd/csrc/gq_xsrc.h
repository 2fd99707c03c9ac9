// gq_xsrc.h -- where a matvec's input vector comes from, shared by the
// matvec kernels: plain x, the SwiGLU of the gate/up outputs, or the
// RMSNorm of the residual stream (with the residual add in front).
#pragma once
#include <hip/hip_runtime.h>

#include "gq_device.h"

namespace gq {

template <bool K4>
__device__ __forceinline__ void load_x16(const float *x, int k, int e0, float (&xv)[16]) {
  if (K4) {  // k % 4 == 0: clamped vector loads, zeroed past k
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int e = e0 + 4 * q;
      const float4 v = *(const float4 *)(x + min(e, k - 4));
      const bool in = e < k;
      xv[4 * q + 0] = in ? v.x : 0.f;
      xv[4 * q + 1] = in ? v.y : 0.f;
      xv[4 * q + 2] = in ? v.z : 0.f;
      xv[4 * q + 3] = in ? v.w : 0.f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float v = x[min(e0 + i, k - 1)];
      xv[i] = e0 + i < k ? v : 0.f;
    }
  }
}

// x sources.  issue() starts the loads of 16 consecutive input values
// (zero past k) into a Raw record, make() turns a Raw record into the 16
// values to stage; pre_barrier()/scale() give a factor applied to every
// row sum (1 except for the normalised source).
template <bool K4>
struct XPlain {
  const float *x;
  int k;
  struct Raw { float v[16]; };
  __device__ __forceinline__ void issue(int e0, Raw &r) const { load_x16<K4>(x, k, e0, r.v); }
  __device__ __forceinline__ void make(const Raw &r, int, float (&xv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = r.v[i];
  }
  __device__ __forceinline__ void pre_barrier(float *) const {}
  __device__ __forceinline__ float scale(const float *) const { return 1.f; }
};

// silu(g) * u of the gate/up outputs (the SwiGLU of ffn_gate_up,
// src/model/llama/cpu_path.rs:225-227); zero past k since silu(0) * 0 = 0.
template <bool K4>
struct XSwiGLU {
  const float *g, *u;
  int k;
  struct Raw { float g[16], u[16]; };
  __device__ __forceinline__ void issue(int e0, Raw &r) const {
    load_x16<K4>(g, k, e0, r.g);
    load_x16<K4>(u, k, e0, r.u);
  }
  __device__ __forceinline__ void make(const Raw &r, int, float (&xv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = r.g[i] / (1.0f + expf(-r.g[i])) * r.u[i];
  }
  __device__ __forceinline__ void pre_barrier(float *) const {}
  __device__ __forceinline__ float scale(const float *) const { return 1.f; }
};

// RMSNorm of the residual stream (rms_norm_into, cpu_path.rs:67-74) with the
// residual add in front (x += proj, cpu_path.rs:780-782 and 806-808):
// v = x + r, the staged input is nw * v, and since every row sum is linear
// in the input, 1 / rms(v) multiplies the row sums instead of the inputs.
// xo (block 0 only) receives v, the new residual stream.
// EXACT (inputs quantized to Q8_K, which is not linear in the input): the
// staged value is rms_norm_into's w * v / rms itself, with rms from a
// first pass over the block's inputs (exact() / set_rms()).
template <bool K4, bool EXACT = false>
struct XNorm {
  const float *x, *r, *nw;
  float *xo;
  int k;
  float eps;
  float ss = 0.f;
  float rms = 1.f;
  struct Raw { float x[16], r[16], w[16]; };
  static constexpr bool kExact = EXACT;
  // sum of squares of the residual-added input (first pass of EXACT)
  __device__ __forceinline__ void accum_ss(const Raw &q) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float v = r ? q.x[i] + q.r[i] : q.x[i];
      ss += v * v;
    }
  }
  __device__ __forceinline__ void set_rms(const float *red) {
    const int nw = blockDim.x >> 6;
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    rms = sqrtf(t / (float)k + eps);
  }
  __device__ __forceinline__ void issue(int e0, Raw &q) const {
    load_x16<K4>(x, k, e0, q.x);
    if (r) load_x16<K4>(r, k, e0, q.r);
    load_x16<K4>(nw, k, e0, q.w);
  }
  __device__ __forceinline__ void make(const Raw &q, int e0, float (&xv)[16]) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      v[i] = r ? q.x[i] + q.r[i] : q.x[i];
      if constexpr (EXACT) {
        xv[i] = q.w[i] * v[i] / rms;
      } else {
        ss += v[i] * v[i];
        xv[i] = q.w[i] * v[i];
      }
    }
    if (xo) {
      if (K4) {
#pragma unroll
        for (int j = 0; j < 4; j++)
          if (e0 + 4 * j < k)
            *(float4 *)(xo + e0 + 4 * j) = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
      } else {
#pragma unroll
        for (int i = 0; i < 16; i++)
          if (e0 + i < k) xo[e0 + i] = v[i];
      }
    }
  }
  __device__ __forceinline__ void pre_barrier(float *red) const {
    float t = ss;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  }
  __device__ __forceinline__ float scale(const float *red) const {
    if constexpr (EXACT) return 1.f;
    const int nw = blockDim.x >> 6;
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return 1.0f / sqrtf(t / (float)k + eps);
  }
};

template <class XS> struct IsExact { static constexpr bool value = false; };
template <bool K4> struct IsExact<XNorm<K4, true>> { static constexpr bool value = true; };

}  // namespace gq
