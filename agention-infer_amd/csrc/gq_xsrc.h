// gq_xsrc.h -- where a matvec's input vector comes from, shared by the
// matvec kernels: plain x, the SwiGLU of the gate/up outputs, or the
// RMSNorm of the residual stream (with the residual add in front).
#pragma once
#include <hip/hip_runtime.h>

#include "gq_device.h"

namespace gq {

// 16 consecutive input values from element e0 on, in two steps so that a
// wave can issue its loads and use them later: load_raw16 loads from
// clamped addresses (every address in [0, k)), mask16 zeroes the values
// past k.
// (Global-address-space loads: a flat load also counts against the LDS
// counter, and the compiler then waits for every outstanding load first.)
typedef float xf32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) float gfloat;
typedef const __attribute__((address_space(1))) xf32x4 gfloat4;
template <bool K4>
__device__ __forceinline__ void load_raw16(const float *xp, int k, int e0, float (&v)[16]) {
  gfloat *x = (gfloat *)xp;
  if (K4) {  // k % 4 == 0: clamped vector loads
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const xf32x4 w = *(gfloat4 *)(x + min(e0 + 4 * q, k - 4));
      v[4 * q + 0] = w.x;
      v[4 * q + 1] = w.y;
      v[4 * q + 2] = w.z;
      v[4 * q + 3] = w.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = x[min(e0 + i, k - 1)];
  }
}
__device__ __forceinline__ void mask16(int k, int e0, float (&v)[16]) {
#pragma unroll
  for (int i = 0; i < 16; i++) v[i] = e0 + i < k ? v[i] : 0.f;
}
template <bool K4>
__device__ __forceinline__ void load_x16(const float *x, int k, int e0, float (&xv)[16]) {
  load_raw16<K4>(x, k, e0, xv);
  mask16(k, e0, xv);
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
  __device__ __forceinline__ void issue(int e0, Raw &r) const { load_raw16<K4>(x, k, e0, r.v); }
  __device__ __forceinline__ void make(const Raw &r, int e0, float (&xv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = r.v[i];
    mask16(k, e0, xv);
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
    load_raw16<K4>(g, k, e0, r.g);
    load_raw16<K4>(u, k, e0, r.u);
  }
  __device__ __forceinline__ void make(const Raw &r, int e0, float (&xv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float gi = e0 + i < k ? r.g[i] : 0.f, ui = e0 + i < k ? r.u[i] : 0.f;
      xv[i] = gi / (1.0f + expf(-gi)) * ui;
    }
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
  __device__ __forceinline__ void accum_ss(const Raw &q, int e0) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float v = e0 + i < k ? (r ? q.x[i] + q.r[i] : q.x[i]) : 0.f;
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
    // (r's loads are unconditional, from x without a residual, so that the
    // waits for these loads count exactly the loads behind them)
    load_raw16<K4>(x, k, e0, q.x);
    load_raw16<K4>(r ? r : x, k, e0, q.r);
    load_raw16<K4>(nw, k, e0, q.w);
  }
  __device__ __forceinline__ void make(const Raw &q, int e0, float (&xv)[16]) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      v[i] = e0 + i < k ? (r ? q.x[i] + q.r[i] : q.x[i]) : 0.f;
      const bool in = e0 + i < k;
      if constexpr (EXACT) {
        xv[i] = in ? q.w[i] * v[i] / rms : 0.f;
      } else {
        ss += v[i] * v[i];
        xv[i] = in ? q.w[i] * v[i] : 0.f;
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
