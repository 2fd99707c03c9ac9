// gq_matvec.hip -- batch-1 decode matvec y = W . x for Q8_0, Q4_K, Q5_K,
// Q6_K and IQ3_XXS weights (gfx950, wave64).
//
// Replaces the reference's per-row dot kernels (src/quant/q8_0.rs:58-90,
// q4_k.rs:95-212, q5_k.rs:189-317, q6_k.rs:82-131) driven row-parallel by
// WeightMap::matmul_into (src/model/mod.rs:362-403).  It does not follow
// the reference GPU kernels (src/ops/kernels_wgpu.rs:1067-1706).
//
// Design (HBM-bound; every weight byte is read exactly once):
//  * Weights sit in the wave-tiled layout (gq_layout.h): one lane owns one
//    256-element unit, and a wave-wide 128-bit load reads 1 KiB of
//    contiguous HBM with a nontemporal hint.  Each lane keeps its next unit
//    in flight while it computes the current one.
//  * x is staged per block in LDS as fixed-point int8 "limbs": for each run
//    of 32 elements, s = max|x| / (127 * 2^16), X = rint(x / s) (|X| <=
//    127 * 2^16) and X = x2 * 2^16 + x1 * 2^8 + x0 with signed bytes.
//    The representation error is <= s/2 (relative 6e-8 of the run's max,
//    the same order as fp32 rounding).
//  * The weight integers (nibbles, 6-bit codes, int8) meet the limbs in
//    v_dot4_i32_i8: 32 elements cost 8 x 3 integer dot instructions, exact,
//    and the block / sub-block scales are applied once per run:
//      Q4_K  sum (d*sc*q - dmin*m) x = d*sc*s*sum(q X) - dmin*m*sum(x)
//      Q6_K  sum d*sc*(q - 32) x     = d*sc*s*(sum(q X) - 32*sum(X))
//      Q8_0  sum d*q*x               = d*s*sum(q X)
//  * Per-unit partial sums go to LDS and are reduced per row in a fixed
//    order (deterministic results).
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "gq_device.h"
#include "gq_internal.h"

namespace gq {

constexpr int LIMB_STRIDE = 272;  // LDS bytes per 256-element block of one limb (16 B pad)

constexpr int AUX_STRIDE = 144;   // LDS bytes per unit of the per-16-run records (16 B pad)

// Per 16-run record: {s of its 32-run, c} with c = sum(x) of the 32-run
// (Q4_K/Q5_K) or sum(X) of the 16-run as int bits (Q6_K).  The 16 B pads
// put the records of consecutive units in different LDS bank groups.
struct Smem {
  uint8_t *l2, *l1, *l0;  // limbs, LIMB_STRIDE bytes per 256 elements
  float2 *aux;            // AUX_STRIDE bytes per unit
  uint32_t *grid;         // IQ3_XXS codebook
  float *part;            // per-wave per-unit partial sums
  float *red;             // 16 floats of block reduction scratch
};

__host__ __device__ inline size_t smem_layout(int units, int part_total, Smem *s, char *base) {
  size_t o = 0;
  auto take = [&](size_t n) { size_t r = o; o += (n + 15) & ~(size_t)15; return r; };
  const size_t limb = (size_t)units * LIMB_STRIDE;
  const size_t o2 = take(limb), o1 = take(limb), o0 = take(limb);
  const size_t oaux = take((size_t)units * AUX_STRIDE), og = take(1024);
  const size_t op = take((size_t)part_total * 4);
  const size_t ored = take(64);
  if (s) {
    s->red = (float *)(base + ored);
    s->l2 = (uint8_t *)(base + o2);
    s->l1 = (uint8_t *)(base + o1);
    s->l0 = (uint8_t *)(base + o0);
    s->aux = (float2 *)(base + oaux);
    s->grid = (uint32_t *)(base + og);
    s->part = (float *)(base + op);
  }
  return o;
}

// Dot of N weight dwords (4 int8 each, elements e..e+4N) with the limbs at
// limb byte offset `off`; returns sum(q X) as float (exact integer parts,
// one rounding when the three limb sums are combined).
template <int N>
__device__ __forceinline__ float limbdot(const uint32_t *w, const Smem &S, int off) {
  int a2 = 0, a1 = 0, a0 = 0;
#pragma unroll
  for (int i = 0; i < N / 4; i++) {
    const uint4 v2 = *(const uint4 *)(S.l2 + off + 16 * i);
    const uint4 v1 = *(const uint4 *)(S.l1 + off + 16 * i);
    const uint4 v0 = *(const uint4 *)(S.l0 + off + 16 * i);
    a2 = __builtin_amdgcn_sdot4(w[4 * i + 0], v2.x, a2, false);
    a2 = __builtin_amdgcn_sdot4(w[4 * i + 1], v2.y, a2, false);
    a2 = __builtin_amdgcn_sdot4(w[4 * i + 2], v2.z, a2, false);
    a2 = __builtin_amdgcn_sdot4(w[4 * i + 3], v2.w, a2, false);
    a1 = __builtin_amdgcn_sdot4(w[4 * i + 0], v1.x, a1, false);
    a1 = __builtin_amdgcn_sdot4(w[4 * i + 1], v1.y, a1, false);
    a1 = __builtin_amdgcn_sdot4(w[4 * i + 2], v1.z, a1, false);
    a1 = __builtin_amdgcn_sdot4(w[4 * i + 3], v1.w, a1, false);
    a0 = __builtin_amdgcn_sdot4(w[4 * i + 0], v0.x, a0, false);
    a0 = __builtin_amdgcn_sdot4(w[4 * i + 1], v0.y, a0, false);
    a0 = __builtin_amdgcn_sdot4(w[4 * i + 2], v0.z, a0, false);
    a0 = __builtin_amdgcn_sdot4(w[4 * i + 3], v0.w, a0, false);
  }
  return fmaf((float)a2, 65536.f, fmaf((float)a1, 256.f, (float)a0));
}

// Record of 16-run r (0..15) of unit u.
__device__ __forceinline__ float2 aux_at(const Smem &S, int u, int r) {
  return *(const float2 *)((const char *)S.aux + u * AUX_STRIDE + 8 * r);
}

__device__ __forceinline__ uint32_t dw(const uint4 *ch, int k) {
  const uint4 c = ch[k >> 2];
  const int m = k & 3;
  return m == 0 ? c.x : m == 1 ? c.y : m == 2 ? c.z : c.w;
}

// ---------------------------------------------------------------- Q4_K
// ch[0] = d, dmin, scales[12]; Q4_K: ch[1..8] = qs[128];
// Q5_K: ch[1..2] = qh[32], ch[3..10] = qs[128].
__device__ __forceinline__ float unit_q4k(const uint4 *ch, int u, const Smem &S, int q5) {
  const uint4 hd = ch[0];
  const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
  const int qs0 = q5 ? 3 : 1;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    uint32_t sc0, m0, sc1, m1;
    scale_min_k4(2 * j, hd.y, hd.z, hd.w, sc0, m0);
    scale_min_k4(2 * j + 1, hd.y, hd.z, hd.w, sc1, m1);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t q = dw(ch + qs0, 8 * j + i);
      lo[i] = q & 0x0F0F0F0Fu;
      hi[i] = (q >> 4) & 0x0F0F0F0Fu;
      if (q5) {
        const uint32_t h = dw(ch + 1, i);  // qh bytes 4i..4i+3: element 4i.. of each sub-block
        lo[i] |= ((h >> (2 * j)) & 0x01010101u) << 4;
        hi[i] |= ((h >> (2 * j + 1)) & 0x01010101u) << 4;
      }
    }
    const int off = u * LIMB_STRIDE + 64 * j;
    const float slo = limbdot<8>(lo, S, off);
    const float shi = limbdot<8>(hi, S, off + 32);
    const float2 alo = aux_at(S, u, 4 * j), ahi = aux_at(S, u, 4 * j + 2);
    acc = fmaf(d * (float)sc0 * alo.x, slo, acc);
    acc = fmaf(-(dmin * (float)m0), alo.y, acc);
    acc = fmaf(d * (float)sc1 * ahi.x, shi, acc);
    acc = fmaf(-(dmin * (float)m1), ahi.y, acc);
  }
  return acc;
}

// ---------------------------------------------------------------- Q6_K
// ch[0..7] = ql[128], ch[8..11] = qh[64], ch[12] = scales[16]; d separate.
// 16-run s (elements 16s..16s+15 of the unit) uses scale index s.
__device__ __forceinline__ float unit_q6k(const uint4 *ch, uint32_t dbits, int u, const Smem &S) {
  const float d = h2f(dbits);
  float acc = 0.f;
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
#pragma unroll
    for (int half = 0; half < 2; half++) {
      uint32_t q[4][4];  // [t][i]
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int ii = 4 * half + i;
        const uint32_t A = dw(ch, 16 * hh + ii), B = dw(ch, 16 * hh + 8 + ii);
        const uint32_t H = dw(ch + 8, 8 * hh + ii);
        q[0][i] = (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
        q[1][i] = (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
        q[2][i] = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
        q[3][i] = ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int s = 8 * hh + 2 * t + half;  // 16-run within the unit = scale index
        const float sc = (float)(int8_t)(dw(ch + 12, s >> 2) >> (8 * (s & 3)));
        const float sqx = limbdot<4>(q[t], S, u * LIMB_STRIDE + 16 * s);
        const float2 ax = aux_at(S, u, s);
        const float corr = sqx - 32.f * (float)__float_as_int(ax.y);
        acc = fmaf(sc * ax.x, corr, acc);
      }
    }
  }
  return d * acc;
}

// ---------------------------------------------------------------- Q8_0
// ch[0..15] = qs of 8 blocks, ch[16] = their 8 f16 scales.
__device__ __forceinline__ float unit_q80(const uint4 *ch, int u, const Smem &S) {
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; k++) w[k] = dw(ch, 8 * i + k);
    const float s = limbdot<8>(w, S, u * LIMB_STRIDE + 32 * i);
    const float d = h2f(dw(ch + 16, i >> 1) >> (16 * (i & 1)));
    acc = fmaf(d * aux_at(S, u, 2 * i).x, s, acc);
  }
  return acc;
}

// ------------------------------------------------------------- IQ3_XXS
// ch[0..3] = 64 grid indices, ch[4..5] = 8 sign/scale words; d separate.
// A sign is applied by two's-complement negation of the magnitude byte:
// (g ^ 0xff) + 1 per byte, which cannot carry because magnitudes are in
// 1..127 (enforced when a codebook is installed).
__device__ __forceinline__ uint32_t neg_bytes(uint32_t g, uint32_t nib) {
  const uint32_t m = ((nib * 0x00204081u) & 0x01010101u) * 0xFFu;  // 0xff per negative byte
  return (g ^ m) + (m & 0x01010101u);
}

__device__ __forceinline__ float unit_iq3(const uint4 *ch, uint32_t dbits, int u, const Smem &S) {
  const float d = h2f(dbits);
  float acc = 0.f;
#pragma unroll
  for (int ib = 0; ib < 8; ib++) {
    const uint32_t aux = dw(ch + 4, ib);
    const uint32_t i0 = dw(ch, 2 * ib), i1 = dw(ch, 2 * ib + 1);
    uint32_t q[8];
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t sg = ksign7((aux >> (7 * l)) & 127u);
      const uint32_t word = l < 2 ? i0 : i1;
      const uint32_t g1 = S.grid[(word >> (16 * (l & 1))) & 0xff];
      const uint32_t g2 = S.grid[(word >> (16 * (l & 1) + 8)) & 0xff];
      q[2 * l] = neg_bytes(g1, sg & 15u);
      q[2 * l + 1] = neg_bytes(g2, sg >> 4);
    }
    const float s = limbdot<8>(q, S, u * LIMB_STRIDE + 32 * ib);
    const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    acc = fmaf(db * aux_at(S, u, 2 * ib).x, s, acc);
  }
  return acc;
}

// ------------------------------------------------------------- staging
// A thread converts elements [e0, e0 + 16) of x; 32-runs are the thread
// pairs (2m, 2m+1), whose e0 differ by 16.  All threads execute the
// shuffles.
template <bool Q6>
__device__ __forceinline__ void stage_x(int kpad, int e0, const float (&xv)[16], const Smem &S) {
  float amax = 0.f, sum = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    amax = fmaxf(amax, fabsf(xv[i]));
    sum += xv[i];
  }
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  const float sum32 = sum + __shfl_xor(sum, 1, 64);
  if (e0 >= kpad) return;
  const float inv = amax > 0.f ? LIMB_RANGE / amax : 0.f;
  // Signed base-256 digits of X (each in [-128, 127], unique): since
  // |X| <= 127 * 2^16, X + 0x808080 lies in [0, 2^24) and its bytes are
  // digit + 128, so the bytes of (X + 0x808080) ^ 0x808080 are the digits.
  uint32_t w2[4], w1[4], w0[4];
  int xs = 0;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    uint32_t V[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int X = (int)rintf(xv[4 * q + r] * inv);
      xs += X;
      V[r] = ((uint32_t)X + 0x808080u) ^ 0x808080u;
    }
    // Byte gathers (v_perm_b32: selector byte i picks byte s of {b, a}):
    // lo = {V0.b0, V1.b0, V0.b1, V1.b1}, hi = {V0.b2, V1.b2, 0, 0} per pair,
    // then limb byte k of the four values from the two pairs.
    const uint32_t l01 = __builtin_amdgcn_perm(V[1], V[0], 0x05010400u);
    const uint32_t l23 = __builtin_amdgcn_perm(V[3], V[2], 0x05010400u);
    const uint32_t h01 = __builtin_amdgcn_perm(V[1], V[0], 0x0c0c0602u);
    const uint32_t h23 = __builtin_amdgcn_perm(V[3], V[2], 0x0c0c0602u);
    w0[q] = __builtin_amdgcn_perm(l23, l01, 0x05040100u);
    w1[q] = __builtin_amdgcn_perm(l23, l01, 0x07060302u);
    w2[q] = __builtin_amdgcn_perm(h23, h01, 0x05040100u);
  }
  const int lo = (e0 >> 8) * LIMB_STRIDE + (e0 & 255);
  *(uint4 *)(S.l2 + lo) = make_uint4(w2[0], w2[1], w2[2], w2[3]);
  *(uint4 *)(S.l1 + lo) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
  *(uint4 *)(S.l0 + lo) = make_uint4(w0[0], w0[1], w0[2], w0[3]);
  put_aux<Q6>(S, e0, amax / LIMB_RANGE, sum32, xs);
}

template <bool Q6>
__device__ __forceinline__ void put_aux(const Smem &S, int e0, float sx, float sum32, int xs) {
  const int u = e0 >> 8, r = (e0 & 255) >> 4;
  *(float2 *)((char *)S.aux + u * AUX_STRIDE + 8 * r) =
      make_float2(sx, Q6 ? __int_as_float(xs) : sum32);
}

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

// ------------------------------------------------------------- kernel
template <int FMT> struct Fmt;
// C: 16-byte chunks per unit.
template <> struct Fmt<T_Q4_K> { static constexpr int C = 9; static constexpr bool HAS_D = false; };
template <> struct Fmt<T_Q5_K> { static constexpr int C = 11; static constexpr bool HAS_D = false; };
template <> struct Fmt<T_Q6_K> { static constexpr int C = 13; static constexpr bool HAS_D = true; };
template <> struct Fmt<T_Q8_0> { static constexpr int C = 17; static constexpr bool HAS_D = false; };
template <> struct Fmt<T_IQ3_XXS> { static constexpr int C = 6; static constexpr bool HAS_D = true; };

template <int FMT>
struct Unit {
  uint4 ch[Fmt<FMT>::C];
  uint32_t d;
};

template <int FMT>
__device__ __forceinline__ void load_unit(Unit<FMT> &U, const uint8_t *p, long cstride,
                                          const uint16_t *dp) {
#pragma unroll
  for (int c = 0; c < Fmt<FMT>::C; c++) U.ch[c] = ldw4(p + c * cstride);
  if (Fmt<FMT>::HAS_D) U.d = ldh(dp);
}

template <int FMT>
__device__ __forceinline__ float unit_dot(const Unit<FMT> &U, int u, const Smem &S) {
  if constexpr (FMT == T_Q4_K) return unit_q4k(U.ch, u, S, 0);
  else if constexpr (FMT == T_Q5_K) return unit_q4k(U.ch, u, S, 1);
  else if constexpr (FMT == T_Q6_K) return unit_q6k(U.ch, U.d, u, S);
  else if constexpr (FMT == T_Q8_0) return unit_q80(U.ch, u, S);
  else return unit_iq3(U.ch, U.d, u, S);
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
template <bool K4>
struct XNorm {
  const float *x, *r, *nw;
  float *xo;
  int k;
  float eps;
  float ss = 0.f;
  struct Raw { float x[16], r[16], w[16]; };
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
      ss += v[i] * v[i];
      xv[i] = q.w[i] * v[i];
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
    const int nw = blockDim.x >> 6;
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return 1.0f / sqrtf(t / (float)k + eps);
  }
};

// Stage x for a block of NTH threads: the raw loads of the first NP passes
// of 16 * NTH inputs are issued together, then pre() (which issues the
// first weight loads, so they are in flight while x is converted), then the
// conversion; later passes follow one by one.  Ends with a block barrier.
// (Issuing more weight loads before the staging keeps more registers live
// through it and costs more in occupancy than it gains.)
template <int FMT, int NP, int NTH, class XS, class PRE>
__device__ __forceinline__ void stage_block(XS &xsrc, int kpad, const Smem &S,
                                            const uint32_t *gsrc, PRE &&pre) {
  const int tid = threadIdx.x;
  const int passes = (kpad + 16 * NTH - 1) / (16 * NTH);
  auto pass_e0 = [&](int p) { return 16 * NTH * p + 16 * tid; };
  typename XS::Raw raw[NP];
#pragma unroll
  for (int p = 0; p < NP; p++)
    if (p < passes) xsrc.issue(pass_e0(p), raw[p]);
  uint32_t gword = 0;
  if constexpr (FMT == T_IQ3_XXS) gword = gsrc[tid & 255];
  __builtin_amdgcn_sched_barrier(0);
  pre();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < NP; p++) {
    if (p < passes) {
      float xv[16];
      const int e0 = pass_e0(p);
      xsrc.make(raw[p], e0, xv);
      stage_x<FMT == T_Q6_K>(kpad, e0, xv, S);
    }
  }
  for (int p = NP; p < passes; p++) {
    typename XS::Raw r1;
    const int e0 = pass_e0(p);
    xsrc.issue(e0, r1);
    float xv[16];
    xsrc.make(r1, e0, xv);
    stage_x<FMT == T_Q6_K>(kpad, e0, xv, S);
  }
  if constexpr (FMT == T_IQ3_XXS)
    if (tid < 256) S.grid[tid] = gword;
  xsrc.pre_barrier(S.red);
  __syncthreads();
}

// One wave's work in the MoE kernels: tile t of a stacked expert matrix.
struct WaveJob {
  const uint8_t *body;
  const uint16_t *d;
  float *y;
  int rows, rt, t;
  bool valid;
};

// The MoE body: a 256-thread block stages x, each wave streams its tile
// with two units per lane in flight and reduces its rows.
template <int FMT, class XS>
__device__ __forceinline__ void matvec_wave(const WaveJob &job, int U, int part_floats,
                                            const uint32_t *gsrc, XS &xsrc, char *smem_raw) {
  Smem S;
  smem_layout(U, 4 * part_floats, &S, smem_raw);
  constexpr int C = Fmt<FMT>::C;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t = job.t;
  const int rows_here = min(job.rt, job.rows - t * job.rt);
  const int uit = rows_here * U;
  const int iters = (uit + 63) >> 6;
  const int nv_last = uit - 64 * (iters - 1);
  const long tile_base = (long)t * job.rt * U * C * 16;
  const long dbase = (long)t * job.rt * U;
  auto load_it = [&](Unit<FMT> &dst, int it) {
    const bool last = it == iters - 1;
    const int l = last ? min(lane, nv_last - 1) : lane;
    load_unit<FMT>(dst, job.body + tile_base + (long)it * C * 1024 + 16 * l,
                   last ? 16L * nv_last : 1024L, job.d + dbase + 64 * it + l);
  };
  Unit<FMT> A, B;
  stage_block<FMT, 1, 256>(xsrc, U * 256, S, gsrc, [&] { load_it(A, 0); });
  const float rscale = xsrc.scale(S.red);
  float *part = S.part + wave * part_floats;
  auto consume = [&](const Unit<FMT> &src, int it) {
    const int j = 64 * it + lane;
    const float v = unit_dot<FMT>(src, j % U, S);
    if (j < uit) part[j] = v;
  };
  for (int it = 0; it < iters; it += 2) {
    const bool hb = it + 1 < iters;
    if (hb) load_it(B, it + 1);
    consume(A, it);
    if (it + 2 < iters) load_it(A, it + 2);
    if (hb) consume(B, it + 1);
  }
  // Row sums: 64/RT lanes per row, fixed order.
  const int lpr = 64 / job.rt;
  const int row = lane / lpr, sub = lane % lpr;
  float acc = 0.f;
  if (row < rows_here)
    for (int c = sub; c < U; c += lpr) acc += part[row * U + c];
  for (int off = lpr >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (job.valid && sub == 0 && row < rows_here) job.y[t * job.rt + row] = acc * rscale;
}

// Decode matvec over one or more matrices (segments) sharing the input.
// Weights are one tile per matrix, i.e. the units of the whole matrix in
// row-major order, 64 per iteration.  Block b of a segment owns rows
// [r0, r1) = [rows * lb / nblk, rows * (lb + 1) / nblk), i.e. units
// [r0 * U, r1 * U): the blocks get equal work (+-1 row) and the grid is one
// block per CU, so every block stages x exactly once and all of them run
// at the same time.  The block's iterations (first and last ones partial:
// lanes outside its units load nothing) are dealt round-robin to its
// waves, each keeping two units per lane in flight; per-unit partial sums
// go to LDS and are reduced per row in a fixed order.  With NT = 2
// (gate/up pair) the block streams the same units of seg[1] as well and
// writes silu(g) * u.
template <int FMT, bool K4, int SRC, int NP, int NT>
__global__ __launch_bounds__(mv_threads(FMT)) void k_matvec(MvArgs a) {
  extern __shared__ __align__(16) char smem_raw[];
  constexpr int NTH = mv_threads(FMT), NW = NTH / 64;
  constexpr int C = Fmt<FMT>::C;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar addressing
  const int b = blockIdx.x;
  MvSeg sg = a.seg[0];
  if constexpr (NT == 1) {
#pragma unroll
    for (int i = 1; i < MV_MAX_SEG; i++)
      if (i < a.nseg && b >= a.seg[i].blk_begin) sg = a.seg[i];
  }
  const int U = a.units;
  const int lb = b - sg.blk_begin;
  const int r0 = (int)((long)sg.rows * lb / sg.nblk);
  const int r1 = (int)((long)sg.rows * (lb + 1) / sg.nblk);
  const int j0 = r0 * U, j1 = r1 * U;
  const int n_units = sg.rows * U;
  const int iters = (n_units + 63) >> 6;
  const int nv_last = n_units - 64 * (iters - 1);
  const int it0 = j0 >> 6;
  const int nit = j1 > j0 ? ((j1 + 63) >> 6) - it0 : 0;
  const int work = NT * nit;
  Smem S;
  smem_layout(U, a.part_floats, &S, smem_raw);

  // Work item w: iteration it0 + w % nit of matrix w / nit.
  auto load_w = [&](Unit<FMT> &dst, int w) {
    const bool m = NT == 2 && w >= nit;
    const int it = it0 + (m ? w - nit : w);
    const int j = 64 * it + lane;
    const bool last = it == iters - 1;
    const int l = last ? min(lane, nv_last - 1) : lane;
    const uint8_t *p = (m ? a.seg[1].body : sg.body) + (long)it * C * 1024 + 16 * l;
    const uint16_t *dp = (m ? a.seg[1].d : sg.d) + 64L * it + l;
    if (j >= j0 && j < j1) load_unit<FMT>(dst, p, last ? 16L * nv_last : 1024L, dp);
  };
  auto consume = [&](const Unit<FMT> &src, int w) {
    const int it = it0 + (NT == 2 && w >= nit ? w - nit : w);
    const int j = 64 * it + lane;
    const float v = unit_dot<FMT>(src, j % U, S);
    // (The branch also keeps the scheduler from interleaving two units'
    // arithmetic, which needs more registers than 2 waves per SIMD have.)
    if (j >= j0 && j < j1) S.part[64 * w + lane] = v;
  };

  Unit<FMT> A, B;
  auto first = [&] {
    if (wave < work) load_w(A, wave);
  };
  float rscale = 1.f;
  if constexpr (SRC == MV_NORM) {
    const float *x = a.in.tok ? a.in.x + (long)(*a.in.tok) * a.k : a.in.x;
    XNorm<K4> xs{x, a.in.r, a.in.nw, b == 0 ? a.in.xo : nullptr, a.k, a.in.eps};
    stage_block<FMT, NP, NTH>(xs, U * 256, S, a.grid, first);
    rscale = xs.scale(S.red);
  } else if constexpr (SRC == MV_SWIGLU) {
    XSwiGLU<K4> xs{a.in.xg, a.in.xu, a.k};
    stage_block<FMT, NP, NTH>(xs, U * 256, S, a.grid, first);
  } else {
    XPlain<K4> xs{a.in.x, a.k};
    stage_block<FMT, NP, NTH>(xs, U * 256, S, a.grid, first);
  }
  // Two units per lane in flight; two inlined copies of the unit arithmetic
  // (kernel code size is launch latency: every launch of a decode step
  // starts with a cold instruction cache).
  for (int w = wave; w < work; w += 2 * NW) {
    const int wb = w + NW;
    if (wb < work) load_w(B, wb);
    consume(A, w);
    if (w + 2 * NW < work) load_w(A, w + 2 * NW);
    if (wb < work) consume(B, wb);
  }
  __syncthreads();

  // Row sums: G lanes per row (a power of two, at most 8, U and the threads
  // per row), strided partial sums then a butterfly; a fixed order.  Few
  // lanes per row: the butterfly steps are dependent LDS round trips.
  const int rows_b = r1 - r0;
  int G = 1;
  while (2 * G <= 8 && 2 * G <= U && 2 * G * rows_b <= NTH) G <<= 1;
  const int per = NTH / G;
  const int base = j0 - 64 * it0;
  for (int rb = 0; rb < rows_b; rb += per) {
    const int r = rb + tid / G, sub = tid % G;
    float v[NT];
#pragma unroll
    for (int m = 0; m < NT; m++) {
      const float *pm = S.part + m * 64 * nit + base + r * U;
      float acc = 0.f;
      if (r < rows_b)
        for (int c = sub; c < U; c += G) acc += pm[c];
      for (int off = G >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
      v[m] = acc * rscale;
    }
    if (sub == 0 && r < rows_b) {
      float out = v[0];
      if constexpr (NT == 2) out = v[0] / (1.0f + expf(-v[0])) * v[1];
      sg.y[r0 + r] = out;
    }
  }
}

// ------------------------------------------------------------------- MoE
// Pair p = (token p / top_k, slot p % top_k) routed to expert ids[p].
// Stage 1: gate_e . x_t and up_e . x_t for every pair (blockIdx.y = p,
// waves over the 2 * F / rt tiles of the two expert matrices).
template <int FMT, bool K4>
__global__ __launch_bounds__(256) void k_moe_gate_up(MoeArgs a) {
  extern __shared__ __align__(16) char smem_raw[];
  const int p = blockIdx.y;
  const int e = a.ids[p];
  const int tok = p / a.top_k;
  const int tiles = a.f / a.rt_h;  // tiles per expert matrix
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool valid = gw < 2 * tiles;
  const int gwc = valid ? gw : 2 * tiles - 1;
  const bool is_up = gwc >= tiles;
  const int lt = is_up ? gwc - tiles : gwc;
  const WaveJob job{is_up ? a.up : a.gate, is_up ? a.up_d : a.gate_d,
                    (is_up ? a.tmp_u : a.tmp_g) + (long)p * a.f - (long)e * a.f,
                    a.n_experts * a.f, a.rt_h, e * tiles + lt, valid};
  XPlain<K4> xs{a.x + (long)tok * a.h, a.h};
  matvec_wave<FMT>(job, a.units_h, a.part_h, a.grid, xs, smem_raw);
}

// Stage 2: down_e . (silu(g) * u) for every pair.
template <int FMT, bool K4>
__global__ __launch_bounds__(256) void k_moe_down(MoeArgs a) {
  extern __shared__ __align__(16) char smem_raw[];
  const int p = blockIdx.y;
  const int e = a.ids[p];
  const int tiles = a.h / a.rt_f;
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool valid = gw < tiles;
  const int gwc = valid ? gw : tiles - 1;
  const WaveJob job{a.down, a.down_d, a.tmp_y + (long)p * a.h - (long)e * a.h,
                    a.n_experts * a.h, a.rt_f, e * tiles + gwc, valid};
  XSwiGLU<K4> xs{a.tmp_g + (long)p * a.f, a.tmp_u + (long)p * a.f, a.f};
  matvec_wave<FMT>(job, a.units_f, a.part_f, a.grid, xs, smem_raw);
}

// Router: per token, top-k of the logits (ties: lower index) and their
// softmax probabilities over all experts.  One 256-thread block per token;
// the logits are staged in LDS and every expert's rank (the number of
// experts that beat it) is counted in parallel: rank < k gives its slot.
__global__ __launch_bounds__(256) void k_moe_route(const float *logits, int n_experts, int top_k,
                                                   int *ids, float *w) {
  __shared__ float lv[4096];
  __shared__ float red[256];
  const int t = blockIdx.x, tid = threadIdx.x;
  const float *l = logits + (long)t * n_experts;
  float mx = -INFINITY;
  for (int e = tid; e < n_experts; e += 256) {
    lv[e] = l[e];
    mx = fmaxf(mx, lv[e]);
  }
  red[tid] = mx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  mx = red[0];
  __syncthreads();
  float sum = 0.f;
  for (int e = tid; e < n_experts; e += 256) sum += expf(lv[e] - mx);
  red[tid] = sum;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) red[tid] += red[tid + s];
    __syncthreads();
  }
  sum = red[0];
  for (int e = tid; e < n_experts; e += 256) {
    const float me = lv[e];
    int rank = 0;
    for (int o = 0; o < n_experts; o++) {
      const float ov = lv[o];
      rank += (ov > me) || (ov == me && o < e);
    }
    if (rank < top_k) {
      ids[t * top_k + rank] = e;
      w[t * top_k + rank] = expf(me - mx) / sum;
    }
  }
}

// out[t][i] = sum_s w[t][s] * y[t*k+s][i], slots in order.
__global__ void k_moe_combine(const float *tmp_y, const float *w, int T, int top_k, int h,
                              float *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)T * h) return;
  const int t = (int)(i / h), c = (int)(i % h);
  float acc = 0.f;
  for (int s = 0; s < top_k; s++) acc += w[t * top_k + s] * tmp_y[((long)t * top_k + s) * h + c];
  out[i] = acc;
}

// ------------------------------------------------------------- launch
size_t matvec_lds_bytes(int dtype, int units, int part_total) {
  (void)dtype;
  return smem_layout(units, part_total, nullptr, nullptr);
}

size_t matvec_plan(MvArgs &a, int num_cus) {
  static const int bpc = [] {
    const char *e = getenv("GQ_MV_BLOCKS_PER_CU");  // tuning override
    return e && atoi(e) > 0 ? atoi(e) : MV_BLOCKS_PER_CU;
  }();
  const int nt = a.pair ? 2 : 1, nseg = a.pair ? 1 : a.nseg;
  long total = 0;
  for (int i = 0; i < nseg; i++) total += a.seg[i].rows;
  long target = std::max(1, num_cus * bpc);
  for (;;) {
    int blk = 0;
    long max_units = 0;
    for (int i = 0; i < nseg; i++) {
      const int rows = a.seg[i].rows;
      const int nb = (int)std::max(1L, std::min((long)rows, std::lround((double)target * rows / total)));
      a.seg[i].blk_begin = blk;
      a.seg[i].nblk = nb;
      blk += nb;
      max_units = std::max(max_units, (long)((rows + nb - 1) / nb) * a.units);
    }
    // A block's units may start mid-iteration: one more iteration.
    const int part = (int)(nt * 64 * ((max_units + 63) / 64 + 1));
    const size_t lds = matvec_lds_bytes(0, a.units, part);
    if (lds <= 160 * 1024 || target >= total) {
      a.blocks = blk;
      a.part_floats = part;
      return lds;
    }
    target *= 2;
  }
}

template <int FMT, bool K4, int SRC, int NP, int NT>
static hipError_t launch_t(const MvArgs &a, hipStream_t st) {
  const size_t lds = matvec_lds_bytes(FMT, a.units, a.part_floats);
  if (lds > 64 * 1024)
    (void)hipFuncSetAttribute((const void *)k_matvec<FMT, K4, SRC, NP, NT>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL((k_matvec<FMT, K4, SRC, NP, NT>), dim3(a.blocks), dim3(mv_threads(FMT)), lds, st, a);
  return hipGetLastError();
}

// Instances: plain x with 1, 4 or (512-thread blocks) 8 staging passes in
// flight together;
// the normalised source (k % 4 == 0, one pass in flight) alone or for a
// gate/up pair; the SwiGLU source with one pass in flight.
template <int FMT>
static hipError_t launch_f(const MvArgs &a, hipStream_t st) {
  const int passes = (a.units * 256 + 16 * mv_threads(FMT) - 1) / (16 * mv_threads(FMT));
  const bool k4 = a.k % 4 == 0;
  switch (a.in.src) {
  case MV_NORM:
    if (!k4) return hipErrorInvalidValue;
    return a.pair ? launch_t<FMT, true, MV_NORM, 1, 2>(a, st) : launch_t<FMT, true, MV_NORM, 1, 1>(a, st);
  case MV_SWIGLU:
    if (a.pair) return hipErrorInvalidValue;
    return k4 ? launch_t<FMT, true, MV_SWIGLU, 1, 1>(a, st) : launch_t<FMT, false, MV_SWIGLU, 1, 1>(a, st);
  default:
    if (a.pair) return hipErrorInvalidValue;
    if (passes == 1)
      return k4 ? launch_t<FMT, true, MV_X, 1, 1>(a, st) : launch_t<FMT, false, MV_X, 1, 1>(a, st);
    // (Any NP is correct: passes past NP are staged one by one.  768-thread
    // blocks stage at most 4 passes within the LDS limit.)
    if (passes <= 4 || mv_threads(FMT) > 512)
      return k4 ? launch_t<FMT, true, MV_X, 4, 1>(a, st) : launch_t<FMT, false, MV_X, 4, 1>(a, st);
    if constexpr (mv_threads(FMT) <= 512)
      return k4 ? launch_t<FMT, true, MV_X, 8, 1>(a, st) : launch_t<FMT, false, MV_X, 8, 1>(a, st);
    return hipErrorInvalidValue;
  }
}

hipError_t launch_moe(const MoeArgs &a, int T, hipStream_t st) {
  if (a.fmt != T_IQ3_XXS && a.fmt != T_Q4_K && a.fmt != T_Q6_K && a.fmt != T_Q8_0 &&
      a.fmt != T_Q5_K)
    return hipErrorInvalidValue;
  const int pairs = T * a.top_k;
  hipLaunchKernelGGL(k_moe_route, dim3(T), dim3(256), 0, st, a.logits, a.n_experts, a.top_k,
                     a.ids, a.w);
  const size_t lds1 = matvec_lds_bytes(a.fmt, a.units_h, 4 * a.part_h);
  const size_t lds2 = matvec_lds_bytes(a.fmt, a.units_f, 4 * a.part_f);
  const dim3 g1((2 * (a.f / a.rt_h) + 3) / 4, pairs), g2(((a.h / a.rt_f) + 3) / 4, pairs);
#define GQ_MOE_LAUNCH(F)                                                                     \
  if (a.fmt == F) {                                                                          \
    if (a.h % 4 == 0)                                                                        \
      hipLaunchKernelGGL((k_moe_gate_up<F, true>), g1, dim3(256), lds1, st, a);              \
    else                                                                                     \
      hipLaunchKernelGGL((k_moe_gate_up<F, false>), g1, dim3(256), lds1, st, a);             \
    if (a.f % 4 == 0)                                                                        \
      hipLaunchKernelGGL((k_moe_down<F, true>), g2, dim3(256), lds2, st, a);                 \
    else                                                                                     \
      hipLaunchKernelGGL((k_moe_down<F, false>), g2, dim3(256), lds2, st, a);                \
  }
  GQ_MOE_LAUNCH(T_IQ3_XXS)
  GQ_MOE_LAUNCH(T_Q4_K)
  GQ_MOE_LAUNCH(T_Q5_K)
  GQ_MOE_LAUNCH(T_Q6_K)
  GQ_MOE_LAUNCH(T_Q8_0)
#undef GQ_MOE_LAUNCH
  const long tot = (long)T * a.h;
  hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st,
                     a.tmp_y, a.w, T, a.top_k, a.h, a.out);
  return hipGetLastError();
}

hipError_t launch_matvec(const MvArgs &a, int fmt, hipStream_t st) {
  switch (fmt) {
  case T_Q4_K: return launch_f<T_Q4_K>(a, st);
  case T_Q5_K: return launch_f<T_Q5_K>(a, st);
  case T_Q6_K: return launch_f<T_Q6_K>(a, st);
  case T_Q8_0: return launch_f<T_Q8_0>(a, st);
  case T_IQ3_XXS: return launch_f<T_IQ3_XXS>(a, st);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace gq
