// gq_matvec.hip -- the v_dot4 MoE expert FFN over stacked expert tensors in
// the wave-tiled layout (rows per expert not a multiple of 16; the others
// take the quad layout and the MFMA stages of gq_mvq.hip), the router
// kernel for more than MOE_ROUTE_MAX experts, and the MoE dispatch
// (gfx950, wave64).
//
// Replaces the reference's per-row dot kernels (src/quant/q8_0.rs:58-90,
// q4_k.rs:95-212, q5_k.rs:189-317, q6_k.rs:82-131) for the expert
// matrices; the MoE layer itself has no counterpart in the reference
// (docs/08-moe-routing.md describes it).
//
// Design (HBM-bound; every weight byte is read exactly once):
//  * Weights sit in the wave-tiled layout (gq_layout.h), one tile per
//    expert: one lane owns one 256-element unit, and a wave-wide 128-bit
//    load reads 1 KiB of contiguous HBM with a nontemporal hint.  Each lane
//    keeps its next unit in flight while it computes the current one.
//  * Blocks own equal row ranges of a (token, slot) pair's expert (gate/up)
//    or of a token's output rows over its experts (down); x is staged once
//    per block.
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
#include "gq_moe.h"
#include "gq_xsrc.h"

namespace gq {

constexpr int LIMB_STRIDE = 272;  // LDS bytes per 256-element block of one limb (16 B pad)

constexpr int AUX_STRIDE = 144;   // LDS bytes per unit of the per-16-run records (16 B pad)

// Per 16-run record: {s of its 32-run, c} with c = sum(x) of the 32-run
// (Q4_K/Q5_K) or sum(X) of the 16-run as int bits (Q6_K).  The 16 B pads
// put the records of consecutive units in different LDS bank groups.
struct Smem {
  uint8_t *l2, *l1, *l0;  // limbs, LIMB_STRIDE bytes per 256 elements
  float2 *aux;            // AUX_STRIDE bytes per unit
  uint32_t *grid;         // IQ3_XXS: [entry][sign nibble] signed codebook words
  float *part;            // per-wave per-unit partial sums
  float *red;             // 16 floats of block reduction scratch
};

__host__ __device__ inline size_t smem_layout(int fmt, int units, int part_total, Smem *s, char *base) {
  size_t o = 0;
  auto take = [&](size_t n) { size_t r = o; o += (n + 15) & ~(size_t)15; return r; };
  const size_t limb = (size_t)units * LIMB_STRIDE;
  const size_t o2 = take(limb), o1 = take(limb), o0 = take(limb);
  // IQ3_XXS: the codebook with the signs applied, 16 sign nibbles per entry
  const size_t oaux = take((size_t)units * AUX_STRIDE), og = take(fmt == T_IQ3_XXS ? 4 * 4096 : 0);
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

// Q5_K against the Q8_K-quantized input (dot_q5_k_q8k, src/quant/q5_k.rs:
// 126-184): the codes sit in limb l0 and each 16-run record holds {d of the
// Q8_K block, the run's bsums entry as int bits}.  The weight codes (5-bit,
// 0..31) meet the int8 codes in v_dot4; acc_pos and acc_min are exact
// integers, and the unit's value is the reference's per-block term
// dx * (d * acc_pos - dmin * acc_min), rounded the same way.
__device__ __forceinline__ float unit_q5k8(const uint4 *ch, int u, const Smem &S) {
  const uint4 hd = ch[0];
  const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
  int acc_pos = 0, acc_min = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    uint32_t sc0, m0, sc1, m1;
    scale_min_k4(2 * j, hd.y, hd.z, hd.w, sc0, m0);
    scale_min_k4(2 * j + 1, hd.y, hd.z, hd.w, sc1, m1);
    int plo = 0, phi = 0;
    const int off = u * LIMB_STRIDE + 64 * j;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t q = dw(ch + 3, 8 * j + i);
      const uint32_t h = dw(ch + 1, i);  // qh bytes 4i..4i+3
      const uint32_t lo = (q & 0x0F0F0F0Fu) | (((h >> (2 * j)) & 0x01010101u) << 4);
      const uint32_t hi = ((q >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * j + 1)) & 0x01010101u) << 4);
      plo = __builtin_amdgcn_sdot4(lo, *(const uint32_t *)(S.l0 + off + 4 * i), plo, false);
      phi = __builtin_amdgcn_sdot4(hi, *(const uint32_t *)(S.l0 + off + 32 + 4 * i), phi, false);
    }
    const int b0 = __float_as_int(aux_at(S, u, 4 * j).y) + __float_as_int(aux_at(S, u, 4 * j + 1).y);
    const int b1 = __float_as_int(aux_at(S, u, 4 * j + 2).y) + __float_as_int(aux_at(S, u, 4 * j + 3).y);
    acc_pos += (int)sc0 * plo + (int)sc1 * phi;
    acc_min += (int)m0 * b0 + (int)m1 * b1;
  }
  const float dx = aux_at(S, u, 0).x;
  return dx * (d * (float)acc_pos - dmin * (float)acc_min);
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
// A sign is applied by two's-complement negation of the magnitude byte
// (neg_bytes, gq_device.h).

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
      const uint32_t e1 = (word >> (16 * (l & 1))) & 0xff, e2 = (word >> (16 * (l & 1) + 8)) & 0xff;
      q[2 * l] = S.grid[(e1 << 4) | (sg & 15u)];
      q[2 * l + 1] = S.grid[(e2 << 4) | (sg >> 4)];
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
__device__ __forceinline__ void put_aux(const Smem &S, int e0, float sx, float sum32, int xs);

// Q8_K route: the 16 threads of each 256-element block quantize it like
// quantize_row_q8_k; the codes go to limb l0, {d, bsum} to the records.
__device__ __forceinline__ void stage_x_q8k(int kpad, int e0, const float (&xv)[16], const Smem &S) {
  const Q8K16 r = q8k_quant16(xv, e0 & 255);
  if (e0 >= kpad) return;
  const int lo = (e0 >> 8) * LIMB_STRIDE + (e0 & 255);
  *(uint4 *)(S.l0 + lo) = make_uint4(r.q[0], r.q[1], r.q[2], r.q[3]);
  const int u = e0 >> 8, rr = (e0 & 255) >> 4;
  *(float2 *)((char *)S.aux + u * AUX_STRIDE + 8 * rr) = make_float2(r.d, __int_as_float(r.bsum));
}

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

// ------------------------------------------------------------- kernel
template <int FMT> struct Fmt;
// C: 16-byte chunks per unit.
template <> struct Fmt<T_Q4_K> { static constexpr int C = 9; static constexpr bool HAS_D = false; };
template <> struct Fmt<T_Q5_K> { static constexpr int C = 11; static constexpr bool HAS_D = false; };
template <> struct Fmt<T_Q5_K8> { static constexpr int C = 11; static constexpr bool HAS_D = false; };
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
  else if constexpr (FMT == T_Q5_K8) return unit_q5k8(U.ch, u, S);
  else if constexpr (FMT == T_Q6_K) return unit_q6k(U.ch, U.d, u, S);
  else if constexpr (FMT == T_Q8_0) return unit_q80(U.ch, u, S);
  else return unit_iq3(U.ch, U.d, u, S);
}


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
  auto stage = [&](int e0, const float (&xv)[16]) {
    if constexpr (FMT == T_Q5_K8) stage_x_q8k(kpad, e0, xv, S);
    else stage_x<FMT == T_Q6_K>(kpad, e0, xv, S);
  };
  typename XS::Raw raw[NP];
#pragma unroll
  for (int p = 0; p < NP; p++)
    if (p < passes) xsrc.issue(pass_e0(p), raw[p]);
  constexpr int GW = FMT == T_IQ3_XXS ? 4096 / NTH : 1;  // signed codebook words per thread
  uint32_t gword[GW];
  if constexpr (FMT == T_IQ3_XXS)
#pragma unroll
    for (int i = 0; i < GW; i++) gword[i] = gsrc[(tid + NTH * i) >> 4];
  __builtin_amdgcn_sched_barrier(0);
  pre();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < NP; p++) {
    if (p < passes) {
      float xv[16];
      const int e0 = pass_e0(p);
      xsrc.make(raw[p], e0, xv);
      stage(e0, xv);
    }
  }
  for (int p = NP; p < passes; p++) {
    typename XS::Raw r1;
    const int e0 = pass_e0(p);
    xsrc.issue(e0, r1);
    float xv[16];
    xsrc.make(r1, e0, xv);
    stage(e0, xv);
  }
  if constexpr (FMT == T_IQ3_XXS)
#pragma unroll
    for (int i = 0; i < GW; i++) {
      const int o = tid + NTH * i;
      S.grid[o] = neg_bytes(gword[i], o & 15);
    }
  if constexpr (!IsExact<XS>::value) xsrc.pre_barrier(S.red);
  __syncthreads();
}

// A matrix streamed by a block: its body and d arrays (one tile: the units
// in row-major order) and the first LDS column of the x it meets.
struct MatRef {
  const uint8_t *body;
  const uint16_t *d;
  int xcol;
};

// The units [j0, j1) (flat row-major index) of nm matrices of n_units
// units each, streamed by the NW waves of a block.  Work item w is
// iteration it0 + w % nit of matrix w / nit (NM: 1, 2 or 0 = any nm); the
// block's first and last iterations are partial, lanes outside [j0, j1)
// load nothing.  Items are dealt round-robin to the waves, each keeping
// two units per lane in flight; per-unit partial sums go to
// S.part[64 * w + lane].
template <int FMT, int NW, int NM, class MATF>
struct BlockStream {
  MATF mat;
  int U, j0, j1, iters, nv_last, it0, nit, work, lane, wave;
  __device__ __forceinline__ BlockStream(MATF m, int U_, int j0_, int j1_, int n_units, int nm,
                                         int lane_, int wave_)
      : mat(m), U(U_), j0(j0_), j1(j1_), lane(lane_), wave(wave_) {
    iters = (n_units + 63) >> 6;
    nv_last = n_units - 64 * (iters - 1);
    it0 = j0 >> 6;
    nit = j1 > j0 ? ((j1 + 63) >> 6) - it0 : 0;
    work = nm * nit;
  }
  __device__ __forceinline__ int mat_of(int w) const {
    return NM == 1 ? 0 : NM == 2 ? (w >= nit ? 1 : 0) : w / nit;
  }
  __device__ __forceinline__ void load(Unit<FMT> &dst, int w) const {
    const int m = mat_of(w), it = it0 + w - m * nit;
    const MatRef r = mat(m);
    const int j = 64 * it + lane;
    const bool last = it == iters - 1;
    const int l = last ? min(lane, nv_last - 1) : lane;
    if (j >= j0 && j < j1)
      load_unit<FMT>(dst, r.body + (long)it * Fmt<FMT>::C * 1024 + 16 * l,
                     last ? 16L * nv_last : 1024L, r.d + 64L * it + l);
  }
  __device__ __forceinline__ void consume(const Unit<FMT> &src, int w, const Smem &S) const {
    const int m = mat_of(w), it = it0 + w - m * nit;
    const int j = 64 * it + lane;
    const float v = unit_dot<FMT>(src, mat(m).xcol + j % U, S);
    // (The branch also keeps the scheduler from interleaving two units'
    // arithmetic, which needs more registers than 2 waves per SIMD have.)
    if (j >= j0 && j < j1) S.part[64 * w + lane] = v;
  }
  __device__ __forceinline__ void first(Unit<FMT> &A) const {
    if (wave < work) load(A, wave);
  }
  // Two inlined copies of the unit arithmetic (kernel code size is launch
  // latency: every launch of a decode step starts with a cold instruction
  // cache).
  __device__ __forceinline__ void run(Unit<FMT> &A, Unit<FMT> &B, const Smem &S) const {
    for (int w = wave; w < work; w += 2 * NW) {
      const int wb = w + NW;
      if (wb < work) load(B, wb);
      consume(A, w, S);
      if (w + 2 * NW < work) load(A, w + 2 * NW);
      if (wb < work) consume(B, wb, S);
    }
  }
  // Partial sums of row r (counted from row j0 / U) of matrix m.
  __device__ __forceinline__ const float *row_part(const Smem &S, int m, int r) const {
    return S.part + m * 64 * nit + (j0 - 64 * it0) + r * U;
  }
};

// Lanes per row of the row sums: a power of two, at most 8, U and the
// block's threads per row (the butterfly steps are dependent LDS round
// trips, so few lanes per row).
__device__ __forceinline__ int row_lanes(int U, int rows, int nth) {
  int G = 1;
  while (2 * G <= 8 && 2 * G <= U && 2 * G * rows <= nth) G <<= 1;
  return G;
}

// Sum of the U partials at p: lane `sub` of G (G in {1, 2, 4, 8}, groups
// aligned in the wave) takes c = sub, sub + G, ..., then DPP row shifts by
// 1, 2, 4 add the group up in its last lane (sub == G - 1, the only lane
// whose result is defined); a fixed order.
__device__ __forceinline__ float row_sum(const float *p, int U, int sub, int G, bool valid) {
  float acc = 0.f;
  if (valid)
    for (int c = sub; c < U; c += G) acc += p[c];
  if (G >= 2)
    acc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x111, 0xF, 0xF, true));
  if (G >= 4)
    acc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x112, 0xF, 0xF, true));
  if (G >= 8)
    acc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x114, 0xF, 0xF, true));
  return acc;
}

// ------------------------------------------------------------------- MoE
// Pair p = (token p / top_k, slot p % top_k) routed to expert ids[p].
// Expert tensors are one tile per expert (rows_per_expert rows, units in
// row-major order), so expert e's matrix starts at tile e.
// Stage 1: h_p = silu(gate_e . x_t) * (up_e . x_t) (the SwiGLU of
// ffn_gate_up, src/model/llama/cpu_path.rs:225-227): the blocks are split
// evenly over the pairs (bpp per pair), block lb of pair p owns rows
// [f * lb / bpp, f * (lb + 1) / bpp) of both matrices of its expert.
// With ROUTE (n_experts <= MOE_ROUTE_MAX) the block also routes: it ranks
// the token's logits (ties: lower index, like k_moe_route) to find its
// slot's expert, and block 0 of the pair stores ids[p] and the softmax
// weight w[p] for stage 2.
template <int FMT, bool K4, bool ROUTE>
__global__ __launch_bounds__(mv_threads(FMT)) void k_moe_gate_up(MoeArgs a) {
  extern __shared__ __align__(16) char smem_raw[];
  constexpr int NTH = mv_threads(FMT), NW = NTH / 64, C = Fmt<FMT>::C;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x, p = b / a.bpp, lb = b - p * a.bpp;
  const int tok = p / a.top_k;
  const int U = a.units_h, f = a.f;
  const int r0 = (int)((long)f * lb / a.bpp), r1 = (int)((long)f * (lb + 1) / a.bpp);
  Smem S;
  smem_layout(FMT, U, a.part_h, &S, smem_raw);
  int e = 0;  // the pair's expert (set before the first weight load)
  auto mat = [&](int m) {
    const long tb = (long)e * f * U;  // first unit of expert e
    return m ? MatRef{a.up + tb * C * 16, a.up_d + tb, 0} : MatRef{a.gate + tb * C * 16, a.gate_d + tb, 0};
  };
  const BlockStream<FMT, NW, 2, decltype(mat)> bs(mat, U, r0 * U, r1 * U, f * U, 2, lane, wave);
  Unit<FMT> A, B;
  XPlain<K4> xs{a.x + (long)tok * a.h, a.h};
  // Routing runs while the x loads are in flight.
  auto route = [&] {
    if constexpr (ROUTE) e = moe_route_pair<NTH>(a, p, lb == 0);
    else e = min(max(a.ids[p], 0), a.n_experts - 1);
  };
  stage_block<FMT, 1, NTH>(xs, U * 256, S, a.grid, [&] {
    route();
    bs.first(A);
  });
  bs.run(A, B, S);
  __syncthreads();
  const int rows_b = r1 - r0;
  const int G = row_lanes(U, rows_b, NTH), per = NTH / G;
  for (int rb = 0; rb < rows_b; rb += per) {
    const int r = rb + tid / G, sub = tid % G;
    const float g = row_sum(bs.row_part(S, 0, r), U, sub, G, r < rows_b);
    const float u = row_sum(bs.row_part(S, 1, r), U, sub, G, r < rows_b);
    if (sub == G - 1 && r < rows_b) a.hbuf[(long)p * f + r0 + r] = g / (1.0f + expf(-g)) * u;
  }
}

// Stage 2 with the weighted combine (moe_ffn): out[t] = sum_s w[t][s] *
// (down_(e_s) . h_(t, s)), slots in order.  Block lb of token t (bpt per
// token) owns rows [h * lb / bpt, h * (lb + 1) / bpt) and streams those
// rows of all top_k routed experts against the token's staged inputs.
template <int FMT, bool K4>
__global__ __launch_bounds__(mv_threads(FMT)) void k_moe_down(MoeArgs a) {
  extern __shared__ __align__(16) char smem_raw[];
  constexpr int NTH = mv_threads(FMT), NW = NTH / 64, C = Fmt<FMT>::C;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x, t = b / a.bpt, lb = b - t * a.bpt;
  const int U = a.units_f, h = a.h, K = a.top_k, p0 = t * K;
  const int r0 = (int)((long)h * lb / a.bpt), r1 = (int)((long)h * (lb + 1) / a.bpt);
  Smem S;
  smem_layout(FMT, K * U, a.part_f, &S, smem_raw);
  auto mat = [&](int m) {
    const long tb = (long)min(max(a.ids[p0 + m], 0), a.n_experts - 1) * h * U;
    return MatRef{a.down + tb * C * 16, a.down_d + tb, m * U};
  };
  const BlockStream<FMT, NW, 0, decltype(mat)> bs(mat, U, r0 * U, r1 * U, h * U, K, lane, wave);
  Unit<FMT> A, B;
  XSlots<K4> xs{a.hbuf, a.f, U * 256, K, p0};
  stage_block<FMT, 4, NTH>(xs, K * U * 256, S, a.grid, [&] { bs.first(A); });
  bs.run(A, B, S);
  __syncthreads();
  const int rows_b = r1 - r0;
  const int G = row_lanes(U, rows_b, NTH), per = NTH / G;
  for (int rb = 0; rb < rows_b; rb += per) {
    const int r = rb + tid / G, sub = tid % G;
    float out = 0.f;
    for (int m = 0; m < K; m++)
      out += a.w[p0 + m] * row_sum(bs.row_part(S, m, r), U, sub, G, r < rows_b);
    if (sub == G - 1 && r < rows_b) a.out[(long)t * h + r0 + r] = out;
  }
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
    // (the count stops once it reaches top_k: such an expert has no slot)
    int rank = 0;
    for (int o0 = 0; o0 < n_experts && rank < top_k; o0 += 16) {
      const int o1 = min(o0 + 16, n_experts);
      for (int o = o0; o < o1; o++) {
        const float ov = lv[o];
        rank += (ov > me) || (ov == me && o < e);
      }
    }
    if (rank < top_k) {
      ids[t * top_k + rank] = e;
      w[t * top_k + rank] = expf(me - mx) / sum;
    }
  }
}

// ------------------------------------------------------------- launch
size_t matvec_lds_bytes(int dtype, int units, int part_total) {
  return smem_layout(dtype, units, part_total, nullptr, nullptr);
}

// Blocks per pair (gate/up) and per token (down): about one block per CU
// in all, more while a block's partial sums would not fit in LDS.  Stages
// over quad-layout experts take the MFMA kernels' plan.
static size_t moe_plan(MoeArgs &a, int T, int cus) {
  const int pairs = T * a.top_k;
  size_t l1, l2;
  if (a.quad_gu) {
    l1 = mvq_moe_plan(a, T, 1, cus);
  } else {
    a.bpp = std::max(1, std::min(a.f, cus / pairs));
    for (;;) {
      const long u1 = (long)((a.f + a.bpp - 1) / a.bpp) * a.units_h;
      a.part_h = (int)(2 * 64 * ((u1 + 63) / 64 + 1));
      a.lds_gu = (int)matvec_lds_bytes(a.fmt, a.units_h, a.part_h);
      l1 = a.lds_gu + MOE_ROUTE_MAX * 16 + 256;  // + routing
      if (l1 <= 160 * 1024 || a.bpp >= a.f) break;
      a.bpp = std::min(a.f, 2 * a.bpp);
    }
  }
  if (a.quad_dn) {
    l2 = mvq_moe_plan(a, T, 2, cus);
  } else {
    a.bpt = std::max(1, std::min(a.h, cus / T));
    for (;;) {
      const long u2 = (long)((a.h + a.bpt - 1) / a.bpt) * a.units_f;
      a.part_f = (int)(a.top_k * 64 * ((u2 + 63) / 64 + 1));
      a.lds_dn = (int)matvec_lds_bytes(a.fmt, a.top_k * a.units_f, a.part_f);
      l2 = a.lds_dn;
      if (l2 <= 160 * 1024 || a.bpt >= a.h) break;
      a.bpt = std::min(a.h, 2 * a.bpt);
    }
  }
  return std::max(l1, l2);
}

size_t moe_lds_bytes(int fmt, int h, int f, int top_k, int T, int cus, bool quad_gu, bool quad_dn) {
  MoeArgs a{};
  a.fmt = fmt;
  a.h = h;
  a.f = f;
  a.top_k = top_k;
  a.units_h = (h + 255) / 256;
  a.units_f = (f + 255) / 256;
  a.quad_gu = quad_gu;
  a.quad_dn = quad_dn;
  return moe_plan(a, T, cus);
}

static void big_lds(const void *fn, int lds) {
  if (lds > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
}

template <int F, bool R>
static void moe_gate_up_f(const MoeArgs &a, int T, hipStream_t st) {
  const dim3 g1(T * a.top_k * a.bpp), nt(mv_threads(F));
  if (a.h % 4 == 0) {
    big_lds((const void *)k_moe_gate_up<F, true, R>, a.lds_gu);
    hipLaunchKernelGGL((k_moe_gate_up<F, true, R>), g1, nt, a.lds_gu, st, a);
  } else {
    big_lds((const void *)k_moe_gate_up<F, false, R>, a.lds_gu);
    hipLaunchKernelGGL((k_moe_gate_up<F, false, R>), g1, nt, a.lds_gu, st, a);
  }
}

template <int F>
static void moe_down_f(const MoeArgs &a, int T, hipStream_t st) {
  const dim3 g2(T * a.bpt), nt(mv_threads(F));
  if (a.f % 4 == 0) {
    big_lds((const void *)k_moe_down<F, true>, a.lds_dn);
    hipLaunchKernelGGL((k_moe_down<F, true>), g2, nt, a.lds_dn, st, a);
  } else {
    big_lds((const void *)k_moe_down<F, false>, a.lds_dn);
    hipLaunchKernelGGL((k_moe_down<F, false>), g2, nt, a.lds_dn, st, a);
  }
}

hipError_t launch_moe(const MoeArgs &args, int T, hipStream_t st) {
  MoeArgs a = args;
  if (moe_plan(a, T, a.cus) > 160 * 1024) return hipErrorInvalidValue;
  // Few experts: the gate/up blocks route (one launch less); many: the
  // router kernel first.
  const bool fused = a.n_experts <= MOE_ROUTE_MAX;
  if (!fused)
    hipLaunchKernelGGL(k_moe_route, dim3(T), dim3(256), 0, st, a.logits, a.n_experts, a.top_k,
                       a.ids, a.w);
  hipError_t e = hipSuccess;
  if (a.quad_gu) {
    e = launch_mvq_moe(a, T, 1, fused, st);
  } else {
#define GQ_MOE_GU(C, F)                                     \
  case C:                                                   \
    if (fused) moe_gate_up_f<F, true>(a, T, st);            \
    else moe_gate_up_f<F, false>(a, T, st);                 \
    break;
    switch (a.fmt) {
      GQ_MOE_GU(T_IQ3_XXS, T_IQ3_XXS)
      GQ_MOE_GU(T_Q4_K, T_Q4_K)
      GQ_MOE_GU(T_Q5_K, T_Q5_K8)  // matmul_into's Q8_K route
      GQ_MOE_GU(T_Q6_K, T_Q6_K)
      GQ_MOE_GU(T_Q8_0, T_Q8_0)
    default: return hipErrorInvalidValue;
    }
#undef GQ_MOE_GU
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  if (a.quad_dn) return launch_mvq_moe(a, T, 2, false, st);
  switch (a.fmt) {
  case T_IQ3_XXS: moe_down_f<T_IQ3_XXS>(a, T, st); break;
  case T_Q4_K: moe_down_f<T_Q4_K>(a, T, st); break;
  case T_Q5_K: moe_down_f<T_Q5_K8>(a, T, st); break;
  case T_Q6_K: moe_down_f<T_Q6_K>(a, T, st); break;
  case T_Q8_0: moe_down_f<T_Q8_0>(a, T, st); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace gq
