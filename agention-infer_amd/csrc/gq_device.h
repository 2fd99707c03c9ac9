// gq_device.h -- device-side formats and helpers shared by the gq kernels.
//
// Device-resident weight layouts (chosen at upload; total bytes equal the
// ggml tensor size, so HBM traffic per matvec is the algorithmic byte count):
//
//   Q4_K    ggml rows unchanged: 144 B blocks are 16 B aligned
//           (d, dmin, scales[12] = one 16 B header, then qs[128]).
//   Q5_K    ggml rows unchanged: 176 B blocks, 16 B aligned
//           (16 B header, qh[32], qs[128]).
//   Q6_K    body[row][blk] = ql[128] qh[64] scales[16] (208 B, 16 B aligned),
//           d[row][blk] f16 in a separate array (ggml puts d last, making the
//           210 B block unaligned for 128-bit loads).
//   Q8_0    body[row][blk] = qs[32] int8, d[row][blk] f16 separate
//           (the 34 B ggml block is unaligned).
//   IQ3_XXS body[row][blk] = qs[64] aux[32] (96 B), d[row][blk] f16 separate.
//
// Arithmetic: the library is compiled with -ffp-contract=off, so an
// expression such as d1 * q - m1 rounds exactly like the reference's Rust
// (which never contracts).  Kernels that want a fused multiply-add say so
// with fmaf().
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace gq {

enum : int { T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ3_XXS = 18 };
// Kernel-side id (not a ggml type) of Q5_K weights dotted against an input
// quantized to Q8_K, the route WeightMap::matmul_into takes for Q5_K
// (src/model/mod.rs:381-394).
enum : int { T_Q5_K8 = 113 };

// Device body bytes per block for each layout.
__host__ __device__ constexpr int body_block_bytes(int t) {
  return t == T_Q4_K ? 144 : t == T_Q5_K ? 176 : t == T_Q6_K ? 208 : t == T_Q8_0 ? 32
       : t == T_IQ3_XXS ? 96 : 0;
}
__host__ __device__ constexpr int ggml_block_bytes(int t) {
  return t == T_Q4_K ? 144 : t == T_Q5_K ? 176 : t == T_Q6_K ? 210 : t == T_Q8_0 ? 34
       : t == T_IQ3_XXS ? 98 : 0;
}
__host__ __device__ constexpr int block_elems(int t) { return t == T_Q8_0 ? 32 : 256; }
__host__ __device__ constexpr bool has_d_array(int t) {
  return t == T_Q6_K || t == T_Q8_0 || t == T_IQ3_XXS;
}

// Streaming (nontemporal) loads for weight bytes: each byte is read once
// per launch, so they should not displace x or other cached data.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ldw4(const void *p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldw2(const void *p) {
  const u32x2_t v = __builtin_nontemporal_load((const u32x2_t *)p);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ldw1(const void *p) {
  return __builtin_nontemporal_load((const uint32_t *)p);
}
__device__ __forceinline__ uint32_t ldh(const uint16_t *p) {
  return __builtin_nontemporal_load(p);
}

// Dword k of an array of 16-byte chunks (k a compile-time constant after
// unrolling, so this is a register pick).
__device__ __forceinline__ uint32_t dw(const uint4 *ch, int k) {
  const uint4 c = ch[k >> 2];
  const int m = k & 3;
  return m == 0 ? c.x : m == 1 ? c.y : m == 2 ? c.z : c.w;
}

// IEEE binary16 -> binary32 (exact; v_cvt_f32_f16 keeps f16 subnormals).
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

// Byte k (0..11) of the 12 packed scale bytes held in three dwords.
__device__ __forceinline__ uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int k) {
  uint32_t w = k < 4 ? s0 : (k < 8 ? s1 : s2);
  return (w >> ((k & 3) * 8)) & 0xffu;
}

// get_scale_min_k4 (src/quant/q4_k.rs:26-35) on the scale dwords.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t &sc, uint32_t &m) {
  if (j < 4) {
    sc = sbyte(s0, s1, s2, j) & 63u;
    m = sbyte(s0, s1, s2, j + 4) & 63u;
  } else {
    sc = (sbyte(s0, s1, s2, j + 4) & 0xFu) | ((sbyte(s0, s1, s2, j - 4) >> 6) << 4);
    m = (sbyte(s0, s1, s2, j + 4) >> 4) | ((sbyte(s0, s1, s2, j) >> 6) << 4);
  }
}

// IQ3_XXS: a sign is applied by two's-complement negation of a magnitude
// byte, (g ^ 0xff) + 1 per byte (bit b of the nibble: byte b negative),
// which cannot carry because magnitudes are in 1..127 (enforced when a
// codebook is installed).
__device__ __forceinline__ uint32_t neg_bytes(uint32_t g, uint32_t nib) {
  const uint32_t m = ((nib * 0x00204081u) & 0x01010101u) * 0xFFu;  // 0xff per negative byte
  return (g ^ m) + (m & 0x01010101u);
}

// ksigns_iq2xs[i]: 7 sign bits plus an even-parity 8th bit.
__device__ __forceinline__ uint32_t ksign7(uint32_t i) {
  return i | ((uint32_t)(__popc(i) & 1) << 7);
}

// IQ3_XXS in the quad layout is re-encoded at upload (same 96 bytes per
// unit): sub-block ib is 12 bytes, a 96-bit little-endian value holding
// four 23-bit groups (group l at bit 23 l) and the 4-bit scale at bit 92.
// Group l of ggml's sub-block (codebook entries e1 = qs[8 ib + 2 l],
// e2 = qs[8 ib + 2 l + 1], 7 sign bits s7 = (aux >> 7 l) & 127) is
//   e1 | lo3 << 8 | x << 11 | hi3 << 12 | e2 << 15,
// lo3 = s7 & 7, hi3 = s7 >> 4, x = parity(s7 & 15).  Bits 0..11 and 11..22
// are then whole indices of two signed-codebook tables:
//   T1[e1 | lo3 << 8 | x << 11] = e1's entry with signs lo3 | (x ^ parity(lo3)) << 3
//   T2[x | hi3 << 1 | e2 << 4]  = e2's entry with signs hi3 | (x ^ parity(hi3)) << 3
// (the 8th sign bit of ksign7 is parity(s7) = x ^ parity(hi3)), so a
// lookup is one shift and one mask.
__host__ __device__ inline uint32_t iq3q_group(uint32_t e1, uint32_t e2, uint32_t s7) {
  const uint32_t lo4 = s7 & 15u;
  const uint32_t x = (lo4 ^ (lo4 >> 1) ^ (lo4 >> 2) ^ (lo4 >> 3)) & 1u;
  return e1 | (s7 & 7u) << 8 | x << 11 | (s7 >> 4) << 12 | e2 << 15;
}
// The 12 bytes of sub-block ib of a ggml IQ3_XXS block (qs = block + 2).
__host__ __device__ inline void iq3q_pack(const uint8_t *qs, int ib, uint32_t w[3]) {
  const uint8_t *a = qs + 64 + 4 * ib;
  const uint32_t aux = a[0] | a[1] << 8 | a[2] << 16 | (uint32_t)a[3] << 24;
  uint32_t g[4];
  for (int l = 0; l < 4; l++)
    g[l] = iq3q_group(qs[8 * ib + 2 * l], qs[8 * ib + 2 * l + 1], (aux >> (7 * l)) & 127u);
  w[0] = g[0] | g[1] << 23;
  w[1] = g[1] >> 9 | g[2] << 14;
  w[2] = g[2] >> 18 | g[3] << 5 | (aux >> 28) << 28;
}
// Back from a group: e1, e2 and ggml's 8 sign bits (ksign7 of s7).
__host__ __device__ inline void iq3q_unpack(uint32_t g, uint32_t &e1, uint32_t &e2, uint32_t &sg) {
  e1 = g & 255u;
  e2 = (g >> 15) & 255u;
  const uint32_t lo3 = (g >> 8) & 7u, x = (g >> 11) & 1u, hi3 = (g >> 12) & 7u;
  const uint32_t b3 = x ^ ((lo3 ^ (lo3 >> 1) ^ (lo3 >> 2)) & 1u);
  const uint32_t ph = (hi3 ^ (hi3 >> 1) ^ (hi3 >> 2)) & 1u;
  sg = lo3 | b3 << 3 | hi3 << 4 | (x ^ ph) << 7;
}

// quantize_row_q8_k (src/quant/q8_k.rs:49-91) of one 256-element block held
// by 16 aligned lanes, 16 consecutive elements each (idx0 = index of this
// lane's first element in the block).  The block's pivot is the first
// element of largest magnitude (the reference's sequential `av > amax`
// scan: lexicographic (magnitude, lowest index) across lanes), iscale =
// -127 / pivot, q = min(round(iscale * x), 127) (round half away from zero),
// d = 1 / iscale; an all-zero block has d = 0 and q = 0.  Returns the
// lane's 16 codes as 4 dwords, their sum (the lane's bsums entry) and d.
struct Q8K16 {
  uint32_t q[4];
  int bsum;
  float d;
};
__device__ __forceinline__ Q8K16 q8k_quant16(const float (&xv)[16], int idx0) {
  float amax = 0.f, mx = 0.f;
  int ia = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const float av = fabsf(xv[i]);
    if (av > amax) {
      amax = av;
      mx = xv[i];
      ia = idx0 + i;
    }
  }
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) {
    const float oa = __shfl_xor(amax, off, 64), om = __shfl_xor(mx, off, 64);
    const int oi = __shfl_xor(ia, off, 64);
    if (oa > amax || (oa == amax && oi < ia)) {
      amax = oa;
      mx = om;
      ia = oi;
    }
  }
  Q8K16 r;
  r.bsum = 0;
  r.d = 0.f;
#pragma unroll
  for (int k = 0; k < 4; k++) r.q[k] = 0;
  if (amax > 0.f) {
    const float iscale = -127.0f / mx;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int v = min((int)roundf(iscale * xv[i]), 127);
      r.bsum += v;
      r.q[i >> 2] |= ((uint32_t)v & 0xffu) << (8 * (i & 3));
    }
    r.d = 1.0f / iscale;
  }
  return r;
}

// Unsigned byte k of w as float (lowers to v_cvt_f32_ubyte{k}).
template <int K>
__device__ __forceinline__ float ub(uint32_t w) { return (float)((w >> (8 * K)) & 0xffu); }

// sum_k ub(w, k) * x[k] over the 4 bytes of w, accumulated into acc.
__device__ __forceinline__ float dot4u(uint32_t w, float4 x, float acc) {
  acc = fmaf(ub<0>(w), x.x, acc);
  acc = fmaf(ub<1>(w), x.y, acc);
  acc = fmaf(ub<2>(w), x.z, acc);
  acc = fmaf(ub<3>(w), x.w, acc);
  return acc;
}


// Wave-wide max / sum of a float, returned to every lane.  DPP steps
// combine within 16-lane rows (quad swaps, then rotations by 4 and 8), the
// four row totals are read as scalars; a fixed order, no LDS round trips.
template <class OP>
__device__ __forceinline__ float wave_reduce(float x, OP op) {
  auto dpp = [](float v, int ctrl) -> float {
    switch (ctrl) {  // the control must be a constant expression
    case 0: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    case 1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
    }
  };
  x = op(x, dpp(x, 0));  // quad_perm [1,0,3,2]
  x = op(x, dpp(x, 1));  // quad_perm [2,3,0,1]
  x = op(x, dpp(x, 2));  // row_ror 4
  x = op(x, dpp(x, 3));  // row_ror 8
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return op(op(r0, r1), op(r2, r3));
}
__device__ __forceinline__ float wave_max(float x) {
  return wave_reduce(x, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float wave_sum(float x) {
  return wave_reduce(x, [](float a, float b) { return a + b; });
}

}  // namespace gq
