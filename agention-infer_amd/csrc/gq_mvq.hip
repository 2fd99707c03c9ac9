// gq_mvq.hip -- batch-1 decode matvec y = W . x on int8 MFMA for dense
// Q4_K, Q5_K, Q6_K, Q8_0 and IQ3_XXS weights, and the two stages of the MoE
// expert FFN over stacked experts in the same layout (gfx950, wave64).
//
// Replaces the reference's per-row dot kernels (src/quant/q8_0.rs:58-90,
// q4_k.rs:95-212, q5_k.rs:126-184 and 189-317, q6_k.rs:82-131) driven
// row-parallel by WeightMap::matmul_into (src/model/mod.rs:362-403).
//
// Weights are in the quad layout (gq_layout.h): a wave-wide load of one
// chunk of an item (16 rows x 4 units) is 1 KiB of contiguous HBM, and lane
// l = 16q + r holds the whole unit (row r, unit q) -- every weight byte is
// read once, by one lane.
//
// x is staged once per block in LDS as three int8 limbs per element: per
// 256-element unit, s = max|x| / (127 * 2^16) and X = rint(x / s) =
// x2 * 2^16 + x1 * 2^8 + x0 (signed bytes), so |x - s * X| <= s / 2 (6e-8
// of the unit's max).
//
// The products run on v_mfma_i32_16x16x64_i8, D = A * B:
//   * B = 16 weight codes of each lane's unit (col r = row r of the group,
//     k-group q = unit q);
//   * A = block-diagonal x: row 4q + i holds limb i of unit q's 16 inputs in
//     k-group q and zero elsewhere (lanes 20q + i read 16 limb bytes from
//     LDS, all other lanes read a zero region).
// Lane 16q + r then holds D[4q + i][r] = sum(codes of (r, q) * limb i of
// unit q): every sum of a lane is its own unit's, so the sub-block scales
// apply in the lane, in exact integer arithmetic where the format allows:
//   Q4_K/Q5_K  acc_i = sum_sb sc_sb * D_sb,i  (i32)
//              y += d * s * (acc_2 2^16 + acc_1 2^8 + acc_0) - dmin * sum_sb m_sb * sum(x_sb)
//   Q6_K       acc_i = sum_run sc_run * D_run,i (codes q in 0..63), and
//              -32 * sum_run sc_run * sum(X_run) for the code offset
//   Q8_0       y += s * sum_b d_b * (D_b,2 2^16 + D_b,1 2^8 + D_b,0)
//   Q5_K x Q8_K (matmul_into's route): A holds the Q8_K codes (one limb)
//              and the block term dx * (d * acc_pos - dmin * acc_min) is
//              the reference's, exactly.
//   IQ3_XXS    B = signed codebook bytes from two LDS tables (the format is
//              re-encoded at upload so that each lookup index is a bit
//              field), acc_i = sum_sb (2 s_sb + 1) * D_sb,i,
//              y += d / 4 * s * (acc_2 2^16 + acc_1 2^8 + acc_0)
// The four lanes of a row add their units (lane swaps), waves write per-row
// partial sums to LDS, and the block adds them per row in a fixed order
// (deterministic results).
//
// Work split: block b owns the row groups b, b + B, b + 2B, ... of the
// launch (all segments' groups in a row); the waves take its items (group,
// matrix, quad) in turn from an LDS counter.  Each lane keeps its next item
// in flight while it computes the current one.  A one-matrix launch may
// split K (MvIn::y2): two sets of blocks, each over all row groups, take the
// first and the second half of every row's quads and stage only that half
// of x; the second half's sums go to y2 for the caller to add.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "gq_device.h"
#include "gq_internal.h"
#include "gq_moe.h"
#include "gq_xsrc.h"

namespace gq {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int QL_STRIDE = 272;  // LDS bytes per unit of one limb (16 B pad: bank spread)
constexpr int QZERO = 256;      // bytes of zeros the A operand's idle lanes read
constexpr int IQ3_TABLE_WORDS = 8192;  // IQ3_XXS: T1 and T2, 4096 words each
constexpr uint32_t IQ3_T2 = 16384;     // byte offset of T2 from T1

// The IQ3_XXS tables live in static LDS: its address is a constant after
// LDS lowering, so a lookup's base folds into the instruction's offset.
__device__ __forceinline__ uint32_t *iq3_tables() {
  __shared__ __align__(16) uint32_t t[IQ3_TABLE_WORDS];
  return t;
}

// Waves per block, and items per lane in registers at once (the current
// one and DEPTH - 1 in flight): 8 waves (two per SIMD; IQ3_XXS, whose item
// math is LDS- and VALU-bound and needs fewer registers, 16), each lane keeping
// one item in flight while it computes another.  (Three items per lane held
// 60 more registers and streamed slower: the Q6_K head 72.5 against 70.0
// us, the Q4_K gate/up pair 16.2 against 15.4; 12 waves of the two-item
// Q4_K kernel were slower still.)
__host__ __device__ constexpr int mvq_waves(int fmt) { return fmt == T_IQ3_XXS ? 16 : 8; }
__host__ __device__ constexpr int mvq_depth(int) { return 2; }

template <int FMT> struct QF;
template <> struct QF<T_Q4_K> { static constexpr int C = 9, AUX = 8; };
template <> struct QF<T_Q5_K> { static constexpr int C = 11, AUX = 8; };
template <> struct QF<T_Q5_K8> { static constexpr int C = 11, AUX = 16; };
template <> struct QF<T_Q6_K> { static constexpr int C = 13, AUX = 16; };
template <> struct QF<T_Q8_0> { static constexpr int C = 17, AUX = 0; };
template <> struct QF<T_IQ3_XXS> { static constexpr int C = 6, AUX = 0; };

// LDS: limbs [3][units][QL_STRIDE] (Q5_K8: the Q8_K codes in limb 0),
// zeros [QZERO], per-unit scale s [units] (Q5_K8: the Q8_K d), per-unit aux
// [units][AUX] (Q4_K/Q5_K: fp32 sums of the 8 sub-blocks; Q6_K: int sums of
// the 16 runs of X; Q5_K8: bsums as int), per-item row sums [items][16],
// 16 floats of reduction scratch and the item counter.  (IQ3_XXS's
// codebook tables are static LDS, iq3_tables.)
struct QSmem {
  uint8_t *limb;
  uint32_t zero_off;
  float *us;
  int *aux;
  float *part;
  float *red;
  int *ctr;
};

__host__ __device__ inline size_t qsmem_layout(int aux_per_unit, int units, int part_floats,
                                               QSmem *s, char *base) {
  size_t o = 0;
  auto take = [&](size_t n) { size_t r = o; o += (n + 15) & ~(size_t)15; return r; };
  const int upad = (units + 3) & ~3;  // the last quad's missing units stay in bounds
  const size_t ol = take((size_t)3 * upad * QL_STRIDE);
  const size_t oz = take(QZERO);
  const size_t ou = take((size_t)upad * 4);
  const size_t oa = take((size_t)upad * aux_per_unit * 4);
  const size_t op = take((size_t)part_floats * 4);
  const size_t orr = take(64);
  const size_t oc = take(16);
  if (s) {
    s->limb = (uint8_t *)(base + ol);
    s->zero_off = (uint32_t)oz;
    s->us = (float *)(base + ou);
    s->aux = (int *)(base + oa);
    s->part = (float *)(base + op);
    s->red = (float *)(base + orr);
    s->ctr = (int *)(base + oc);
  }
  return o;
}

__device__ __forceinline__ i32x4 lds16(const char *smem, uint32_t off) {
  return *(const i32x4 *)(smem + off);
}

__device__ __forceinline__ i32x4 mfma(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i32x4 v4(uint4 q) { return i32x4{(int)q.x, (int)q.y, (int)q.z, (int)q.w}; }

__device__ __forceinline__ float combine(int a2, int a1, int a0) {
  return fmaf((float)a2, 65536.f, fmaf((float)a1, 256.f, (float)a0));
}

// -------------------------------------------------------------- staging
// Thread t converts elements [16t, 16t + 16) of a pass; the 16 threads of a
// unit are aligned lanes of one wave (xor shuffles 1..8).
template <int FMT>
__device__ __forceinline__ void stage16(int kpad, int e0, const float (&xv)[16], const QSmem &S,
                                        int upad) {
  const int u = e0 >> 8, w16 = (e0 & 255) >> 4;
  if constexpr (FMT == T_Q5_K8) {
    const Q8K16 r = q8k_quant16(xv, e0 & 255);
    if (e0 >= kpad) return;
    *(uint4 *)(S.limb + u * QL_STRIDE + (e0 & 255)) = make_uint4(r.q[0], r.q[1], r.q[2], r.q[3]);
    S.aux[u * 16 + w16] = r.bsum;
    if (w16 == 0) S.us[u] = r.d;
  } else {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(xv[i]));
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    float sum = 0.f;
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
#pragma unroll
      for (int i = 0; i < 16; i++) sum += xv[i];
    }
    const float sum32 = sum + __shfl_xor(sum, 1, 64);
    if (e0 >= kpad) return;
    const float inv = amax > 0.f ? LIMB_RANGE / amax : 0.f;
    uint32_t w2[4], w1[4], w0[4];
    int xs = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint32_t V[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int X = (int)rintf(xv[4 * q + r] * inv);
        xs += X;
        V[r] = ((uint32_t)X + 0x808080u) ^ 0x808080u;  // signed base-256 digits
      }
      const uint32_t l01 = __builtin_amdgcn_perm(V[1], V[0], 0x05010400u);
      const uint32_t l23 = __builtin_amdgcn_perm(V[3], V[2], 0x05010400u);
      const uint32_t h01 = __builtin_amdgcn_perm(V[1], V[0], 0x0c0c0602u);
      const uint32_t h23 = __builtin_amdgcn_perm(V[3], V[2], 0x0c0c0602u);
      w0[q] = __builtin_amdgcn_perm(l23, l01, 0x05040100u);
      w1[q] = __builtin_amdgcn_perm(l23, l01, 0x07060302u);
      w2[q] = __builtin_amdgcn_perm(h23, h01, 0x05040100u);
    }
    const int lo = u * QL_STRIDE + (e0 & 255);
    const int lstride = upad * QL_STRIDE;
    *(uint4 *)(S.limb + lo) = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    *(uint4 *)(S.limb + lstride + lo) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
    *(uint4 *)(S.limb + 2 * lstride + lo) = make_uint4(w0[0], w0[1], w0[2], w0[3]);
    if (w16 == 0) S.us[u] = amax / LIMB_RANGE;
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
      if (!(w16 & 1)) ((float *)S.aux)[u * 8 + (w16 >> 1)] = sum32;
    } else if constexpr (FMT == T_Q6_K) {
      S.aux[u * 16 + w16] = xs;
    }
  }
}

// ------------------------------------------------------------ item math
// One unit per lane.  ch: the unit's chunks, a: this lane's A-operand LDS
// byte offset for the unit's quad (idle lanes: the zero region), u: the
// lane's unit (column index in x units), S: staged x.
template <int FMT>
__device__ __forceinline__ float item_dot(const uint4 *ch, uint32_t dbits, const char *smem,
                                          uint32_t a, int u, const QSmem &S) {
  if constexpr (FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q5_K8) {
    constexpr bool Q5 = FMT != T_Q4_K;
    constexpr int QS = Q5 ? 3 : 1;  // first qs chunk
    const uint4 hd = ch[0];
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    int acc2 = 0, acc1 = 0, acc0 = 0, amin = 0;
    float mt = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t sc0, m0, sc1, m1;
      scale_min_k4(2 * j, hd.y, hd.z, hd.w, sc0, m0);
      scale_min_k4(2 * j + 1, hd.y, hd.z, hd.w, sc1, m1);
      i32x4 dlo = {0, 0, 0, 0}, dhi = {0, 0, 0, 0};
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const uint4 q = ch[QS + 2 * j + h];
        uint4 lo = make_uint4(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu);
        uint4 hi = make_uint4((q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu,
                              (q.z >> 4) & 0x0F0F0F0Fu, (q.w >> 4) & 0x0F0F0F0Fu);
        if constexpr (Q5) {  // qh bytes 16h..16h+15: bit 2j -> low, 2j+1 -> high
          const uint4 qh = ch[1 + h];
          lo.x |= ((qh.x >> (2 * j)) & 0x01010101u) << 4;
          lo.y |= ((qh.y >> (2 * j)) & 0x01010101u) << 4;
          lo.z |= ((qh.z >> (2 * j)) & 0x01010101u) << 4;
          lo.w |= ((qh.w >> (2 * j)) & 0x01010101u) << 4;
          hi.x |= ((qh.x >> (2 * j + 1)) & 0x01010101u) << 4;
          hi.y |= ((qh.y >> (2 * j + 1)) & 0x01010101u) << 4;
          hi.z |= ((qh.z >> (2 * j + 1)) & 0x01010101u) << 4;
          hi.w |= ((qh.w >> (2 * j + 1)) & 0x01010101u) << 4;
        }
        dlo = mfma(lds16(smem, a + 64 * j + 16 * h), v4(lo), dlo);
        dhi = mfma(lds16(smem, a + 64 * j + 32 + 16 * h), v4(hi), dhi);
      }
      if constexpr (FMT == T_Q5_K8) {
        acc0 += __mul24((int)sc0, dlo[0]) + __mul24((int)sc1, dhi[0]);
        const int4 bs = *(const int4 *)(S.aux + u * 16 + 4 * j);
        amin += __mul24((int)m0, bs.x + bs.y) + __mul24((int)m1, bs.z + bs.w);
      } else {
        acc2 += __mul24((int)sc0, dlo[0]) + __mul24((int)sc1, dhi[0]);
        acc1 += __mul24((int)sc0, dlo[1]) + __mul24((int)sc1, dhi[1]);
        acc0 += __mul24((int)sc0, dlo[2]) + __mul24((int)sc1, dhi[2]);
        const float2 sx = *(const float2 *)((const float *)S.aux + u * 8 + 2 * j);
        mt = fmaf((float)m0, sx.x, mt);
        mt = fmaf((float)m1, sx.y, mt);
      }
    }
    if constexpr (FMT == T_Q5_K8) return S.us[u] * (d * (float)acc0 - dmin * (float)amin);
    return d * S.us[u] * combine(acc2, acc1, acc0) - dmin * mt;
  } else if constexpr (FMT == T_Q6_K) {
    // ch[0..7] ql, ch[8..11] qh, ch[12] scales; run s = elements 16s.. uses scale s
    int acc2 = 0, acc1 = 0, acc0 = 0;
    float corr = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
#pragma unroll
      for (int half = 0; half < 2; half++) {
        uint32_t q[4][4];
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
          const int s = 8 * hh + 2 * t + half;
          const int sc = (int)(int8_t)(dw(ch + 12, s >> 2) >> (8 * (s & 3)));
          const i32x4 z = {0, 0, 0, 0};
          const i32x4 dd = mfma(lds16(smem, a + 16 * s),
                                i32x4{(int)q[t][0], (int)q[t][1], (int)q[t][2], (int)q[t][3]}, z);
          acc2 += __mul24(sc, dd[0]);
          acc1 += __mul24(sc, dd[1]);
          acc0 += __mul24(sc, dd[2]);
          corr = fmaf((float)sc, (float)S.aux[u * 16 + s], corr);
        }
      }
    }
    return h2f(dbits) * S.us[u] * (combine(acc2, acc1, acc0) - 32.f * corr);
  } else if constexpr (FMT == T_IQ3_XXS) {
    // ch: 8 sub-blocks of 12 bytes in the re-encoded format (iq3q_pack):
    // each 12-bit field of a group is an index into T1 (LDS byte 0) or T2
    // (LDS byte IQ3_T2) whose words are the signed codebook bytes, i.e. the
    // MFMA codes.  w = d (0.5 + s) 0.5 * grid * sign = d/4 * (2s + 1) *
    // (signed grid): (2s + 1) applies per sub-block in integers.
    const char *tb = (const char *)iq3_tables();
    auto tw = [&](uint32_t off) { return *(const uint32_t *)(tb + off); };
    int acc2 = 0, acc1 = 0, acc0 = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ib++) {
      const uint32_t w0 = dw(ch, 3 * ib), w1 = dw(ch, 3 * ib + 1), w2 = dw(ch, 3 * ib + 2);
      // byte offsets 4 * field: the field's bits shifted to bit 2, masked
      const uint32_t q0 = tw((w0 << 2) & 0x3FFCu);
      const uint32_t q1 = tw(IQ3_T2 + ((w0 >> 9) & 0x3FFCu));
      const uint32_t q2 = tw(__builtin_amdgcn_alignbit(w1, w0, 21) & 0x3FFCu);
      const uint32_t q3 = tw(IQ3_T2 + (w1 & 0x3FFCu));
      const uint32_t q4 = tw((w1 >> 12) & 0x3FFCu);
      const uint32_t q5 = tw(IQ3_T2 + (__builtin_amdgcn_alignbit(w2, w1, 23) & 0x3FFCu));
      const uint32_t q6 = tw((w2 >> 3) & 0x3FFCu);
      const uint32_t q7 = tw(IQ3_T2 + ((w2 >> 14) & 0x3FFCu));
      i32x4 dd = mfma(lds16(smem, a + 32 * ib), i32x4{(int)q0, (int)q1, (int)q2, (int)q3},
                      i32x4{0, 0, 0, 0});
      dd = mfma(lds16(smem, a + 32 * ib + 16), i32x4{(int)q4, (int)q5, (int)q6, (int)q7}, dd);
      const int s2 = (int)(2 * (w2 >> 28) + 1);
      acc2 += __mul24(s2, dd[0]);
      acc1 += __mul24(s2, dd[1]);
      acc0 += __mul24(s2, dd[2]);
    }
    return 0.25f * h2f(dbits) * S.us[u] * combine(acc2, acc1, acc0);
  } else {  // Q8_0: ch[0..15] qs of 8 blocks, ch[16] their f16 d
    float acc = 0.f;
#pragma unroll
    for (int b = 0; b < 8; b++) {
      const i32x4 z = {0, 0, 0, 0};
      i32x4 dd = mfma(lds16(smem, a + 32 * b), v4(ch[2 * b]), z);
      dd = mfma(lds16(smem, a + 32 * b + 16), v4(ch[2 * b + 1]), dd);
      const float db = h2f(dw(ch + 16, b >> 1) >> (16 * (b & 1)));
      acc = fmaf(db, combine(dd[0], dd[1], dd[2]), acc);
    }
    return S.us[u] * acc;
  }
}

template <int FMT>
struct QItem {
  uint4 ch[QF<FMT>::C];
  uint32_t d;
};


// What a launch of the body computes: a dense matvec (MvArgs), or one of
// the two MoE stages (MoeArgs) over stacked experts in the quad layout
// (rows per expert a multiple of 16, so expert e's matrix is a quad matrix
// starting at unit e rows U).
enum { MQ_DENSE = 0, MQ_GATE_UP = 1, MQ_DOWN = 2 };

template <int FMT, bool K4, int SRC, int NT, int MODE, bool ROUTE, bool ONE>
__device__ __forceinline__ void mvq_body(const MvArgs &a, const MoeArgs &mo) {
  extern __shared__ __align__(16) char smem[];
  constexpr int NW = mvq_waves(FMT), NTH = 64 * NW, C = QF<FMT>::C;
  constexpr bool HAS_D = FMT == T_Q6_K || FMT == T_IQ3_XXS;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // This block's row groups: flat groups b, b + B, b + 2B, ... (local
  // group lg is flat group b + lg B: at any time the blocks stream
  // neighbouring groups, spreading the traffic evenly over the memory
  // channels), and their items (group, matrix, quad), numbered
  // it = (lg NM + m) T + t.  The waves take items in turn: wave w starts
  // with items w and w + NW, and each further item comes from an LDS
  // counter, so the waves finish within about one item of each other.
  // Each item's 16 row sums go to their own LDS slot and a row adds its
  // items in item order, so results do not depend on which wave took what.
  //   dense:   the launch's flat groups over all blocks; NM = NT matrices.
  //   gate/up: pair p = (token, slot) takes blocks [p bpp, (p + 1) bpp) and
  //            the f / 16 groups of its expert's gate and up (NM = 2).
  //   down:    token p takes blocks [p bpt, (p + 1) bpt) and the h / 16
  //            groups of its top_k experts' down matrices (NM = top_k,
  //            matrix m = slot m, against slot m's input).
  //   split (a.ksplit > 0, dense one-matrix launches): blocks [0, blocks0)
  //            take quads [0, ksplit) of their groups, the others quads
  //            [ksplit, T), each over all groups; a block stages only its
  //            half's inputs.
  int G, B, b, p = 0, Uw;
  bool h1 = false;  // split: this block runs half 1
  if constexpr (MODE == MQ_DENSE) {
    G = a.groups;
    B = a.blocks;
    b = blockIdx.x;
    Uw = a.units;
    if (a.ksplit > 0) {
      h1 = (int)blockIdx.x >= a.blocks0;
      B = h1 ? a.blocks - a.blocks0 : a.blocks0;
      b = h1 ? (int)blockIdx.x - a.blocks0 : (int)blockIdx.x;
    }
  } else if constexpr (MODE == MQ_GATE_UP) {
    B = mo.bpp;
    p = blockIdx.x / B;
    b = blockIdx.x - p * B;
    G = mo.f / QROWS;
    Uw = mo.units_h;
  } else {
    B = mo.bpt;
    p = blockIdx.x / B;
    b = blockIdx.x - p * B;
    G = mo.h / QROWS;
    Uw = mo.units_f;
  }
  const int NM = MODE == MQ_DOWN ? mo.top_k : NT;  // matrices per group
  const int U = Uw, T = (U + 3) >> 2;              // weight units per row, quads
  // This block's quads of a row: [tq0, tq0 + Tl) (T without a split).
  const int tq0 = h1 ? a.ksplit : 0;
  const int Tl = MODE == MQ_DENSE && a.ksplit > 0 ? (h1 ? T - a.ksplit : a.ksplit) : T;
  // Staged x: U units (split: the half's units; down: top_k slot inputs of
  // 4T units each).
  const int Ux = MODE == MQ_DOWN ? NM * 4 * T : min(U, 4 * (tq0 + Tl)) - 4 * tq0;
  const int upad = 4 * ((Ux + 3) >> 2);
  const int ngb = (G - b + B - 1) / B;
  // Row sums go to one LDS slot per (group, matrix, quad): (lg NM + m) T + t.
  // down with 4F + 2 units per row and an even top_k (SP): the 2-unit tail
  // quads of slots 2j and 2j + 1 form one item (lanes q < 2: slot 2j,
  // q >= 2: slot 2j + 1), so no lane idles; per group and slot pair the
  // items are slot 2j's F full quads, slot 2j + 1's, then the tail pair.
  const int F = U >> 2;
  const bool SP = MODE == MQ_DOWN && (U & 3) == 2 && (NM & 1) == 0;
  const int per_sp = (NM / 2) * (2 * F + 1);
  const int nslots = ngb * NM * Tl;
  const int nitems = SP ? ngb * per_sp : nslots;
  const int rows_blk = ngb * QROWS;
  if (nitems == 0) return;  // (plans give every block a group; uniform per block)
  QSmem S;
  qsmem_layout(QF<FMT>::AUX, Ux, nslots * QROWS, &S, smem);

  // Item cursor (wave-uniform): local and flat group, matrix, quad, segment,
  // row-sum slot, and whether it is a down tail pair (slots m and m + 1).
  struct Cur {
    int lg, fg, m, t, seg, slot;
    bool pair;
  };
  auto cur_at = [&](int it) {
    Cur c;
    c.pair = false;
    if (SP) {
      const int gi = it / per_sp, rem = it - gi * per_sp;
      const int jp = rem / (2 * F + 1), k = rem - jp * (2 * F + 1);
      c.lg = gi;
      c.m = 2 * jp + (k >= F && k < 2 * F);
      c.t = k < F ? k : k < 2 * F ? k - F : F;
      c.pair = k == 2 * F;
    } else {
      const int per = NM * Tl, gi = it / per, rem = it - gi * per;
      c.lg = gi;
      c.m = rem / Tl;
      c.t = rem - c.m * Tl;
    }
    c.fg = b + c.lg * B;
    c.slot = (c.lg * NM + c.m) * Tl + c.t;
    c.seg = 0;
    if constexpr (MODE == MQ_DENSE && NT == 1) {
#pragma unroll
      for (int i = 1; i < MV_MAX_SEG; i++)
        if (i < a.nseg && c.fg >= a.seg[i].blk_begin) c.seg = i;
    }
    return c;
  };
  // The matrix of item cursor c: body, d array, rows, and c's group in it.
  int eid = 0;  // gate/up: the pair's expert (set before the first load)
  // down: lane m holds slot m's expert (loaded with the x loads in flight)
  // (clamped: an expert index out of range, whatever a router wrote, stays a
  // read inside the stacked tensor)
  const int eids = MODE == MQ_DOWN && lane < NM ? min(max(mo.ids[p * NM + lane], 0), mo.n_experts - 1) : 0;
  struct Mat {
    const uint8_t *body;
    const uint16_t *d;
    int rows, g;
  };
  auto mat_of = [&](const Cur &c) {
    Mat M;
    if constexpr (MODE == MQ_DENSE) {
      const MvSeg &sg = a.seg[NT == 2 ? c.m : c.seg];
      M = Mat{sg.body, sg.d, sg.rows, c.fg - a.seg[c.seg].blk_begin};
    } else if constexpr (MODE == MQ_GATE_UP) {
      const long e0 = (long)eid * mo.f * U;  // expert's first unit
      M = c.m ? Mat{mo.up + e0 * (C * 16), mo.up_d + e0, mo.f, c.fg}
              : Mat{mo.gate + e0 * (C * 16), mo.gate_d + e0, mo.f, c.fg};
    } else {
      const int e = __builtin_amdgcn_readlane(eids, c.m);
      const long e0 = (long)e * mo.h * U;
      M = Mat{mo.down + e0 * (C * 16), mo.down_d + e0, mo.h, c.fg};
    }
    return M;
  };
  auto grab = [&]() {
    int v = 0;
    if (lane == 0) v = atomicAdd(S.ctr, 1);
    return __builtin_amdgcn_readfirstlane(v);
  };
  const int q = lane >> 4, r = lane & 15;
  // idle: a wave without an item issues the same loads, every one of them
  // reading the item's first 16 bytes (one line), so that the staging's
  // waits do not depend on whether the wave has an item.
  auto load = [&](QItem<FMT> &dst, int it, bool idle = false) {
    const Cur lc = cur_at(it);
    Mat sg = mat_of(lc);
    if constexpr (MODE == MQ_DOWN) {
      if (lc.pair) {  // lanes q >= 2: slot m + 1's expert
        Cur c2 = lc;
        c2.m = lc.m + 1;
        const Mat s2 = mat_of(c2);
        if (q >= 2) sg = s2;
      }
    }
    const int g = sg.g, tg = tq0 + lc.t;  // (the quad in the row)
    const int nr = min(QROWS, sg.rows - QROWS * g), nq = lc.pair ? 2 : min(4, U - 4 * tg);
    const int ql = lc.pair ? (q & 1) : q;
    const long base = (long)g * QROWS * U + (long)tg * 4 * nr;  // quad_item_unit
    const bool live = r < nr && ql < nq && !idle;
    const int l = live ? nr * ql + r : 0;  // idle lanes re-read lane 0 (same lines)
    const uint8_t *bp = sg.body + base * (C * 16);
    const int cs = idle ? 0 : 16 * nr * nq;
#pragma unroll
    for (int c = 0; c < C; c++) dst.ch[c] = ldw4(bp + (uint32_t)(c * cs + 16 * l));
    if constexpr (HAS_D) dst.d = ldh(sg.d + base + l);
  };

  constexpr int DEPTH = mvq_depth(FMT);
  QItem<FMT> R0, R1, R2;
  // The first item's loads go out once the staging's x has arrived (not
  // before: a wave's loads complete in order, so x would wait behind the
  // weights), the second one's after the x conversion (issuing both first
  // holds the conversion back while the memory pipeline takes them).

  // ---- stage x (and set the item counter)
  if (tid == 0) *S.ctr = (DEPTH - 1) * NW;
  int c0 = wave, c1 = wave + NW, c2 = nitems;  // items held by R0, R1, R2
  if (tid < QZERO / 16) *(uint4 *)(smem + S.zero_off + 16 * tid) = make_uint4(0, 0, 0, 0);
  float rscale = 1.f;
  const int kpad = Ux * 256;
  auto stage_all = [&](auto &xsrc) {
    const int passes = (kpad + 16 * NTH - 1) / (16 * NTH);
    using XS = std::remove_reference_t<decltype(xsrc)>;
    if constexpr (IsExact<XS>::value) {
      for (int p = 0; p < passes; p++) {
        typename XS::Raw r0;
        xsrc.issue(16 * NTH * p + 16 * tid, r0);
        xsrc.accum_ss(r0, 16 * NTH * p + 16 * tid);
      }
      xsrc.pre_barrier(S.red);
      __syncthreads();
      xsrc.set_rms(S.red);
      __syncthreads();
    }
    // the x loads of the first NP passes, then the first items' loads, then
    // the conversion (later passes one by one)
    constexpr int NP = sizeof(typename XS::Raw) <= 64 ? 3 : 2;
    // IQ3_XXS: this thread's codebook entries, loaded first (before x and
    // the weights: loads complete in order), signed into T1 and T2 below:
    // entries o = tid + NTH i of each table (T1's all take entry tid % 256).
    constexpr int GW = FMT == T_IQ3_XXS ? 4096 / NTH : 1;
    static_assert(FMT != T_IQ3_XXS || (NTH % 256 == 0 && 4096 % NTH == 0),
                  "table staging assumes 256 | NTH | 4096");
    uint32_t gword[GW], gword1 = 0;
    if constexpr (FMT == T_IQ3_XXS) {
      const uint32_t *gr = MODE == MQ_DENSE ? a.grid : mo.grid;
      gword1 = gr[tid & 255];
#pragma unroll
      for (int i = 0; i < GW; i++) gword[i] = gr[(tid + NTH * i) >> 4];
    }
    // All NPc passes' loads go out (NPc = 1 for one pass, else NP; clamped
    // addresses past the input, masked in make), then the first item's,
    // right behind them: a wave's loads complete in order, so x still
    // arrives first, and the item's HBM latency overlaps x's.  Later passes
    // go one by one.
    auto pipeline = [&](auto npc) {
      constexpr int NPc = decltype(npc)::value;
      typename XS::Raw raw[NPc];
#pragma unroll
      for (int k = 0; k < NPc; k++) xsrc.issue(16 * NTH * k + 16 * tid, raw[k]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (MODE == MQ_GATE_UP) {  // (while the x loads are in flight)
        if constexpr (ROUTE) eid = moe_route_pair<NTH>(mo, p, b == 0);
        else eid = __builtin_amdgcn_readfirstlane(min(max(mo.ids[p], 0), mo.n_experts - 1));
      }
      // (unconditional, so that the waits for x count exactly the loads
      // behind them)
      load(R0, min(c0, nitems - 1), c0 >= nitems);
      __builtin_amdgcn_sched_barrier(0);
      float xv[NPc][16];
#pragma unroll
      for (int k = 0; k < NPc; k++) xsrc.make(raw[k], 16 * NTH * k + 16 * tid, xv[k]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < NPc; k++)
        if (k < passes) stage16<FMT>(kpad, 16 * NTH * k + 16 * tid, xv[k], S, upad);
      __builtin_amdgcn_sched_barrier(0);
      if (DEPTH == 3 && c1 < nitems) load(R1, c1);
      __builtin_amdgcn_sched_barrier(0);
      for (int p = NPc; p < passes; p++) {
        typename XS::Raw r1;
        const int e0 = 16 * NTH * p + 16 * tid;
        xsrc.issue(e0, r1);
        float xv1[16];
        xsrc.make(r1, e0, xv1);
        stage16<FMT>(kpad, e0, xv1, S, upad);
      }
    };
    // ONE: the launch stages x in one pass (k <= 16 NTH)
    if constexpr (ONE) pipeline(std::integral_constant<int, 1>{});
    else pipeline(std::integral_constant<int, NP>{});
    if constexpr (FMT == T_IQ3_XXS) {
      auto par3 = [](uint32_t v) { return (v ^ (v >> 1) ^ (v >> 2)) & 1u; };
#pragma unroll
      for (int i = 0; i < GW; i++) {
        const uint32_t o = tid + NTH * i;
        const uint32_t lo3 = (o >> 8) & 7u, x1 = o >> 11;  // T1[e1 | lo3 << 8 | x << 11]
        iq3_tables()[o] = neg_bytes(gword1, lo3 | (x1 ^ par3(lo3)) << 3);
        const uint32_t hi3 = (o >> 1) & 7u, x2 = o & 1u;   // T2[x | hi3 << 1 | e2 << 4]
        iq3_tables()[4096 + o] = neg_bytes(gword[i], hi3 | (x2 ^ par3(hi3)) << 3);
      }
    }
    if constexpr (!IsExact<XS>::value) xsrc.pre_barrier(S.red);
    __syncthreads();
    rscale = xsrc.scale(S.red);
  };
  if constexpr (MODE == MQ_GATE_UP) {
    XPlain<K4> xs{mo.x + (long)(p / mo.top_k) * mo.h, mo.h};
    stage_all(xs);
  } else if constexpr (MODE == MQ_DOWN) {
    XSlots<K4> xs{mo.hbuf, mo.f, 4 * T * 256, NM, p * NM};
    stage_all(xs);
  } else if constexpr (SRC == MV_NORM) {
    const float *x = a.in.tok ? a.in.x + (long)(*a.in.tok) * a.k : a.in.x;
    XNorm<K4, FMT == T_Q5_K8> xs{x, a.in.r, a.in.nw, blockIdx.x == 0 ? a.in.xo : nullptr, a.k, a.in.eps};
    stage_all(xs);
  } else if constexpr (SRC == MV_SWIGLU) {
    XSwiGLU<K4> xs{a.in.xg, a.in.xu, a.k};
    stage_all(xs);
  } else if (a.ksplit > 0) {  // this half's inputs
    XPlain<K4> xs{a.in.x + 1024 * tq0, min(a.k, 1024 * (tq0 + Tl)) - 1024 * tq0};
    stage_all(xs);
  } else {
    XPlain<K4> xs{a.in.x, a.k};
    stage_all(xs);
  }

  // ---- stream this wave's items
  // A operand: lanes 20q' + i (i < 3) read limb i of unit q' of the quad
  // (Q5_K8: limb 0 only), every other lane the zero region.
  const int aq = lane >> 4, ai = lane & 15;
  const bool alive = (ai >> 2) == aq && (ai & 3) < (FMT == T_Q5_K8 ? 1 : 3);
  const uint32_t limb_off = (uint32_t)((ai & 3) * upad * QL_STRIDE);
  auto consume = [&](const QItem<FMT> &src, int it) {
    const Cur cc = cur_at(it);
    // lane group j (0..3) works on unit 4t + j of slot m, or for a tail pair
    // on unit 4F + (j & 1) of slot m + j / 2
    const int ql = cc.pair ? (q & 1) : q;
    const int u = 4 * (tq0 + cc.t) + ql;  // this lane's unit in its row
    // staged unit of lane group j's input (down: in its slot's input)
    auto xunit = [&](int j) {
      const int m = cc.pair ? cc.m + (j >> 1) : cc.m;
      return (MODE == MQ_DOWN ? m * 4 * T : 0) + 4 * cc.t + (cc.pair ? (j & 1) : j);
    };
    const uint32_t aoff = alive ? limb_off + (uint32_t)xunit(aq) * QL_STRIDE : S.zero_off;
    float v = item_dot<FMT>(src.ch, src.d, smem, aoff, min(xunit(q), upad - 1), S);
    int rows, g;
    if constexpr (MODE == MQ_DENSE) {
      rows = a.seg[NT == 2 ? cc.m : cc.seg].rows;
      g = cc.fg - a.seg[cc.seg].blk_begin;
    } else {
      rows = MODE == MQ_GATE_UP ? mo.f : mo.h;
      g = cc.fg;
    }
    if (!(u < U && QROWS * g + r < rows)) v = 0.f;
    v += __shfl_xor(v, 16, 64);
    if (!cc.pair) v += __shfl_xor(v, 32, 64);
    if (q == 0) S.part[cc.slot * QROWS + r] = v;
    if (cc.pair && q == 2) S.part[(cc.slot + Tl) * QROWS + r] = v;  // slot m + 1, same quad
  };
  if constexpr (DEPTH == 3) {
    for (;;) {
      if (c0 >= nitems) break;
      c2 = grab();
      if (c2 < nitems) load(R2, c2);
      consume(R0, c0);
      if (c1 >= nitems) break;
      c0 = grab();
      if (c0 < nitems) load(R0, c0);
      consume(R1, c1);
      if (c2 >= nitems) break;
      c1 = grab();
      if (c1 < nitems) load(R1, c1);
      consume(R2, c2);
    }
  } else {
    for (;;) {
      if (c0 >= nitems) break;
      c1 = grab();
      if (c1 < nitems) load(R1, c1);
      consume(R0, c0);
      if (c1 >= nitems) break;
      c0 = grab();
      if (c0 < nitems) load(R0, c0);
      consume(R1, c1);
    }
  }
  __syncthreads();

  // ---- per-row sums over the items, in item order
  if constexpr (MODE == MQ_GATE_UP) {  // h_p = silu(gate . x) * (up . x)
    for (int lr = tid; lr < rows_blk; lr += NTH) {
      const int lg = lr / QROWS, rr = lr % QROWS;
      const int row = (b + lg * B) * QROWS + rr;
      float v[2];
#pragma unroll
      for (int m = 0; m < 2; m++) {
        float s = 0.f;
        const float *pp = S.part + ((lg * 2 + m) * Tl) * QROWS + rr;
        for (int t = 0; t < Tl; t++) s += pp[t * QROWS];
        v[m] = s;
      }
      mo.hbuf[(long)p * mo.f + row] = v[0] / (1.0f + expf(-v[0])) * v[1];
    }
    return;
  }
  if constexpr (MODE == MQ_DOWN) {  // out_t = sum_s w_s (down_(e_s) . h_s), slots in order
    for (int lr = tid; lr < rows_blk; lr += NTH) {
      const int lg = lr / QROWS, rr = lr % QROWS;
      const int row = (b + lg * B) * QROWS + rr;
      float out = 0.f;
      for (int m = 0; m < NM; m++) {
        float s = 0.f;
        const float *pp = S.part + ((lg * NM + m) * Tl) * QROWS + rr;
        for (int t = 0; t < Tl; t++) s += pp[t * QROWS];
        out += mo.w[p * NM + m] * s;
      }
      mo.out[(long)p * mo.h + row] = out;
    }
    return;
  }
  float bv = -INFINITY;  // this thread's first maximum (fused argmax)
  int bi = 0x7fffffff;
  for (int lr = tid; lr < rows_blk; lr += NTH) {
    const int lg = lr / QROWS, rr = lr % QROWS;
    const int fg = b + lg * B;
    int sgi = 0;
    if constexpr (NT == 1) {
#pragma unroll
      for (int i = 1; i < MV_MAX_SEG; i++)
        if (i < a.nseg && fg >= a.seg[i].blk_begin) sgi = i;
    }
    const MvSeg &sg = a.seg[sgi];
    const int row = (fg - sg.blk_begin) * QROWS + rr;
    if (row >= sg.rows) continue;
    float v[NT];
#pragma unroll
    for (int m = 0; m < NT; m++) {
      float s = 0.f;
      const float *pp = S.part + ((lg * NT + m) * Tl) * QROWS + rr;
      for (int t = 0; t < Tl; t++) s += pp[t * QROWS];
      v[m] = s * rscale;
    }
    float out = v[0];
    if constexpr (NT == 2) out = v[0] / (1.0f + expf(-v[0])) * v[1];
    if (NT == 1 && a.in.res && !h1) out = a.in.res[row] + out;  // (one-matrix launches)
    (h1 ? a.in.y2 : sg.y)[row] = out;
    if (out > bv) {  // rows rise with lr: strict > keeps the first maximum; NaN never wins
      bv = out;
      bi = row;
    }
  }
  if constexpr (NT == 1) {
    if (a.in.amax_v) {  // the block's first maximum (ties: lower row)
      __shared__ float av[NW];
      __shared__ int ai[NW];
      auto merge = [](float &v0, int &i0, float v1, int i1) {
        if (v1 > v0 || (v1 == v0 && i1 < i0)) {
          v0 = v1;
          i0 = i1;
        }
      };
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) merge(bv, bi, __shfl_xor(bv, off, 64), __shfl_xor(bi, off, 64));
      if (lane == 0) {
        av[wave] = bv;
        ai[wave] = bi;
      }
      __syncthreads();
      if (tid == 0) {
        for (int w = 1; w < NW; w++) merge(bv, bi, av[w], ai[w]);
        a.in.amax_v[b] = bv;
        a.in.amax_i[b] = bi;
      }
    }
  }
}

template <int FMT, bool K4, int SRC, int NT, bool ONE>
__global__ __launch_bounds__(64 * mvq_waves(FMT)) void k_mvq(MvArgs a) {
  mvq_body<FMT, K4, SRC, NT, MQ_DENSE, false, ONE>(a, MoeArgs{});
}

// The MoE stages (MODE MQ_GATE_UP with or without in-kernel routing, or
// MQ_DOWN); K4: the staged inputs' length (h, f) is a multiple of 4.
template <int FMT, bool K4, int MODE, bool ROUTE, bool ONE>
__global__ __launch_bounds__(64 * mvq_waves(FMT)) void k_mvq_moe(MoeArgs mo) {
  mvq_body<FMT, K4, MV_X, MODE == MQ_GATE_UP ? 2 : 1, MODE, ROUTE, ONE>(MvArgs{}, mo);
}

template <int FMT, bool K4, int SRC, int NT, bool ONE>
hipError_t mvq_launch_o(const MvArgs &a, size_t lds, hipStream_t st) {
  if (lds > 64 * 1024)
    (void)hipFuncSetAttribute((const void *)k_mvq<FMT, K4, SRC, NT, ONE>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL((k_mvq<FMT, K4, SRC, NT, ONE>), dim3(a.blocks), dim3(64 * mvq_waves(FMT)), lds, st, a);
  return hipGetLastError();
}

// one staging pass when the input fits one (units <= NTH / 16)
template <int FMT, bool K4, int SRC, int NT>
hipError_t mvq_launch_t(const MvArgs &a, size_t lds, hipStream_t st) {
  const int ux = a.ksplit > 0 ? std::max(4 * a.ksplit, a.units - 4 * a.ksplit) : a.units;
  return ux * 16 <= 64 * mvq_waves(FMT) ? mvq_launch_o<FMT, K4, SRC, NT, true>(a, lds, st)
                                        : mvq_launch_o<FMT, K4, SRC, NT, false>(a, lds, st);
}

template <int FMT>
hipError_t mvq_launch_f(const MvArgs &a, size_t lds, hipStream_t st) {
  const bool k4 = a.k % 4 == 0;
  switch (a.in.src) {
  case MV_NORM:
    if (!k4) return hipErrorInvalidValue;
    return a.pair ? mvq_launch_t<FMT, true, MV_NORM, 2>(a, lds, st) : mvq_launch_t<FMT, true, MV_NORM, 1>(a, lds, st);
  case MV_SWIGLU:
    if (a.pair) return hipErrorInvalidValue;
    return k4 ? mvq_launch_t<FMT, true, MV_SWIGLU, 1>(a, lds, st) : mvq_launch_t<FMT, false, MV_SWIGLU, 1>(a, lds, st);
  default:
    if (a.pair) return hipErrorInvalidValue;
    return k4 ? mvq_launch_t<FMT, true, MV_X, 1>(a, lds, st) : mvq_launch_t<FMT, false, MV_X, 1>(a, lds, st);
  }
}

}  // namespace

// Static LDS of the quad-layout kernels' blocks, a bound: IQ3_XXS's tables
// and the fused argmax's per-wave maxima.
size_t mvq_static_lds(int fmt) { return (fmt == T_IQ3_XXS ? IQ3_TABLE_WORDS * 4 : 0) + 256; }

namespace {
int aux_per_unit(int fmt) {
  return fmt == T_Q4_K || fmt == T_Q5_K ? 8 : fmt == T_Q8_0 || fmt == T_IQ3_XXS ? 0 : 16;
}

}  // namespace

// Groups and blocks of a quad-layout launch; returns the LDS bytes a block
// needs.  The launch's flat row-group count goes to groups, segment i's
// first flat group to seg[i].blk_begin.
size_t mvq_plan(MvArgs &a, int num_cus) {
  const int nt = a.pair ? 2 : 1, nseg = a.pair ? 1 : a.nseg;
  int G = 0;
  for (int i = 0; i < nseg; i++) {
    a.seg[i].blk_begin = G;
    a.seg[i].nblk = 0;
    G += (a.seg[i].rows + QROWS - 1) / QROWS;
  }
  if (a.pair) a.seg[1].blk_begin = 0;
  a.groups = G;
  a.ksplit = 0;
  a.blocks0 = 0;
  const int fmt = a.fmt == T_Q5_K && a.in.q8k && !a.pair ? T_Q5_K8 : a.fmt;
  const int T = (a.units + 3) / 4;
  if (a.in.y2) {
    // K split: half 0 takes quads [0, T / 2), half 1 the rest; the blocks
    // (at most one per CU, at most G per half) go to the halves in
    // proportion to their quads.
    const int ts = T / 2, tot = std::max(2, std::min(2 * G, num_cus));
    a.ksplit = ts;
    a.blocks0 = std::max(1, std::min(G, (int)((long)tot * ts / T)));
    const int b1 = std::max(1, std::min(G, tot - a.blocks0));
    a.blocks = a.blocks0 + b1;
    const int ngb = std::max((G + a.blocks0 - 1) / a.blocks0, (G + b1 - 1) / b1);
    const int ux = std::max(4 * ts, a.units - 4 * ts), tl = std::max(ts, T - ts);
    return qsmem_layout(aux_per_unit(fmt), ux, ngb * tl * QROWS, nullptr, nullptr);
  }
  static const int bpc = [] {
    const char *e = getenv("GQ_MVQ_BLOCKS_PER_CU");  // tuning override
    return e && atoi(e) > 0 ? atoi(e) : 1;
  }();
  a.blocks = std::max(1, std::min(G, num_cus * bpc));
  // Launches that stream many row groups per block (the output head: 9504
  // groups) run faster on 27 blocks per 32 CUs than on one per CU (measured
  // on the 152064 x 3584 Q6_K head: 67.9 against 70.2 us; smaller launches
  // keep one block per CU).
  if (bpc == 1 && G >= 16 * num_cus) a.blocks = std::max(1, num_cus * 27 / 32);
  // Small launches: no more blocks than give each wave one item (group x
  // quad) to stream -- fewer x stagings, and every block's waves busy.
  // Measured: q/k/v 3584+512+512 x 3584 on 144 blocks 5.30-5.37 against
  // 5.63-5.65 us on 256; the Q8_0 8192 x 2048 matrix on 128 blocks 6.44-6.52
  // against 6.81-6.82 us.
  if (bpc == 1) {
    const long items = (long)G * ((a.units + 3) / 4) * nt;
    const int nw = mvq_waves(a.fmt == T_Q5_K && a.in.q8k && !a.pair ? T_Q5_K8 : a.fmt);
    a.blocks = (int)std::max(1L, std::min((long)a.blocks, (items + nw - 1) / nw));
  }
  // Even split: as few blocks as give the same largest number of row groups
  // per block (gate/up, 2368 groups: 237 blocks of 10 instead of 256 of 9 or
  // 10; measured 15.3 against 15.6-15.8 us).
  {
    const int gpb = (G + a.blocks - 1) / a.blocks;
    a.blocks = (G + gpb - 1) / gpb;
  }
  static const int maxb = [] {
    const char *e = getenv("GQ_MVQ_MAX_BLOCKS");  // tuning override: at most this many blocks
    return e && atoi(e) > 0 ? atoi(e) : 1 << 30;
  }();
  a.blocks = std::min(a.blocks, maxb);
  // The fused argmax writes one partial per block into ARGMAX_SLOTS slots.
  if (a.in.amax_v) a.blocks = std::min(a.blocks, ARGMAX_SLOTS);
  const int ngb = (G + a.blocks - 1) / a.blocks;
  return qsmem_layout(aux_per_unit(fmt), a.units, ngb * nt * T * QROWS, nullptr, nullptr);
}

// MoE stage plans: about one block per CU in all (blocks per pair / per
// token), more while a block's LDS would not fit.
size_t mvq_moe_plan(MoeArgs &a, int T, int stage, int num_cus) {
  const int fmt = a.fmt == T_Q5_K ? T_Q5_K8 : a.fmt, aux = aux_per_unit(fmt);  // (Q5_K: Q8_K route)
  const int st = (int)mvq_static_lds(fmt);
  if (stage == 1) {
    const int G = a.f / QROWS, Tq = (a.units_h + 3) / 4, pairs = T * a.top_k;
    const int rstatic = MOE_ROUTE_MAX * 16 + 256;  // moe_route_pair's arrays
    a.bpp = std::max(1, std::min(G, num_cus / std::max(1, pairs)));
    for (;;) {
      const int ngb = (G + a.bpp - 1) / a.bpp;
      a.part_h = ngb * 2 * Tq * QROWS;
      a.lds_gu = (int)qsmem_layout(aux, a.units_h, a.part_h, nullptr, nullptr);
      if (a.lds_gu + rstatic + st <= 160 * 1024 || a.bpp >= G) return a.lds_gu + rstatic + st;
      a.bpp = std::min(G, 2 * a.bpp);
    }
  }
  const int G = a.h / QROWS, Tq = (a.units_f + 3) / 4, K = a.top_k;
  a.bpt = std::max(1, std::min(G, num_cus / std::max(1, T)));
  for (;;) {
    const int ngb = (G + a.bpt - 1) / a.bpt;
    a.part_f = ngb * K * Tq * QROWS;
    a.lds_dn = (int)qsmem_layout(aux, K * 4 * Tq, a.part_f, nullptr, nullptr);
    if (a.lds_dn + st <= 160 * 1024 || a.bpt >= G) return a.lds_dn + st;
    a.bpt = std::min(G, 2 * a.bpt);
  }
}

template <int FMT, bool K4, int MODE, bool ROUTE, bool ONE>
static hipError_t mvq_moe_o(const MoeArgs &a, int grid, int lds, hipStream_t st) {
  if (lds > 64 * 1024)
    (void)hipFuncSetAttribute((const void *)k_mvq_moe<FMT, K4, MODE, ROUTE, ONE>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  hipLaunchKernelGGL((k_mvq_moe<FMT, K4, MODE, ROUTE, ONE>), dim3(grid), dim3(64 * mvq_waves(FMT)),
                     lds, st, a);
  return hipGetLastError();
}

template <int FMT, bool K4, int MODE, bool ROUTE>
static hipError_t mvq_moe_t(const MoeArgs &a, int grid, int lds, hipStream_t st) {
  // staged units: gate/up units_h; down top_k slots of 4T units each
  const int ux = MODE == MQ_GATE_UP ? a.units_h : a.top_k * 4 * ((a.units_f + 3) / 4);
  return ux * 16 <= 64 * mvq_waves(FMT) ? mvq_moe_o<FMT, K4, MODE, ROUTE, true>(a, grid, lds, st)
                                        : mvq_moe_o<FMT, K4, MODE, ROUTE, false>(a, grid, lds, st);
}

template <int FMT>
static hipError_t mvq_moe_f(const MoeArgs &a, int T, int stage, bool route, hipStream_t st) {
  if (stage == 1) {
    const int grid = T * a.top_k * a.bpp;
    if (a.h % 4 == 0)
      return route ? mvq_moe_t<FMT, true, MQ_GATE_UP, true>(a, grid, a.lds_gu, st)
                   : mvq_moe_t<FMT, true, MQ_GATE_UP, false>(a, grid, a.lds_gu, st);
    return route ? mvq_moe_t<FMT, false, MQ_GATE_UP, true>(a, grid, a.lds_gu, st)
                 : mvq_moe_t<FMT, false, MQ_GATE_UP, false>(a, grid, a.lds_gu, st);
  }
  const int grid = T * a.bpt;
  return a.f % 4 == 0 ? mvq_moe_t<FMT, true, MQ_DOWN, false>(a, grid, a.lds_dn, st)
                      : mvq_moe_t<FMT, false, MQ_DOWN, false>(a, grid, a.lds_dn, st);
}

hipError_t launch_mvq_moe(const MoeArgs &a, int T, int stage, bool route, hipStream_t st) {
  if ((stage == 1 ? a.f : a.h) % QROWS || a.top_k > 64) return hipErrorInvalidValue;
  switch (a.fmt) {
  case T_Q4_K: return mvq_moe_f<T_Q4_K>(a, T, stage, route, st);
  case T_Q5_K: return mvq_moe_f<T_Q5_K8>(a, T, stage, route, st);  // matmul_into's Q8_K route
  case T_Q6_K: return mvq_moe_f<T_Q6_K>(a, T, stage, route, st);
  case T_Q8_0: return mvq_moe_f<T_Q8_0>(a, T, stage, route, st);
  case T_IQ3_XXS: return mvq_moe_f<T_IQ3_XXS>(a, T, stage, route, st);
  default: return hipErrorInvalidValue;
  }
}

hipError_t launch_mvq(const MvArgs &a, size_t lds, hipStream_t st) {
  if (lds + mvq_static_lds(a.fmt) > 160 * 1024) return hipErrorInvalidValue;
  if (a.in.amax_v && a.blocks > ARGMAX_SLOTS) return hipErrorInvalidValue;
  // the split: one matrix, plain x, two quads per row, no argmax
  if (a.in.y2 && (a.pair || a.nseg != 1 || a.in.src != MV_X || a.in.amax_v || !mv_ksplit_ok(a.units) ||
                  a.ksplit <= 0))
    return hipErrorInvalidValue;
  switch (a.fmt) {
  case T_Q4_K: return mvq_launch_f<T_Q4_K>(a, lds, st);
  case T_Q5_K: return a.in.q8k && !a.pair ? mvq_launch_f<T_Q5_K8>(a, lds, st) : mvq_launch_f<T_Q5_K>(a, lds, st);
  case T_Q6_K: return mvq_launch_f<T_Q6_K>(a, lds, st);
  case T_Q8_0: return mvq_launch_f<T_Q8_0>(a, lds, st);
  case T_IQ3_XXS: return mvq_launch_f<T_IQ3_XXS>(a, lds, st);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace gq

