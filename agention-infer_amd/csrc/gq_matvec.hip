// gq_matvec.hip -- batch-1 decode matvec y = W . x for Q8_0, Q4_K, Q5_K,
// Q6_K and IQ3_XXS weights (gfx950, wave64).
//
// Replaces the reference's per-row dot kernels (src/quant/q8_0.rs:58-90,
// q4_k.rs:95-212, q5_k.rs:189-317, q6_k.rs:82-131) driven row-parallel by
// WeightMap::matmul_into (src/model/mod.rs:362-403), and the reference GPU
// matvec (src/ops/kernels_wgpu.rs:1067-1706), which this does not follow.
//
// Design (HBM-bound: every weight byte is read once):
//  * A 256-thread block first stages x (fp32, zero-padded to whole blocks)
//    and the sums of x over each 16-element run in LDS.  The runs let the
//    kernels factor constant offsets out of the inner loop:
//      Q4_K  sum (d*sc*q - dmin*m) x = d*sc*sum(q x) - dmin*m*sum(x)
//      Q6_K  sum (q - 32) x          = sum(q x) - 32*sum(x)
//      Q8_0  sum q x with q = u - 128, u = q ^ 0x80 unsigned byte
//    so each weight element costs one byte->float convert and one FMA.
//  * LPR lanes cooperate on one row; consecutive lanes read consecutive
//    16-byte pieces of a weight block with 128-bit loads, so one load
//    instruction of a wave covers 64/LPR rows x LPR*16 contiguous bytes.
//  * Partial sums are reduced across the LPR lanes with xor shuffles.
//  * The grid is capped and waves loop over row groups, so x is staged
//    once per block rather than once per row group.
#include "gq_device.h"
#include "gq_internal.h"

namespace gq {

struct RowCtx {
  const uint8_t *body;  // this segment's body
  const uint16_t *d;    // per-block f16 scales (layouts with a d array)
  long stride;          // body bytes per row
  int nb;               // blocks per row
};

// ---------------------------------------------------------------- Q4_K
// One unit = 16 B of qs: group j = s/2, half h = s%2.  Low nibbles are
// elements 64j+16h+[0,16) (sub-block 2j), high nibbles +32 (sub-block 2j+1).
template <int LPR>
__device__ __forceinline__ float row_q4k(const RowCtx &c, int r, int sl, const float *xs,
                                         const float *s16) {
  const int s = sl & 7, bo = sl >> 3;
  constexpr int step = LPR / 8;
  const int j = s >> 1, h = s & 1;
  const int e_lo = 64 * j + 16 * h;
  const uint8_t *rp = c.body + (long)r * c.stride;
  float acc = 0.f;
#pragma unroll 2
  for (int b = bo; b < c.nb; b += step) {
    const uint4 hd = *(const uint4 *)(rp + b * 144);
    const uint4 q = *(const uint4 *)(rp + b * 144 + 16 + 16 * s);
    uint32_t sc0, m0, sc1, m1;
    scale_min_k4(2 * j, hd.y, hd.z, hd.w, sc0, m0);
    scale_min_k4(2 * j + 1, hd.y, hd.z, hd.w, sc1, m1);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    const float *xl = xs + b * 256 + e_lo;
    float sl_ = 0.f, sh_ = 0.f;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
      sl_ = dot4u(lo, *(const float4 *)(xl + 4 * k), sl_);
      sh_ = dot4u(hi, *(const float4 *)(xl + 32 + 4 * k), sh_);
    }
    const int g = (b * 256 + e_lo) >> 4;
    acc = fmaf(d * (float)sc0, sl_, acc);
    acc = fmaf(-(dmin * (float)m0), s16[g], acc);
    acc = fmaf(d * (float)sc1, sh_, acc);
    acc = fmaf(-(dmin * (float)m1), s16[g + 2], acc);
  }
  return acc;
}

// ---------------------------------------------------------------- Q5_K
// As Q4_K, plus the fifth bit from qh[l] (bit `is` of the 32-byte qh).
template <int LPR>
__device__ __forceinline__ float row_q5k(const RowCtx &c, int r, int sl, const float *xs,
                                         const float *s16) {
  const int s = sl & 7, bo = sl >> 3;
  constexpr int step = LPR / 8;
  const int j = s >> 1, h = s & 1;
  const int e_lo = 64 * j + 16 * h;
  const uint8_t *rp = c.body + (long)r * c.stride;
  float acc = 0.f;
#pragma unroll 2
  for (int b = bo; b < c.nb; b += step) {
    const uint8_t *bp = rp + b * 176;
    const uint4 hd = *(const uint4 *)bp;
    const uint4 qh = *(const uint4 *)(bp + 16 + 16 * h);
    const uint4 q = *(const uint4 *)(bp + 48 + 16 * s);
    uint32_t sc0, m0, sc1, m1;
    scale_min_k4(2 * j, hd.y, hd.z, hd.w, sc0, m0);
    scale_min_k4(2 * j + 1, hd.y, hd.z, hd.w, sc1, m1);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    const float *xl = xs + b * 256 + e_lo;
    float sl_ = 0.f, sh_ = 0.f;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const uint32_t hw[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t lo = (qw[k] & 0x0F0F0F0Fu) | (((hw[k] >> (2 * j)) & 0x01010101u) << 4);
      const uint32_t hi =
          ((qw[k] >> 4) & 0x0F0F0F0Fu) | (((hw[k] >> (2 * j + 1)) & 0x01010101u) << 4);
      sl_ = dot4u(lo, *(const float4 *)(xl + 4 * k), sl_);
      sh_ = dot4u(hi, *(const float4 *)(xl + 32 + 4 * k), sh_);
    }
    const int g = (b * 256 + e_lo) >> 4;
    acc = fmaf(d * (float)sc0, sl_, acc);
    acc = fmaf(-(dmin * (float)m0), s16[g], acc);
    acc = fmaf(d * (float)sc1, sh_, acc);
    acc = fmaf(-(dmin * (float)m1), s16[g + 2], acc);
  }
  return acc;
}

// ---------------------------------------------------------------- Q6_K
// One unit = half hh = s/2, l in [16*(s%2), +16): 16 B of ql at l, 16 B of
// ql at l+32, 16 B of qh at l -> 64 elements in four runs of 16
// (elements 128hh + l + 32t, t = 0..3), scale index 8hh + s%2 + 2t.
template <int LPR>
__device__ __forceinline__ float row_q6k(const RowCtx &c, int r, int sl, const float *xs,
                                         const float *s16) {
  const int s = sl & 3, bo = sl >> 2;
  constexpr int step = LPR / 4;
  const int hh = s >> 1, lh = s & 1;
  const uint8_t *rp = c.body + (long)r * c.stride;
  const uint16_t *dp = c.d + (long)r * c.nb;
  float acc = 0.f;
#pragma unroll 2
  for (int b = bo; b < c.nb; b += step) {
    const uint8_t *bp = rp + b * 208;
    const uint4 A = *(const uint4 *)(bp + 64 * hh + 16 * lh);
    const uint4 B = *(const uint4 *)(bp + 64 * hh + 32 + 16 * lh);
    const uint4 H = *(const uint4 *)(bp + 128 + 32 * hh + 16 * lh);
    const uint4 SC = *(const uint4 *)(bp + 192);
    const float d = h2f(dp[b]);
    const uint32_t w0 = hh ? SC.z : SC.x, w1 = hh ? SC.w : SC.y;
    const int sh = 8 * lh;
    const float sc0 = (float)(int8_t)(w0 >> sh), sc1 = (float)(int8_t)(w0 >> (sh + 16));
    const float sc2 = (float)(int8_t)(w1 >> sh), sc3 = (float)(int8_t)(w1 >> (sh + 16));
    const uint32_t aw[4] = {A.x, A.y, A.z, A.w}, bw[4] = {B.x, B.y, B.z, B.w};
    const uint32_t hw[4] = {H.x, H.y, H.z, H.w};
    const float *xb = xs + b * 256 + 128 * hh + 16 * lh;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t q1 = (aw[k] & 0x0F0F0F0Fu) | ((hw[k] << 4) & 0x30303030u);
      const uint32_t q2 = (bw[k] & 0x0F0F0F0Fu) | ((hw[k] << 2) & 0x30303030u);
      const uint32_t q3 = ((aw[k] >> 4) & 0x0F0F0F0Fu) | (hw[k] & 0x30303030u);
      const uint32_t q4 = ((bw[k] >> 4) & 0x0F0F0F0Fu) | ((hw[k] >> 2) & 0x30303030u);
      s0 = dot4u(q1, *(const float4 *)(xb + 4 * k), s0);
      s1 = dot4u(q2, *(const float4 *)(xb + 32 + 4 * k), s1);
      s2 = dot4u(q3, *(const float4 *)(xb + 64 + 4 * k), s2);
      s3 = dot4u(q4, *(const float4 *)(xb + 96 + 4 * k), s3);
    }
    const int g = (b * 256 + 128 * hh + 16 * lh) >> 4;
    float t = sc0 * fmaf(-32.f, s16[g], s0);
    t = fmaf(sc1, fmaf(-32.f, s16[g + 2], s1), t);
    t = fmaf(sc2, fmaf(-32.f, s16[g + 4], s2), t);
    t = fmaf(sc3, fmaf(-32.f, s16[g + 6], s3), t);
    acc = fmaf(d, t, acc);
  }
  return acc;
}

// ---------------------------------------------------------------- Q8_0
// One unit = 16 int8 quants (half a block).
template <int LPR>
__device__ __forceinline__ float row_q80(const RowCtx &c, int r, int sl, const float *xs,
                                         const float *s16) {
  const uint8_t *rp = c.body + (long)r * c.stride;
  const uint16_t *dp = c.d + (long)r * c.nb;
  const int nc = 2 * c.nb;
  float acc = 0.f;
#pragma unroll 2
  for (int u = sl; u < nc; u += LPR) {
    const uint4 q = *(const uint4 *)(rp + 16 * u);
    const float d = h2f(dp[u >> 1]);
    const float *xb = xs + 16 * u;
    float sum = 0.f;
    sum = dot4u(q.x ^ 0x80808080u, *(const float4 *)(xb + 0), sum);
    sum = dot4u(q.y ^ 0x80808080u, *(const float4 *)(xb + 4), sum);
    sum = dot4u(q.z ^ 0x80808080u, *(const float4 *)(xb + 8), sum);
    sum = dot4u(q.w ^ 0x80808080u, *(const float4 *)(xb + 12), sum);
    acc = fmaf(d, fmaf(-128.f, s16[u], sum), acc);
  }
  return acc;
}

// ------------------------------------------------------------- IQ3_XXS
// One unit = one 32-element sub-block ib = s: 8 grid indices + one aux word.
template <int LPR>
__device__ __forceinline__ float row_iq3(const RowCtx &c, int r, int sl, const float *xs,
                                         const uint32_t *grid) {
  const int s = sl & 7, bo = sl >> 3;
  constexpr int step = LPR / 8;
  const uint8_t *rp = c.body + (long)r * c.stride;
  const uint16_t *dp = c.d + (long)r * c.nb;
  float acc = 0.f;
#pragma unroll 2
  for (int b = bo; b < c.nb; b += step) {
    const uint8_t *bp = rp + b * 96;
    const uint2 qi = *(const uint2 *)(bp + 8 * s);
    const uint32_t aux = *(const uint32_t *)(bp + 64 + 4 * s);
    const float d = h2f(dp[b]);
    const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    const float *xb = xs + b * 256 + 32 * s;
    float sum = 0.f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t sg = ksign7((aux >> (7 * l)) & 127u);
      const uint32_t word = l < 2 ? qi.x : qi.y;
      const uint32_t g1 = grid[(word >> (16 * (l & 1))) & 0xff];
      const uint32_t g2 = grid[(word >> (16 * (l & 1) + 8)) & 0xff];
      const float4 xa = *(const float4 *)(xb + 8 * l), xc = *(const float4 *)(xb + 8 * l + 4);
      float4 ya, yc;
      ya.x = __uint_as_float(__float_as_uint(xa.x) ^ ((sg & 1u) << 31));
      ya.y = __uint_as_float(__float_as_uint(xa.y) ^ ((sg & 2u) << 30));
      ya.z = __uint_as_float(__float_as_uint(xa.z) ^ ((sg & 4u) << 29));
      ya.w = __uint_as_float(__float_as_uint(xa.w) ^ ((sg & 8u) << 28));
      yc.x = __uint_as_float(__float_as_uint(xc.x) ^ ((sg & 16u) << 27));
      yc.y = __uint_as_float(__float_as_uint(xc.y) ^ ((sg & 32u) << 26));
      yc.z = __uint_as_float(__float_as_uint(xc.z) ^ ((sg & 64u) << 25));
      yc.w = __uint_as_float(__float_as_uint(xc.w) ^ ((sg & 128u) << 24));
      sum = dot4u(g1, ya, sum);
      sum = dot4u(g2, yc, sum);
    }
    acc = fmaf(db, sum, acc);
  }
  return acc;
}

// ------------------------------------------------------------- kernel
template <int FMT, int LPR>
__global__ __launch_bounds__(256) void k_matvec(MvArgs a) {
  extern __shared__ float smem[];
  float *xs = smem;
  float *s16 = smem + a.kpad;
  uint32_t *grid = (uint32_t *)(s16 + a.kpad / 16);
  const int tid = threadIdx.x;
  for (int i = tid; i < a.kpad; i += 256) xs[i] = i < a.k ? a.x[i] : 0.f;
  if (FMT == T_IQ3_XXS) grid[tid] = a.grid[tid];
  __syncthreads();
  for (int i = tid; i < a.kpad / 16; i += 256) {
    const float4 *p = (const float4 *)(xs + 16 * i);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float4 v = p[k];
      s += v.x; s += v.y; s += v.z; s += v.w;
    }
    s16[i] = s;
  }
  __syncthreads();

  constexpr int RPW = 64 / LPR;
  const int lane = tid & 63, wave = tid >> 6;
  const int sl = lane % LPR, rg = lane / LPR;
  for (int row0 = (blockIdx.x * 4 + wave) * RPW; row0 < a.total_rows;
       row0 += gridDim.x * 4 * RPW) {
    const int r = row0 + rg;
    float acc = 0.f;
    int seg = 0;
    if (r < a.total_rows) {
#pragma unroll
      for (int i = 1; i < MV_MAX_SEG; i++)
        if (i < a.nseg && r >= a.seg[i].row_begin) seg = i;
      const MvSeg &S = a.seg[seg];
      const RowCtx c{S.body, S.d, S.stride, a.nb};
      const int rr = r - S.row_begin;
      if (FMT == T_Q4_K) acc = row_q4k<LPR>(c, rr, sl, xs, s16);
      else if (FMT == T_Q5_K) acc = row_q5k<LPR>(c, rr, sl, xs, s16);
      else if (FMT == T_Q6_K) acc = row_q6k<LPR>(c, rr, sl, xs, s16);
      else if (FMT == T_Q8_0) acc = row_q80<LPR>(c, rr, sl, xs, s16);
      else acc = row_iq3<LPR>(c, rr, sl, xs, grid);
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (sl == 0 && r < a.total_rows) a.seg[seg].y[r - a.seg[seg].row_begin] = acc;
  }
}

// ------------------------------------------------------------- launch
template <int FMT, int LPR>
static void launch_one(const MvArgs &a, int blocks, size_t lds, hipStream_t st) {
  if (lds > 64 * 1024)
    (void)hipFuncSetAttribute((const void *)k_matvec<FMT, LPR>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL((k_matvec<FMT, LPR>), dim3(blocks), dim3(256), lds, st, a);
}

template <int FMT>
static hipError_t launch_fmt(const MvArgs &a, int lpr, int blocks, size_t lds, hipStream_t st) {
  switch (lpr) {
  case 4:
    if (FMT == T_Q6_K) { launch_one<FMT, 4>(a, blocks, lds, st); break; }
    [[fallthrough]];  // the other formats need at least 8 lanes per row
  case 8: launch_one<FMT, 8>(a, blocks, lds, st); break;
  case 16: launch_one<FMT, 16>(a, blocks, lds, st); break;
  case 32: launch_one<FMT, 32>(a, blocks, lds, st); break;
  default: launch_one<FMT, 64>(a, blocks, lds, st); break;
  }
  return hipGetLastError();
}

size_t matvec_lds_bytes(int kpad) { return (size_t)kpad * 4 + (size_t)kpad / 16 * 4 + 1024; }

// Lanes per row: the smallest that still gives >= ~8 waves per CU, but no
// more lanes than units in a row.
static int pick_lpr(int fmt, int rows, int nb) {
  const int unit_lanes = fmt == T_Q6_K ? 4 : 8;
  const int units = fmt == T_Q8_0 ? 2 * nb : nb * unit_lanes;  // units per row
  int lpr = fmt == T_Q8_0 ? 8 : unit_lanes;
  while (lpr < 64 && (long)rows * lpr / 64 < 2048 && units >= 2 * lpr) lpr *= 2;
  return lpr;
}

hipError_t launch_matvec(const MvArgs &a, int fmt, int num_cus, hipStream_t st) {
  const int lpr = pick_lpr(fmt, a.total_rows, a.nb);
  const int rows_per_block = 4 * (64 / lpr);
  long blocks = (a.total_rows + rows_per_block - 1) / rows_per_block;
  const size_t lds = matvec_lds_bytes(a.kpad);
  // Blocks that fit per CU given LDS, times CUs: one resident wave of blocks.
  long per_cu = (long)(160 * 1024 / lds);
  if (per_cu > 8) per_cu = 8;
  if (per_cu < 1) per_cu = 1;
  const long cap = per_cu * num_cus;
  if (blocks > cap) blocks = cap;
  switch (fmt) {
  case T_Q4_K: return launch_fmt<T_Q4_K>(a, lpr, (int)blocks, lds, st);
  case T_Q5_K: return launch_fmt<T_Q5_K>(a, lpr, (int)blocks, lds, st);
  case T_Q6_K: return launch_fmt<T_Q6_K>(a, lpr, (int)blocks, lds, st);
  case T_Q8_0: return launch_fmt<T_Q8_0>(a, lpr, (int)blocks, lds, st);
  case T_IQ3_XXS: return launch_fmt<T_IQ3_XXS>(a, lpr, (int)blocks, lds, st);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace gq
