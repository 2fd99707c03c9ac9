// gq_dequant.hip -- upload re-layout, bit-exact dequant, and the per-32 Q8
// activation pack.
//
// Dequant restates, per element, the arithmetic of the reference's
// dequant_q8_0 (src/quant/q8_0.rs:14-51), dequant_q4_k (q4_k.rs:37-91),
// dequant_q5_k (q5_k.rs:41-99) and dequant_q6_k (q6_k.rs:34-77), in the same
// operation order; the library is built with -ffp-contract=off, so each
// product and difference rounds separately, as in Rust.  IQ3_XXS follows
// ggml's dequantize_row_iq3_xxs (no reference implementation exists).
#include "gq_device.h"
#include "gq_internal.h"

namespace gq {

// ------------------------------------------------------------------ repack
// Byte o of the logical bytes of unit `u` of row r, read from the raw ggml
// row (nb ggml blocks).  Q8_0 units past the row's last block read zero.
__device__ inline uint8_t logical_byte(int dtype, bool quad, const uint8_t *row, int nb, int u, int o) {
  if (dtype == T_IQ3_XXS && quad) {  // re-encoded sub-blocks (iq3q_pack)
    uint32_t w[3];
    iq3q_pack(row + u * 98 + 2, o / 12, w);
    return (uint8_t)(w[(o % 12) >> 2] >> (8 * (o & 3)));
  }
  switch (dtype) {
  case T_Q4_K: return row[u * 144 + o];
  case T_Q5_K: return row[u * 176 + o];
  case T_Q6_K: return row[u * 210 + o];
  case T_IQ3_XXS: return row[u * 98 + 2 + o];
  default: {  // Q8_0: qs of blocks 8u..8u+7, then their d's
    const int b = 8 * u + (o < 256 ? o >> 5 : (o - 256) >> 1);
    if (b >= nb) return 0;
    return o < 256 ? row[b * 34 + 2 + (o & 31)] : row[b * 34 + ((o - 256) & 1)];
  }
  }
}

// One thread per (row, unit): scatter the unit's chunks into the layout.
__global__ void k_repack(Layout L, const uint8_t *raw, long raw_row_bytes, int nb, uint8_t *body,
                         uint16_t *dd) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)L.rows * L.units) return;
  const int r = (int)(i / L.units), u = (int)(i % L.units);
  const uint8_t *row = raw + (long)r * raw_row_bytes;
  const int t = r / L.rt, j = (r % L.rt) * L.units + u;
  for (int c = 0; c < L.chunks; c++) {
    uint8_t *dst = body + chunk_offset(L, t, j, c);
    for (int k = 0; k < 16; k++) dst[k] = logical_byte(L.dtype, L.quad, row, nb, u, 16 * c + k);
  }
  if (dd) {
    const uint8_t *b = L.dtype == T_Q6_K ? row + u * 210 + 208 : row + u * 98;
    dd[unit_index(L, t, j)] = (uint16_t)(b[0] | (b[1] << 8));
  }
}

hipError_t launch_repack(const Layout &L, const uint8_t *raw, uint8_t *body, uint16_t *d,
                         hipStream_t st) {
  const long n = (long)L.rows * L.units;
  if (n == 0) return hipSuccess;
  const int be = block_elems(L.dtype);
  const int nb = (L.k + be - 1) / be;
  const long raw_row = (long)nb * ggml_block_bytes(L.dtype);
  hipLaunchKernelGGL(k_repack, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, L, raw,
                     raw_row, nb, body, d);
  return hipGetLastError();
}

// ----------------------------------------------------------------- dequant
// Element e (0..255) of a unit whose logical bytes are read through `lb`.
template <typename LB>
__device__ float dq_element(int dtype, bool quad, const LB &lb, uint32_t dbits, int e,
                           const uint32_t *grid) {
  if (dtype == T_Q8_0) {
    const int b = e >> 5;
    const float scale = h2f(lb(256 + 2 * b) | (lb(257 + 2 * b) << 8));
    return scale * (float)(int8_t)lb(e);
  }
  if (dtype == T_Q4_K || dtype == T_Q5_K) {
    const float d = h2f(lb(0) | (lb(1) << 8)), dmin = h2f(lb(2) | (lb(3) << 8));
    uint32_t sw[3];
    for (int w = 0; w < 3; w++)
      sw[w] = lb(4 + 4 * w) | (lb(5 + 4 * w) << 8) | (lb(6 + 4 * w) << 16) |
              ((uint32_t)lb(7 + 4 * w) << 24);
    const int j = e / 64, w = e % 64, l = w % 32;
    const int is = 2 * j + (w >= 32);
    uint32_t sc, m;
    scale_min_k4(is, sw[0], sw[1], sw[2], sc, m);
    const int qs = (dtype == T_Q5_K ? 48 : 16) + 32 * j;
    uint32_t q = w < 32 ? (lb(qs + l) & 0xF) : (lb(qs + l) >> 4);
    if (dtype == T_Q5_K) q += ((lb(16 + l) >> is) & 1u) << 4;
    const float dl = d * (float)sc;
    const float ml = dmin * (float)m;
    return dl * (float)q - ml;
  }
  if (dtype == T_Q6_K) {
    const float d = h2f(dbits);
    const int h = e / 128, t = (e % 128) / 32, l = e % 32;
    const int lo = (t & 1) ? lb(64 * h + l + 32) : lb(64 * h + l);
    const int nib = (t & 2) ? (lo >> 4) : (lo & 0xF);
    const int q = (nib | (((lb(128 + 32 * h + l) >> (2 * t)) & 3) << 4)) - 32;
    const int sc = (int)(int8_t)lb(192 + 8 * h + l / 16 + 2 * t);
    return d * (float)sc * (float)q;
  }
  const float d = h2f(dbits);
  const int ib = e / 32, l = (e % 32) / 8, j = e % 8;
  if (quad) {  // re-encoded sub-blocks (iq3q_pack)
    auto word = [&](int i) {
      const int o = 12 * ib + 4 * i;
      return lb(o) | (lb(o + 1) << 8) | (lb(o + 2) << 16) | ((uint32_t)lb(o + 3) << 24);
    };
    const uint32_t w0 = word(0), w1 = word(1), w2 = word(2);
    const uint64_t lo = (uint64_t)w1 << 32 | w0;
    const uint32_t g = l == 0 ? w0 & 0x7FFFFFu : l == 1 ? (uint32_t)(lo >> 23) & 0x7FFFFFu
                     : l == 2 ? (uint32_t)((((uint64_t)w2 << 32 | w1) >> 14)) & 0x7FFFFFu
                              : (w2 >> 5) & 0x7FFFFFu;
    uint32_t e1, e2, sg;
    iq3q_unpack(g, e1, e2, sg);
    const float db = d * (0.5f + (float)(w2 >> 28)) * 0.5f;
    const uint32_t gv = grid[j < 4 ? e1 : e2];
    const float mag = (float)((gv >> (8 * (j & 3))) & 0xff);
    return db * mag * (((sg >> j) & 1u) ? -1.0f : 1.0f);
  }
  // IQ3_XXS, wave-tiled: logical bytes are ggml bytes 2..97
  const uint32_t aux = lb(64 + 4 * ib) | (lb(65 + 4 * ib) << 8) | (lb(66 + 4 * ib) << 16) |
                       ((uint32_t)lb(67 + 4 * ib) << 24);
  const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
  const uint32_t sg = ksign7((aux >> (7 * l)) & 127u);
  const uint32_t g = grid[lb(8 * ib + 2 * l + (j >> 2))];
  const float mag = (float)((g >> (8 * (j & 3))) & 0xff);
  return db * mag * (((sg >> j) & 1u) ? -1.0f : 1.0f);
}

__global__ void k_dequant(Layout L, const uint8_t *body, const uint16_t *dd,
                          const uint32_t *grid, int row0, long total, float *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int r = row0 + (int)(i / L.k);
  const int c = (int)(i % L.k);
  const int t = r / L.rt, j = (r % L.rt) * L.units + c / 256;
  auto lb = [&](int o) -> uint32_t { return body[chunk_offset(L, t, j, o >> 4) + (o & 15)]; };
  const uint32_t dbits = dd ? dd[unit_index(L, t, j)] : 0u;
  out[i] = dq_element(L.dtype, L.quad, lb, dbits, c % 256, grid);
}

hipError_t launch_dequant(const gq_weight *w, const uint32_t *grid, int row0, int nrows,
                          float *out, hipStream_t st) {
  const long total = (long)nrows * w->L.k;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, w->L,
                     (const uint8_t *)w->body, (const uint16_t *)w->d, grid, row0, total, out);
  return hipGetLastError();
}

// ------------------------------------------------------ per-32 Q8 pack
// KvDtype::Q8_0::pack (src/model/mod.rs:574-583): amax over 32 elements,
// scale = amax / 127 (1.0 if amax == 0), stored as f16 (round to nearest
// even); q = clamp(round(x / scale), -127, 127) with the f32 scale.
// One 32-lane half-wave per block of 32.
__global__ void k_quantize_q8_32(const float *x, long nblk, uint16_t *scale, int8_t *q) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long b = gid >> 5;
  const int l = threadIdx.x & 31;
  const float v = b < nblk ? x[b * 32 + l] : 0.f;
  float amax = fabsf(v);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
  if (b >= nblk) return;
  const float s = amax > 0.f ? amax / 127.0f : 1.0f;
  if (l == 0) scale[b] = __half_as_ushort(__float2half_rn(s));
  float r = roundf(v / s);
  r = fminf(fmaxf(r, -127.f), 127.f);
  q[b * 32 + l] = (int8_t)r;
}

hipError_t launch_quantize_q8_32(const float *x, long n, uint16_t *scale, int8_t *q,
                                 hipStream_t st) {
  const long nblk = n / 32;
  if (nblk == 0) return hipSuccess;
  const long threads = nblk * 32;
  hipLaunchKernelGGL(k_quantize_q8_32, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     x, nblk, scale, q);
  return hipGetLastError();
}

// ------------------------------------------------------ Q8_K quantizer
// quantize_row_q8_k (src/quant/q8_k.rs:49-91) of x[n]: 16 lanes per
// 256-element block (16 elements each, zero past n), q8k_quant16 per block;
// qs [nb*256] (zero padded), d [nb], bsums [nb*16].
__global__ __launch_bounds__(256) void k_quantize_row_q8k(const float *x, long n, long nb, float *d,
                                                          int8_t *qs, int16_t *bsums) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long b = gid >> 4;
  const int g = (int)(gid & 15);
  const long e0 = b * 256 + 16 * g;
  float xv[16];
#pragma unroll
  for (int i = 0; i < 16; i++) xv[i] = (b < nb && e0 + i < n) ? x[e0 + i] : 0.f;
  const Q8K16 r = q8k_quant16(xv, 16 * g);
  if (b >= nb) return;
  *(uint4 *)(qs + e0) = make_uint4(r.q[0], r.q[1], r.q[2], r.q[3]);
  bsums[b * 16 + g] = (int16_t)r.bsum;
  if (g == 0) d[b] = r.d;
}

hipError_t launch_quantize_row_q8k(const float *x, long n, float *d, int8_t *qs, int16_t *bsums,
                                   hipStream_t st) {
  const long nb = (n + 255) / 256;
  if (nb == 0) return hipSuccess;
  hipLaunchKernelGGL(k_quantize_row_q8k, dim3((unsigned)((nb * 16 + 255) / 256)), dim3(256), 0, st,
                     x, n, nb, d, qs, bsums);
  return hipGetLastError();
}

}  // namespace gq
