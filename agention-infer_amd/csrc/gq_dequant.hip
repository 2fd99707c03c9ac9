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
// One thread per (row, block): split the ggml block into the body and the
// separate f16 scale array (Q6_K, Q8_0, IQ3_XXS); plain copy otherwise.
__global__ void k_repack(int dtype, const uint8_t *raw, long nblocks, uint8_t *body,
                         uint16_t *dd) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblocks) return;
  const int gb = ggml_block_bytes(dtype), bb = body_block_bytes(dtype);
  const uint8_t *src = raw + i * gb;
  uint8_t *dst = body + i * bb;
  int off = 0;
  if (dtype == T_Q6_K) {
    dd[i] = (uint16_t)(src[208] | (src[209] << 8));
  } else if (dtype == T_Q8_0 || dtype == T_IQ3_XXS) {
    dd[i] = (uint16_t)(src[0] | (src[1] << 8));
    off = 2;
  }
  for (int k = 0; k < bb; k++) dst[k] = src[off + k];
}

hipError_t launch_repack(int dtype, const uint8_t *raw, long rows, int nb, uint8_t *body,
                         uint16_t *d, hipStream_t st) {
  const long n = rows * nb;
  if (n == 0) return hipSuccess;
  const long blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_repack, dim3((unsigned)blocks), dim3(256), 0, st, dtype, raw, n, body, d);
  return hipGetLastError();
}

// ----------------------------------------------------------------- dequant
__device__ float dq_element(int dtype, const uint8_t *bp, const uint16_t *dp, int e,
                            const uint32_t *grid) {
  if (dtype == T_Q8_0) {
    const float scale = h2f(*dp);
    return scale * (float)(int8_t)bp[e];
  }
  if (dtype == T_Q4_K || dtype == T_Q5_K) {
    const float d = h2f(bp[0] | (bp[1] << 8)), dmin = h2f(bp[2] | (bp[3] << 8));
    const uint32_t s0 = bp[4] | (bp[5] << 8) | (bp[6] << 16) | ((uint32_t)bp[7] << 24);
    const uint32_t s1 = bp[8] | (bp[9] << 8) | (bp[10] << 16) | ((uint32_t)bp[11] << 24);
    const uint32_t s2 = bp[12] | (bp[13] << 8) | (bp[14] << 16) | ((uint32_t)bp[15] << 24);
    const int j = e / 64, w = e % 64, l = w % 32;
    const int is = 2 * j + (w >= 32);
    uint32_t sc, m;
    scale_min_k4(is, s0, s1, s2, sc, m);
    const uint8_t *qs = bp + (dtype == T_Q5_K ? 48 : 16) + 32 * j;
    uint32_t q = w < 32 ? (qs[l] & 0xF) : (qs[l] >> 4);
    if (dtype == T_Q5_K) q += ((bp[16 + l] >> is) & 1u) << 4;
    const float dl = d * (float)sc;
    const float ml = dmin * (float)m;
    return dl * (float)q - ml;
  }
  if (dtype == T_Q6_K) {
    const float d = h2f(*dp);
    const int h = e / 128, t = (e % 128) / 32, l = e % 32;
    const uint8_t *ql = bp + 64 * h, *qh = bp + 128 + 32 * h;
    const int8_t *sc = (const int8_t *)(bp + 192);
    const int lo = (t & 1) ? ql[l + 32] : ql[l];
    const int nib = (t & 2) ? (lo >> 4) : (lo & 0xF);
    const int q = (nib | (((qh[l] >> (2 * t)) & 3) << 4)) - 32;
    return d * (float)sc[8 * h + l / 16 + 2 * t] * (float)q;
  }
  // IQ3_XXS
  const float d = h2f(*dp);
  const int ib = e / 32, l = (e % 32) / 8, j = e % 8;
  const uint8_t *aux8 = bp + 64 + 4 * ib;
  const uint32_t aux = aux8[0] | (aux8[1] << 8) | (aux8[2] << 16) | ((uint32_t)aux8[3] << 24);
  const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
  const uint32_t sg = ksign7((aux >> (7 * l)) & 127u);
  const uint32_t g = grid[bp[8 * ib + 2 * l + (j >> 2)]];
  const float mag = (float)((g >> (8 * (j & 3))) & 0xff);
  return db * mag * (((sg >> j) & 1u) ? -1.0f : 1.0f);
}

__global__ void k_dequant(gq_weight w, const uint32_t *grid, int row0, long total, float *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int r = row0 + (int)(i / w.in_dim);
  const int c = (int)(i % w.in_dim);
  const int be = block_elems(w.dtype), bb = body_block_bytes(w.dtype);
  const int b = c / be;
  const uint8_t *bp = w.body + (long)r * w.stride + (long)b * bb;
  const uint16_t *dp = w.d ? w.d + (long)r * w.nb + b : nullptr;
  out[i] = dq_element(w.dtype, bp, dp, c % be, grid);
}

hipError_t launch_dequant(const gq_weight *w, const uint32_t *grid, int row0, int nrows,
                          float *out, hipStream_t st) {
  const long total = (long)nrows * w->in_dim;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, *w,
                     grid, row0, total, out);
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

}  // namespace gq
