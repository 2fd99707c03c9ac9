// gq_gemm.hip -- batched prefill GEMM Y[n][m] = sum_k W[m][k] X[n][k] for
// Q4_K weights (gfx950 MFMA).
//
// Replaces the prefill contraction of WeightMap::matmul_batch_into
// (src/model/mod.rs:414-464: dequant each row once, dot it with every
// token) and the reference's launch_only_batch / coop batch kernels
// (src/ops/wgpu_backend/resident.rs:76-183), which it does not follow.
//
// Two modes:
//  GQ_GEMM_BF16  Each 64-element group of a W row is dequantized exactly
//                (d*sc*q - dmin*m in fp32, as dequant_q4_k) and rounded to
//                bf16 into LDS; X is converted to bf16 once (round to
//                nearest even) by a prepass.  v_mfma_f32_16x16x32_bf16,
//                fp32 accumulation.
//  GQ_GEMM_INT8  X is packed per 32 elements exactly as KvDtype::Q8_0::pack
//                (src/model/mod.rs:574-583): f16 scale xs, int8 q.  W
//                nibbles (0..15) go to LDS as int8.  Each 32-element
//                sub-block is one v_mfma_i32_16x16x32_i8 (exact integer
//                dot); its result is scaled by (d*sc)*xs and the min term
//                dmin*m*xs*sum(q) is subtracted in fp32.
//
// Tiling: a block computes BM=160 weight rows x BN=256 tokens with 4
// waves (2 x 2, 80 x 128 each = 5 x 8 MFMA tiles of 16 x 16).  18944 rows
// x 512 tokens -> 119 x 2 = 238 blocks: one round on 256 CUs.  K advances
// 64 elements (one Q4_K group) per stage; LDS tiles are double-buffered and
// the next stage's global loads are issued before the current stage's MFMAs.
#include "gq_device.h"
#include "gq_internal.h"
#include "../../include/gq.h"

namespace gq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 160, BN = 256, BK = 64;
constexpr int WM = 80, WN = 128;  // per-wave tile
constexpr int TM = WM / 16, TN = WN / 16;

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// ----------------------------------------------------------- prepasses
// X fp32 [n][k] -> bf16 [n][kpad] (zero padded).
__global__ void k_x_to_bf16(const float *X, int n, int k, int kpad, uint16_t *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)n * kpad;
  if (i >= total) return;
  const int t = (int)(i / kpad), c = (int)(i % kpad);
  out[i] = c < k ? (uint16_t)f2bf(X[(long)t * k + c]) : 0;
}

// X fp32 [n][k] -> per-32 Q8 (KvDtype::Q8_0::pack): q [n][kpad] int8,
// scale [n][kpad/32] f32 (the f16-rounded scale, widened), qsum [n][kpad/32]
// int (sum of the 32 quants).  One 32-lane group per block of 32.
__global__ void k_x_to_q8(const float *X, int n, int k, int kpad, int8_t *q, float *scale,
                          int *qsum) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long b = gid >> 5;
  const long nblk = (long)n * (kpad / 32);
  const int l = threadIdx.x & 31;
  const int t = (int)(b / (kpad / 32)), c = (int)(b % (kpad / 32)) * 32 + l;
  const float v = (b < nblk && c < k) ? X[(long)t * k + c] : 0.f;
  float amax = fabsf(v);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
  const float s = amax > 0.f ? amax / 127.0f : 1.0f;
  float r = roundf(v / s);
  r = fminf(fmaxf(r, -127.f), 127.f);
  int qi = (int)r;
  int sum = qi;
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 32);
  if (b >= nblk) return;
  q[(long)t * kpad + c] = (int8_t)qi;
  if (l == 0) {
    scale[b] = __half2float(__float2half_rn(s));
    qsum[b] = sum;
  }
}

// ----------------------------------------------------------- W loading
struct WRegs {
  uint4 hd, q0, q1;  // header and the 32 qs bytes of group j
  bool ok;
};

__device__ __forceinline__ WRegs load_w(const Layout &L, const uint8_t *body, int r, int u,
                                        int j) {
  WRegs w;
  w.ok = r < L.rows;
  const int rc = w.ok ? r : L.rows - 1;
  const int t = rc / L.rt, jj = (rc % L.rt) * L.units + u;
  w.hd = *(const uint4 *)(body + chunk_offset(L, t, jj, 0));
  w.q0 = *(const uint4 *)(body + chunk_offset(L, t, jj, 1 + 2 * j));
  w.q1 = *(const uint4 *)(body + chunk_offset(L, t, jj, 2 + 2 * j));
  return w;
}

// int8 mode: 64 nibbles as int8 (k order as above), plus per sub-block
// (d*sc, dmin*m) for the two sub-blocks of group j.
__device__ __forceinline__ void store_w_i8(const WRegs &w, int j, uint8_t *dst, float *wsc) {
  const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
  uint32_t lo[8], hi[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    lo[i] = w.ok ? (qw[i] & 0x0F0F0F0Fu) : 0u;
    hi[i] = w.ok ? ((qw[i] >> 4) & 0x0F0F0F0Fu) : 0u;
  }
  *(uint4 *)(dst + 0) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  *(uint4 *)(dst + 16) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
  *(uint4 *)(dst + 32) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  *(uint4 *)(dst + 48) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
  uint32_t sc0, m0, sc1, m1;
  scale_min_k4(2 * j, w.hd.y, w.hd.z, w.hd.w, sc0, m0);
  scale_min_k4(2 * j + 1, w.hd.y, w.hd.z, w.hd.w, sc1, m1);
  const float d = h2f(w.hd.x), dmin = h2f(w.hd.x >> 16);
  wsc[0] = w.ok ? d * (float)sc0 : 0.f;
  wsc[1] = w.ok ? dmin * (float)m0 : 0.f;
  wsc[2] = w.ok ? d * (float)sc1 : 0.f;
  wsc[3] = w.ok ? dmin * (float)m1 : 0.f;
}

// ----------------------------------------------------------- bf16 kernel
// 512 threads = 8 waves as 2 (rows) x 4 (tokens); wave tile 80 x 64.
// Per 64-wide K stage, threads 0..319 each dequantize one 32-element
// sub-block of one row (row t/2, low nibbles for even t, high for odd);
// all 512 threads stage the X tile.  Two waves per SIMD let one wave's
// dequant VALU run beside the other's MFMAs.
constexpr int LDA = BK + 8;  // bf16 elements per LDS row (16 B pad)
constexpr int WN2 = 64, TN2 = WN2 / 16;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const bf16x2_t v = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32: round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

// 32 values of sub-block 2j+hi of a row: (d*sc)*q - dmin*m, as bf16.
__device__ __forceinline__ void dequant_sub_bf16(const WRegs &w, int j, int hi, uint16_t *dst) {
  uint32_t sc, m;
  scale_min_k4(2 * j + hi, w.hd.y, w.hd.z, w.hd.w, sc, m);
  const float d = h2f(w.hd.x), dmin = h2f(w.hd.x >> 16);
  const float ds = d * (float)sc, mm = dmin * (float)m;
  const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
  uint32_t o[16];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t q = hi ? (qw[i] >> 4) & 0x0F0F0F0Fu : qw[i] & 0x0F0F0F0Fu;
    const float e0 = ds * ub<0>(q) - mm, e1 = ds * ub<1>(q) - mm;
    const float e2 = ds * ub<2>(q) - mm, e3 = ds * ub<3>(q) - mm;
    o[2 * i] = w.ok ? pack_bf16(e0, e1) : 0u;
    o[2 * i + 1] = w.ok ? pack_bf16(e2, e3) : 0u;
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
    *(uint4 *)(dst + 8 * i) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

__global__ __launch_bounds__(512) void k_gemm_bf16(Layout L, const uint8_t *body,
                                                   const uint16_t *Xb, int n, int kpad,
                                                   float *Y) {
  __shared__ __align__(16) uint16_t As[2][BM * LDA];
  __shared__ __align__(16) uint16_t Bs[2][BN * LDA];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  const int stages = kpad / BK;
  const bool wtask = tid < 2 * BM;
  const int wrow = tid >> 1, whi = tid & 1;

  auto load_x = [&](int kt, uint4 (&xr)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = tid + 512 * i, tok = c >> 3, part = c & 7;
      const int tn = min(n0 + tok, n - 1);
      xr[i] = *(const uint4 *)(Xb + (long)tn * kpad + kt * BK + 8 * part);
      if (n0 + tok >= n) xr[i] = make_uint4(0, 0, 0, 0);
    }
  };
  auto store_x = [&](int buf, const uint4 (&xr)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = tid + 512 * i, tok = c >> 3, part = c & 7;
      *(uint4 *)(&Bs[buf][tok * LDA + 8 * part]) = xr[i];
    }
  };

  f32x4_t acc[TM][TN2];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN2; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  WRegs wr;
  uint4 xr[4];
  if (wtask) wr = load_w(L, body, m0 + wrow, 0, 0);
  load_x(0, xr);
  if (wtask) dequant_sub_bf16(wr, 0, whi, &As[0][wrow * LDA + 32 * whi]);
  store_x(0, xr);
  __syncthreads();

  for (int kt = 0; kt < stages; kt++) {
    const int buf = kt & 1;
    // Straight-line stage body (no branch around the next stage's loads and
    // dequant) so the scheduler can interleave the dequant VALU work with
    // this stage's MFMAs; past the last stage it reloads the last stage into
    // the unused buffer.
    const int kn = min(kt + 1, stages - 1);
    if (wtask) wr = load_w(L, body, m0 + wrow, kn >> 2, kn & 3);
    load_x(kn, xr);
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const int kk = 32 * ks + 8 * (lane >> 4);
      bf16x8_t a[TM];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const uint4 v = *(const uint4 *)(&As[buf][(WM * wm + 16 * i + (lane & 15)) * LDA + kk]);
        a[i] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int j = 0; j < TN2; j++) {
        const uint4 v = *(const uint4 *)(&Bs[buf][(WN2 * wn + 16 * j + (lane & 15)) * LDA + kk]);
        const bf16x8_t b = __builtin_bit_cast(bf16x8_t, v);
#pragma unroll
        for (int i = 0; i < TM; i++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b, acc[i][j], 0, 0, 0);
      }
    }
    if (wtask) dequant_sub_bf16(wr, kn & 3, whi, &As[buf ^ 1][wrow * LDA + 32 * whi]);
    store_x(buf ^ 1, xr);
    __syncthreads();
  }

  // D layout: lane holds rows 4*(lane/16)+r (weight rows) of column lane%16 (token).
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int m = m0 + WM * wm + 16 * i + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < TN2; j++) {
      const int t = n0 + WN2 * wn + 16 * j + (lane & 15);
      if (t >= n) continue;
      float *yp = Y + (long)t * L.rows + m;
      if (m + 3 < L.rows && (L.rows & 3) == 0) {
        *(float4 *)yp = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (m + r < L.rows) yp[r] = acc[i][j][r];
      }
    }
  }
}

// ----------------------------------------------------------- int8 kernel
// LDS: W int8 [BM][64+16], X int8 [BN][64+16] (16 B pad); per-row scale
// pairs for the stage's two sub-blocks; per-token (xs, xs*sum(q)) for them.
constexpr int LDQ = BK + 16;
// int8 mode keeps its fp32 accumulators in VGPRs (each sub-block's integer
// result is scaled on the VALU), so its tile is half as wide in tokens.
constexpr int BN8 = 128, WN8 = 64, TN8 = WN8 / 16;

__global__ __launch_bounds__(256) void k_gemm_i8(Layout L, const uint8_t *body, const int8_t *Xq,
                                                 const float *Xs, const int *Xsum, int n,
                                                 int kpad, float *Y) {
  __shared__ __align__(16) uint8_t As[2][BM * LDQ];
  __shared__ __align__(16) uint8_t Bs[2][BN8 * LDQ];
  __shared__ __align__(16) float Ws[2][BM][4];  // d*sc0, dmin*m0, d*sc1, dmin*m1
  __shared__ __align__(16) float Xa[2][BN8][4];  // xs0, xs0*sum0, xs1, xs1*sum1
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN8;
  const int stages = kpad / BK;
  const int nb32 = kpad / 32;

  auto load_x = [&](int kt, uint4 (&xr)[2], float4 &xa) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int c = tid + 256 * i, tok = c >> 2, part = c & 3;
      const int tn = min(n0 + tok, n - 1);
      xr[i] = *(const uint4 *)(Xq + (long)tn * kpad + kt * BK + 16 * part);
      if (n0 + tok >= n) xr[i] = make_uint4(0, 0, 0, 0);
    }
    const int tn = min(n0 + (tid & (BN8 - 1)), n - 1);
    const long bi = (long)tn * nb32 + 2 * kt;
    const float s0 = Xs[bi], s1 = Xs[bi + 1];
    xa = make_float4(s0, s0 * (float)Xsum[bi], s1, s1 * (float)Xsum[bi + 1]);
    if (n0 + (tid & (BN8 - 1)) >= n) xa = make_float4(0.f, 0.f, 0.f, 0.f);
  };
  auto store_x = [&](int buf, const uint4 (&xr)[2], const float4 &xa) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int c = tid + 256 * i, tok = c >> 2, part = c & 3;
      *(uint4 *)(&Bs[buf][tok * LDQ + 16 * part]) = xr[i];
    }
    if (tid < BN8) *(float4 *)(&Xa[buf][tid][0]) = xa;
  };

  f32x4_t acc[TM][TN8];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN8; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  WRegs wr;
  uint4 xr[2];
  float4 xa;
  if (tid < BM) wr = load_w(L, body, m0 + tid, 0, 0);
  load_x(0, xr, xa);
  if (tid < BM) store_w_i8(wr, 0, &As[0][tid * LDQ], &Ws[0][tid][0]);
  store_x(0, xr, xa);
  __syncthreads();

  for (int kt = 0; kt < stages; kt++) {
    const int buf = kt & 1;
    const bool more = kt + 1 < stages;
    if (more) {
      if (tid < BM) wr = load_w(L, body, m0 + tid, (kt + 1) >> 2, (kt + 1) & 3);
      load_x(kt + 1, xr, xa);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {  // one 32-element sub-block per ks
      const int kk = 32 * ks + 8 * (lane >> 4);
      long bfr[TN8];
      float xs[TN8], xm[TN8];
#pragma unroll
      for (int j = 0; j < TN8; j++) {
        const int tok = WN8 * wn + 16 * j + (lane & 15);
        bfr[j] = *(const long *)(&Bs[buf][tok * LDQ + kk]);
        xs[j] = Xa[buf][tok][2 * ks];
        xm[j] = Xa[buf][tok][2 * ks + 1];
      }
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int rb = WM * wm + 16 * i;
        const long afr = *(const long *)(&As[buf][(rb + (lane & 15)) * LDQ + kk]);
        float wsc[4], wmn[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int row = rb + 4 * (lane >> 4) + r;
          wsc[r] = Ws[buf][row][2 * ks];
          wmn[r] = Ws[buf][row][2 * ks + 1];
        }
#pragma unroll
        for (int j = 0; j < TN8; j++) {
          const i32x4_t z = {0, 0, 0, 0};
          const i32x4_t dq = __builtin_amdgcn_mfma_i32_16x16x32_i8(afr, bfr[j], z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float v = fmaf(wsc[r] * xs[j], (float)dq[r], acc[i][j][r]);
            acc[i][j][r] = fmaf(-wmn[r], xm[j], v);
          }
        }
      }
    }
    if (more) {
      if (tid < BM) store_w_i8(wr, (kt + 1) & 3, &As[buf ^ 1][tid * LDQ], &Ws[buf ^ 1][tid][0]);
      store_x(buf ^ 1, xr, xa);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int m = m0 + WM * wm + 16 * i + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < TN8; j++) {
      const int t = n0 + WN8 * wn + 16 * j + (lane & 15);
      if (t >= n) continue;
      float *yp = Y + (long)t * L.rows + m;
      if (m + 3 < L.rows && (L.rows & 3) == 0) {
        *(float4 *)yp = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (m + r < L.rows) yp[r] = acc[i][j][r];
      }
    }
  }
}

// ----------------------------------------------------------- host side
size_t gemm_workspace_bytes(const gq_weight *w, int n, int mode) {
  if (w->L.dtype != T_Q4_K) return (size_t)-1;
  const size_t kpad = (size_t)w->L.units * 256;
  if (mode == GQ_GEMM_BF16) return (size_t)n * kpad * 2 + 256;
  // int8: q [n][kpad] + scale f32 [n][kpad/32] + qsum int [n][kpad/32]
  return (size_t)n * kpad + (size_t)n * (kpad / 32) * 8 + 512;
}

hipError_t launch_gemm(const gq_weight *w, const float *X, int n, float *Y, int mode,
                       void *workspace, size_t ws_bytes, int num_cus, hipStream_t st) {
  (void)ws_bytes;
  (void)num_cus;
  const Layout &L = w->L;
  const int kpad = L.units * 256;
  if (mode == GQ_GEMM_BF16) {
    const dim3 grid((L.rows + BM - 1) / BM, (n + BN - 1) / BN);
    uint16_t *xb = (uint16_t *)workspace;
    const long total = (long)n * kpad;
    hipLaunchKernelGGL(k_x_to_bf16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, X, n,
                       L.k, kpad, xb);
    hipLaunchKernelGGL(k_gemm_bf16, grid, dim3(512), 0, st, L, (const uint8_t *)w->body,
                       (const uint16_t *)xb, n, kpad, Y);
  } else {
    int8_t *xq = (int8_t *)workspace;
    float *xs = (float *)((char *)workspace + (((size_t)n * kpad + 255) & ~(size_t)255));
    int *xsum = (int *)(xs + (size_t)n * (kpad / 32));
    const dim3 grid((L.rows + BM - 1) / BM, (n + BN8 - 1) / BN8);
    const long threads = (long)n * kpad;
    hipLaunchKernelGGL(k_x_to_q8, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, X, n,
                       L.k, kpad, xq, xs, xsum);
    hipLaunchKernelGGL(k_gemm_i8, grid, dim3(256), 0, st, L, (const uint8_t *)w->body,
                       (const int8_t *)xq, (const float *)xs, (const int *)xsum, n, kpad, Y);
  }
  return hipGetLastError();
}

}  // namespace gq
