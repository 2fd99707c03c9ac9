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
// Tiling (bf16): a block computes 80 weight rows x 512 tokens when the
// batch is longer than 256 tokens (18944 rows x 512 tokens -> 237 blocks:
// one round on 256 CUs, every weight element dequantized once), else 160
// rows x 256 tokens.  K advances 64 elements (one Q4_K group) per stage.
// int8: 160 rows x 128 tokens.
#include <type_traits>

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
// X fp32 [n][k] -> bf16 in MFMA B-operand fragments: fragment (token tile
// nt, k-step ks) of 16 tokens x 32 k is 64 lane slots of 8 bf16 (lane l:
// token 16nt + l%16, k 32ks + 8(l/16)), fragments ordered [nt][ks], so the
// GEMM loads each one as 1 KiB of contiguous memory.  Tokens are padded
// with zeros to npad, k to kpad.  One thread per slot.
__global__ void k_x_to_bf16_frag(const float *X, int n, int npad, int k, int kpad, uint16_t *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;  // slot
  const int ksteps = kpad / 32;
  if (i >= (long)(npad / 16) * ksteps * 64) return;
  const int l = (int)(i & 63);
  const long f = i >> 6;
  const int nt = (int)(f / ksteps), ks = (int)(f % ksteps);
  const int t = 16 * nt + (l & 15), c0 = 32 * ks + 8 * (l >> 4);
  uint32_t o[4];
  if ((k & 7) == 0) {  // the 8 values are one aligned 32-byte run (or all padding)
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (t < n && c0 < k) {
      a = *(const float4 *)(X + (long)t * k + c0);
      b = *(const float4 *)(X + (long)t * k + c0 + 4);
    }
    o[0] = f2bf(a.x) | (f2bf(a.y) << 16);
    o[1] = f2bf(a.z) | (f2bf(a.w) << 16);
    o[2] = f2bf(b.x) | (f2bf(b.y) << 16);
    o[3] = f2bf(b.z) | (f2bf(b.w) << 16);
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int c = c0 + 2 * e;
      const float a = t < n && c < k ? X[(long)t * k + c] : 0.f;
      const float b = t < n && c + 1 < k ? X[(long)t * k + c + 1] : 0.f;
      o[e] = f2bf(a) | (f2bf(b) << 16);
    }
  }
  *(uint4 *)(out + 8 * i) = make_uint4(o[0], o[1], o[2], o[3]);
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
// Producer / consumer: 512 threads.  Waves 0-3 only multiply: each owns an
// 80-row x 128-token tile (5 x 8 MFMA tiles) of the 160 x 256 block tile.
// Waves 4-7 only move and dequantize data, straight from memory to LDS
// (global_load_lds_dwordx4, no registers):
//   * waves 4-5 fetch the raw Q4_K units of the block's 160 rows (ggml
//     order, 144 B per row per 256 k), one unit (4 stages of 64 k) ahead;
//   * all four fetch the X tile (256 tokens x 64 bf16) one stage ahead and
//     dequantize the next stage's W tile (d*sc*q - dmin*m, bf16).
// LDS tiles are fragment-major: MFMA operand (ks, t) -- 16 rows or tokens x
// 32 k -- is 64 lane slots of 16 B (lane l: row / token 16t + l%16, k
// 32ks + 8(l/16) .. +8), so every operand read is a conflict-free 128-bit
// load of consecutive slots and every X load writes a whole fragment.
// Rings (2 slots each): dequantized W, X, raw W units (152 KiB).  One
// barrier per stage.  A wave's waits count only its own loads (in issue
// order), so the long-lived unit loads are issued after each stage's X
// loads and only waves 4-5 carry them.
constexpr int AT = BM / 16, BT = BN / 16;     // 10 row tiles, 16 token tiles
constexpr int A_FR = 2 * AT, B_FR = 2 * BT;   // fragments per stage
constexpr int FR16 = 512;                     // bf16 per 1 KiB fragment

typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt vmcnt(N), leaving the other counters alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

__device__ __forceinline__ void dma16(const void *g, void *lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t *)lds, 16, 0, 0);
}

// LDS reads written as asm and waited for inside: the compiler, seeing
// loads straight to LDS still outstanding, would otherwise wait for all of
// them (vmcnt(0)) before any LDS read; the callers wait for exactly the
// loads they read.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void lds_read2(const uint4 *p0, const uint4 *p1, uint4 &a, uint4 &b) {
  const uint32_t a0 = (uint32_t)(uintptr_t)(lds_void_t *)p0;
  const uint32_t a1 = (uint32_t)(uintptr_t)(lds_void_t *)p1;
  u32x4_t x, y;
  asm volatile(
      "ds_read_b128 %0, %2\n\t"
      "ds_read_b128 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x), "=&v"(y)
      : "v"(a0), "v"(a1)
      : "memory");
  a = make_uint4(x[0], x[1], x[2], x[3]);
  b = make_uint4(y[0], y[1], y[2], y[3]);
}

// Two / four 16-byte LDS reads, one wait.
__device__ __forceinline__ void lds_read2_a(const uint32_t (&ad)[2], uint4 (&v)[2]) {
  u32x4_t x0, x1;
  asm volatile(
      "ds_read_b128 %0, %2\n\t"
      "ds_read_b128 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x0), "=&v"(x1)
      : "v"(ad[0]), "v"(ad[1])
      : "memory");
  v[0] = make_uint4(x0[0], x0[1], x0[2], x0[3]);
  v[1] = make_uint4(x1[0], x1[1], x1[2], x1[3]);
}
__device__ __forceinline__ void lds_read4(const uint32_t (&ad)[4], uint4 (&v)[4]) {
  u32x4_t x0, x1, x2, x3;
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %5\n\t"
      "ds_read_b128 %2, %6\n\t"
      "ds_read_b128 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
      : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3])
      : "memory");
  v[0] = make_uint4(x0[0], x0[1], x0[2], x0[3]);
  v[1] = make_uint4(x1[0], x1[1], x1[2], x1[3]);
  v[2] = make_uint4(x2[0], x2[1], x2[2], x2[3]);
  v[3] = make_uint4(x3[0], x3[1], x3[2], x3[3]);
}

// Six 16-byte LDS reads, one wait.
__device__ __forceinline__ void lds_read6(const uint32_t (&ad)[6], uint4 (&v)[6]) {
  u32x4_t x0, x1, x2, x3, x4, x5;
  asm volatile(
      "ds_read_b128 %0, %6\n\t"
      "ds_read_b128 %1, %7\n\t"
      "ds_read_b128 %2, %8\n\t"
      "ds_read_b128 %3, %9\n\t"
      "ds_read_b128 %4, %10\n\t"
      "ds_read_b128 %5, %11\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3), "=&v"(x4), "=&v"(x5)
      : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5])
      : "memory");
  v[0] = make_uint4(x0[0], x0[1], x0[2], x0[3]);
  v[1] = make_uint4(x1[0], x1[1], x1[2], x1[3]);
  v[2] = make_uint4(x2[0], x2[1], x2[2], x2[3]);
  v[3] = make_uint4(x3[0], x3[1], x3[2], x3[3]);
  v[4] = make_uint4(x4[0], x4[1], x4[2], x4[3]);
  v[5] = make_uint4(x5[0], x5[1], x5[2], x5[3]);
}

// Byte K of w (0..255) as float: one v_cvt_f32_ubyteK.  Written as asm
// because the compiler otherwise folds a preceding nibble mask into a
// v_bfe per element.
template <int K>
__device__ __forceinline__ float cvt_ubyte(uint32_t w) {
  float f;
  if constexpr (K == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(w));
  else if constexpr (K == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(w));
  else if constexpr (K == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(w));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(w));
  return f;
}

// get_scale_min_k4 (src/quant/q4_k.rs:26-35) without branches: both forms,
// then a select on j < 4.
__device__ __forceinline__ void scale_min_k4_sel(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                                 uint32_t &sc, uint32_t &m) {
  const uint32_t a = sbyte(s0, s1, s2, j & 7), b = sbyte(s0, s1, s2, j + 4);
  const uint32_t c = sbyte(s0, s1, s2, (j - 4) & 7);
  const uint32_t lo_sc = a & 63u, lo_m = b & 63u;
  const uint32_t hi_sc = (b & 0xFu) | ((c >> 6) << 4), hi_m = (b >> 4) | ((a >> 6) << 4);
  sc = j < 4 ? lo_sc : hi_sc;
  m = j < 4 ? lo_m : hi_m;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const bf16x2_t v = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32: round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

// Raw (ggml-order) Q4_K bytes for the GEMM: a row's 144-byte units are
// contiguous, so a producer fetches whole units (2.25 cache lines) instead
// of the scattered 16-byte chunks of the tiled matvec layout.
constexpr int UB = 144;                        // bytes per Q4_K unit
constexpr int WU_SLOT = 24 * 1024;             // one unit of BM rows (23040 B) + pad
constexpr int W_INSTR = WU_SLOT / 1024;        // 24 loads of 64 x 16 B per unit

// ----------------------------------------------------------- bf16 kernel, ring pipeline
// Block tile TBM rows x TBN tokens, 4 multiply waves of 80 x 128 (as in
// k_gemm_bf16: fragment-major LDS operands) and 4 producer waves, with a
// deeper pipeline than k_gemm_bf16:
//   * W is fetched per stage, only the bytes the stage needs (the unit's
//     16-byte header and the group's 32 quant bytes per row), two stages
//     ahead, into a ring private to each producer wave: producer wave p
//     fetches and dequantizes rows TBM/4 * p .. + TBM/4 itself, so it waits
//     only for its own loads and no W bytes cross waves;
//   * X fragments go through an NXR-slot ring, fetched NXR - 1 stages ahead;
//   * the multiply waves only multiply.
// With TBN = 512 (80 x 512 tiles) a block covers all tokens of a 512-token
// batch, so every weight element is dequantized once per call.
// Iteration kt: multiply waves run stage kt; producer waves issue the loads
// of stage kt + NXR - 1 (X) and kt + 2 (W), wait for W of stage kt + 1,
// dequantize it, and (NXR = 2) wait for X of stage kt + 1.  One barrier per
// iteration.  Blocks are numbered so that the token tiles of a row tile are
// 8 apart, i.e. on the same XCD (consecutive blocks go to consecutive
// XCDs): the row tile's W bytes are fetched into one L2.
constexpr int WR = 3;  // W ring slots

template <int TBM, int TBN, int NXR>
struct Ring {
  static constexpr int AT_ = TBM / 16, BT_ = TBN / 16;
  static constexpr int A_FR_ = 2 * AT_, B_FR_ = 2 * BT_;
  static constexpr int PROWS = TBM / 4;        // rows per producer wave
  static constexpr int WSLOTS = 3 * PROWS;     // 16-byte W chunks per producer wave per stage
  static constexpr int WINS = (WSLOTS + 63) / 64;
  static constexpr int XPW = B_FR_ / 4;        // X fragment loads per producer wave per stage
  static constexpr int WGM = TBM / WM;         // multiply waves along the rows
  static_assert(WGM * (TBN / WN) == 4, "4 multiply waves");
  static constexpr int TASKS = 4 * PROWS;      // 16-element dequant tasks per producer wave
  static constexpr int ROUNDS = (TASKS + 63) / 64;
};

template <int TBM, int TBN, int NXR>
__global__ __launch_bounds__(512) void k_gemm_bf16_ring(Layout L, const uint8_t *raw,
                                                        long row_bytes, const uint16_t *Xb, int n,
                                                        int kpad, int mtiles, int ntiles,
                                                        float *Y) {
  using R = Ring<TBM, TBN, NXR>;
  constexpr int AT_ = R::AT_, BT_ = R::BT_, PROWS = R::PROWS, WSLOTS = R::WSLOTS;
  constexpr int WINS = R::WINS, XPW = R::XPW;
  __shared__ __align__(16) uint16_t As[2][R::A_FR_ * FR16];
  __shared__ __align__(16) uint16_t Xs[NXR][R::B_FR_ * FR16];
  __shared__ __align__(16) uint8_t Wg[4][WR][WSLOTS * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // block -> (row tile, token tile): blocks b, b + 8, b + 16, ... of a group
  // of 8 * ntiles share the row tile
  const int b = blockIdx.x, grp = b / (8 * ntiles), rem = b % (8 * ntiles);
  const int mt = 8 * grp + (rem & 7), ntile = rem >> 3;
  if (mt >= mtiles) return;
  const int m0 = mt * TBM, n0 = ntile * TBN;
  const int stages = kpad / BK, last = stages - 1;
  const bool mma = wave < 4;

  if (!mma) {
    const int pw = wave - 4;
    const int ksteps = kpad / 32;
    const uint16_t *xsrc = Xb + ((long)(n0 / 16) * ksteps * 64 + lane) * 8;
    // W chunk slots of this wave: q = 64 i + lane (q < WSLOTS): row
    // PROWS * pw + q / 3, chunk q % 3 (header, quant bytes 0-15, 16-31 of
    // the group).
    const uint8_t *wrow[WINS];
    int wc[WINS];
#pragma unroll
    for (int i = 0; i < WINS; i++) {
      const int q = min(64 * i + lane, WSLOTS - 1);
      const int row = min(m0 + PROWS * pw + q / 3, L.rows - 1);
      wrow[i] = raw + (long)row * row_bytes;
      wc[i] = q % 3;
    }
    auto issue_x = [&](int s) {  // X fragments of stage s (clamped) into slot s % NXR
      const int sc = min(s, last);
#pragma unroll
      for (int qd = 0; qd < XPW; qd++) {
        const int f = XPW * pw + qd, nt = f % BT_, ks = f / BT_;
        dma16(xsrc + ((long)nt * ksteps + 2 * sc + ks) * 512, &Xs[s % NXR][f * FR16]);
      }
    };
    auto issue_w = [&](int s) {  // this wave's W rows of stage s (clamped) into slot s % WR
      const int sc = min(s, last);
      const int u = sc >> 2, j = sc & 3;
#pragma unroll
      for (int i = 0; i < WINS; i++) {
        const int off = wc[i] == 0 ? 0 : 16 + 32 * j + 16 * (wc[i] - 1);
        if (64 * i + lane < WSLOTS) dma16(wrow[i] + (long)u * UB + off, &Wg[pw][s % WR][1024 * i]);
      }
    };
    // Dequantize stage s of this wave's rows: task t = 4 rr + 2 h + qq (row
    // rr, nibble half h, 16-element quarter qq), t = lane + 64 round.
    auto dequant = [&](int s) {
      const int j = s & 3;
      const uint8_t *wg = Wg[pw][s % WR];
      // (asm reads: a plain LDS read would make the compiler wait for every
      // outstanding load straight to LDS, the ones just issued included)
      uint4 hd[3], qs[3];
      uint32_t ad[6];
#pragma unroll
      for (int round = 0; round < 3; round++) {
        const int t = min(lane + 64 * round, R::TASKS - 1);
        const int rr = t >> 2, qq = t & 1;
        ad[2 * round] = (uint32_t)(uintptr_t)(lds_void_t *)(wg + 48 * rr);
        ad[2 * round + 1] = (uint32_t)(uintptr_t)(lds_void_t *)(wg + 48 * rr + 16 + 16 * qq);
      }
      if constexpr (R::ROUNDS == 3) {
        uint4 v6[6];
        lds_read6(ad, v6);
        hd[0] = v6[0]; qs[0] = v6[1]; hd[1] = v6[2]; qs[1] = v6[3]; hd[2] = v6[4]; qs[2] = v6[5];
      } else {
        static_assert(R::ROUNDS == 2, "2 or 3 dequant rounds");
        const uint32_t ad4[4] = {ad[0], ad[1], ad[2], ad[3]};
        uint4 v4[4];
        lds_read4(ad4, v4);
        hd[0] = v4[0]; qs[0] = v4[1]; hd[1] = v4[2]; qs[1] = v4[3];
      }
#pragma unroll
      for (int round = 0; round < R::ROUNDS; round++) {
        const int t = lane + 64 * round;
        if (round < R::ROUNDS - 1 || t < R::TASKS) {
          const int rr = t >> 2, h = (t >> 1) & 1, qq = t & 1;
          const int r = PROWS * pw + rr;
          const bool ok = m0 + r < L.rows;
          uint32_t sc, mn;
          scale_min_k4_sel(2 * j + h, hd[round].y, hd[round].z, hd[round].w, sc, mn);
          const float ds = ok ? h2f(hd[round].x) * (float)sc : 0.f;
          const float nm = ok ? -(h2f(hd[round].x >> 16) * (float)mn) : 0.f;
          const uint32_t qw[4] = {qs[round].x, qs[round].y, qs[round].z, qs[round].w};
          const uint32_t sh = 4u * (uint32_t)h;
          uint32_t o[8];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const uint32_t qv = (qw[i] >> sh) & 0x0F0F0F0Fu;
            o[2 * i] = pack_bf16(fmaf(ds, cvt_ubyte<0>(qv), nm), fmaf(ds, cvt_ubyte<1>(qv), nm));
            o[2 * i + 1] = pack_bf16(fmaf(ds, cvt_ubyte<2>(qv), nm), fmaf(ds, cvt_ubyte<3>(qv), nm));
          }
          uint16_t *dst = &As[s & 1][((h * AT_ + (r >> 4)) * 64 + (r & 15) + 32 * qq) * 8];
          *(uint4 *)dst = make_uint4(o[0], o[1], o[2], o[3]);
          *(uint4 *)(dst + 128) = make_uint4(o[4], o[5], o[6], o[7]);
        }
      }
    };
    if constexpr (NXR == 3) {
      // prologue: stages 0 and 1 in flight, stage 0 dequantized
      issue_x(0);
      issue_w(0);
      issue_x(1);
      issue_w(1);
      wait_vm<XPW + WINS>();
      dequant(0);
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
      for (int kt = 0; kt < stages; kt++) {
        issue_x(kt + 2);
        issue_w(kt + 2);
        wait_vm<XPW + WINS>();  // stage kt + 1 (X and this wave's W rows) in LDS
        if (kt + 1 < stages) dequant(kt + 1);
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
      }
    } else {
      static_assert(NXR == 2, "2 or 3 X slots");
      issue_x(0);
      issue_w(0);
      issue_w(1);
      wait_vm<WINS>();  // X and W of stage 0
      dequant(0);
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
      for (int kt = 0; kt < stages; kt++) {
        issue_x(kt + 1);
        issue_w(kt + 2);
        wait_vm<XPW + WINS>();  // W of stage kt + 1
        if (kt + 1 < stages) dequant(kt + 1);
        wait_vm<WINS>();  // X of stage kt + 1
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
      }
    }
    wait_vm<0>();  // drain the clamped loads before the block ends
    return;
  }

  // ---- multiply waves
  const int wm = wave % R::WGM, wn = wave / R::WGM;
  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int jj = 0; jj < TN; jj++) acc[i][jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  __builtin_amdgcn_s_barrier();  // stage 0 in LDS
  for (int kt = 0; kt < stages; kt++) {
    const uint16_t *A = As[kt & 1], *B = Xs[kt % NXR];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      bf16x8_t a[TM];
#pragma unroll
      for (int i = 0; i < TM; i++)
        a[i] = *(const bf16x8_t *)(A + ((ks * AT_ + TM * wm + i) * 64 + lane) * 8);
#pragma unroll
      for (int jn = 0; jn < TN; jn++) {
        const bf16x8_t bb = *(const bf16x8_t *)(B + ((ks * BT_ + TN * wn + jn) * 64 + lane) * 8);
#pragma unroll
        for (int i = 0; i < TM; i++)
          acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bb, acc[i][jn], 0, 0, 0);
      }
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
  }
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int m = m0 + WM * wm + 16 * i + 4 * (lane >> 4);
#pragma unroll
    for (int jj = 0; jj < TN; jj++) {
      const int t = n0 + WN * wn + 16 * jj + (lane & 15);
      if (t >= n) continue;
      float *yp = Y + (long)t * L.rows + m;
      if (m + 3 < L.rows && (L.rows & 3) == 0) {
        *(float4 *)yp = make_float4(acc[i][jj][0], acc[i][jj][1], acc[i][jj][2], acc[i][jj][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (m + r < L.rows) yp[r] = acc[i][jj][r];
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
  if (mode == GQ_GEMM_BF16) return (size_t)((n + 511) / 512 * 512) * kpad * 2 + 256;
  // int8: q [n][kpad] + scale f32 [n][kpad/32] + qsum int [n][kpad/32]
  return (size_t)n * kpad + (size_t)n * (kpad / 32) * 8 + 512;
}

// ggml-order copy of a Q4_K tiled body: chunk c of unit u of a row holds
// the unit's bytes 16c .. 16c+15.
__global__ void k_unrepack_q4k(Layout L, const uint8_t *body, long row_bytes, uint8_t *raw) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)L.rows * L.units * 9) return;
  const int c = (int)(i % 9);
  const long ru = i / 9;
  const int r = (int)(ru / L.units), u = (int)(ru % L.units);
  const int t = r / L.rt, j = (r % L.rt) * L.units + u;
  *(uint4 *)(raw + (long)r * row_bytes + (long)u * UB + 16 * c) =
      *(const uint4 *)(body + chunk_offset(L, t, j, c));
}

hipError_t launch_unrepack_q4k(const Layout &L, const uint8_t *body, uint8_t *raw, hipStream_t st) {
  const long n = (long)L.rows * L.units * 9;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_unrepack_q4k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, L,
                     body, (long)L.units * UB, raw);
  return hipGetLastError();
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
    const int npad = (n + 511) / 512 * 512;  // a multiple of every token tile
    const long slots = (long)(npad / 16) * (kpad / 32) * 64;
    hipLaunchKernelGGL(k_x_to_bf16_frag, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, st,
                       X, n, npad, L.k, kpad, xb);
    // 80 x 512 tiles when the batch is longer than one 256-token tile (each
    // weight element dequantized once per 512 tokens), else 160 x 256
    const bool wide = n > BN;
    const int tbm = wide ? 80 : BM, tbn = wide ? 512 : BN;
    const int mtiles = (L.rows + tbm - 1) / tbm, ntiles = (n + tbn - 1) / tbn;
    // 8 * ntiles consecutive blocks hold 8 row tiles x all token tiles
    const long nb = (long)((mtiles + 7) / 8) * 8 * ntiles;
    if (nb > 0x7fffffffL) return hipErrorInvalidValue;
    auto kern = wide ? k_gemm_bf16_ring<80, 512, 2> : k_gemm_bf16_ring<160, 256, 3>;
    hipLaunchKernelGGL(kern, dim3((unsigned)nb), dim3(512), 0, st, L, (const uint8_t *)w->gemm_raw,
                       (long)L.units * UB, (const uint16_t *)xb, n, kpad, mtiles, ntiles, Y);
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
