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
// Tiling (bf16): a block computes 160 weight rows x 256 tokens (18944 rows
// x 512 tokens -> 238 blocks, one round on 256 CUs).  K advances 64
// elements (one Q4_K group) per stage.  Batches longer than 128 tokens take
// the direct-X kernel (X fragments straight from L2 into the multiply
// waves' registers), shorter ones the ring kernel (X through LDS).
// int8 (k_gemm_i8_direct): 160 rows x 256 tokens, W nibbles straight to
// int8 MFMA, per-32 scaling on the VALU.
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

// ----------------------------------------------------------- bf16 GEMM weights
// The bf16 GEMM streams its own copy of a weight, made once: per row, one
// record per 64-element stage (K-step), holding exactly the bytes the
// stage's dequant needs, so that a producer fetches each stage's rows as
// whole 16-byte chunks:
//   Q4_K: the ggml block order itself (144-byte units); a stage reads the
//                unit's 16-byte header (d, dmin, 12 scale bytes; the same
//                bytes for the unit's 4 stages, so 3 of 4 reads hit L2) and
//                the group's 32 quant bytes (byte i holds element i in its
//                low and element 32 + i in its high nibble);
//   Q6_K (64 B): chunk 0 = the 4 int8 scales of the stage's 16-element
//                groups, then d (f16); chunks 1-2 = the low 4 bits of the
//                6-bit codes in the same nibble order as Q4_K; chunk 3 = the
//                high 2 bits, dword g (16-element group g) holding element
//                16 g + i at bits 2i, 2i + 1;
//   Q5_K (64 B): chunk 0 = the unit's 16-byte header (as Q4_K); chunks
//                1-2 = the group's 32 quant bytes (as Q4_K); chunk 3 = the
//                fifth bits, dword 2 h + qq holding element 32 h + 16 qq + i
//                at bit i;
//   Q8_0 (80 B): chunk 0 = the f16 d of the stage's two 32-element blocks;
//                chunks 1-4 = the 64 int8 codes.
template <int FMT> struct GemmFmt;
template <> struct GemmFmt<T_Q4_K> { static constexpr int C = 3; };
template <> struct GemmFmt<T_Q6_K> { static constexpr int C = 4; };
template <> struct GemmFmt<T_Q5_K> { static constexpr int C = 4; };
template <> struct GemmFmt<T_Q8_0> { static constexpr int C = 5; };
// Bytes of the copy per unit (4 stages) of a row.
__host__ __device__ constexpr int gemm_unit_bytes(int fmt) {
  return fmt == T_Q4_K ? 144 : fmt == T_Q8_0 ? 320 : 256;
}
// Offset of chunk c of stage s within a row of the copy.
template <int FMT>
__device__ __forceinline__ long gemm_chunk_off(int s, int c) {
  if constexpr (FMT == T_Q4_K) return (long)(s >> 2) * 144 + (c == 0 ? 0 : 16 + 32 * (s & 3) + 16 * (c - 1));
  else return (long)s * (16 * GemmFmt<FMT>::C) + 16 * c;
}
// The chunk of a stage record holding the quant bytes of dequant task
// (half h, quarter qq).
template <int FMT>
__host__ __device__ constexpr int gemm_qs_chunk(int h, int qq) {
  return FMT == T_Q8_0 ? 1 + 2 * h + qq : 1 + qq;
}

// Record of stage j (0..3) of one unit from the unit's ggml bytes u[] (Q6_K:
// ql 0..127, qh 128..191, scales 192..207, d at 208).
__device__ void q6k_stage_record(const uint8_t *u, int j, uint8_t *rec) {
  for (int i = 0; i < 64; i++) rec[i] = 0;
  for (int g = 0; g < 4; g++) {
    for (int i = 0; i < 16; i++) {
      const int x = 16 * g + i, e = 64 * j + x;  // element of the unit (dequant_q6_k order)
      const int nh = e >> 7, r = e & 127, p = r >> 5, l = r & 31;
      const uint8_t qlb = u[64 * nh + l + 32 * (p & 1)];
      const int lo = (p >> 1) ? qlb >> 4 : qlb & 15;
      const int hi = (u[128 + 32 * nh + l] >> (2 * p)) & 3;
      // low nibble: byte 16 (g & 1) + i of chunks 1-2, nibble g >> 1
      rec[16 + 16 * (g & 1) + i] |= (uint8_t)(lo << (4 * (g >> 1)));
      rec[48 + 4 * g + (i >> 2)] |= (uint8_t)(hi << (2 * (i & 3)));
      if (i == 0) rec[g] = u[192 + 8 * nh + (l >> 4) + 2 * p];
    }
  }
  rec[4] = u[208];
  rec[5] = u[209];
}

// One thread per (row, unit): the unit's part of the GEMM copy, from the
// tiled body.
__global__ void k_gemm_records(Layout L, const uint8_t *body, const uint16_t *dd, uint8_t *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)L.rows * L.units) return;
  const int r = (int)(i / L.units), u = (int)(i % L.units);
  const int t = r / L.rt, j = (r % L.rt) * L.units + u;
  uint8_t *dst = out + ((long)r * L.units + u) * gemm_unit_bytes(L.dtype);
  if (L.dtype == T_Q4_K) {
    for (int c = 0; c < 9; c++)
      *(uint4 *)(dst + 16 * c) = *(const uint4 *)(body + chunk_offset(L, t, j, c));
  } else if (L.dtype == T_Q6_K) {
    uint8_t ub[210];
    for (int c = 0; c < 13; c++) {
      const uint4 v = *(const uint4 *)(body + chunk_offset(L, t, j, c));
      __builtin_memcpy(ub + 16 * c, &v, 16);
    }
    const uint16_t dv = dd[unit_index(L, t, j)];
    ub[208] = (uint8_t)dv;
    ub[209] = (uint8_t)(dv >> 8);
    for (int s = 0; s < 4; s++) {
      uint8_t rb[64];
      q6k_stage_record(ub, s, rb);
      for (int q = 0; q < 4; q++) {
        uint4 v;
        __builtin_memcpy(&v, rb + 16 * q, 16);
        *(uint4 *)(dst + 64 * s + 16 * q) = v;
      }
    }
  } else {
    // Q5_K (the 176 B block) or Q8_0 (8 x 32 codes, then the 8 f16 d)
    const int nc = L.dtype == T_Q5_K ? 11 : 17;
    uint8_t ub[272];
    for (int c = 0; c < nc; c++) {
      const uint4 v = *(const uint4 *)(body + chunk_offset(L, t, j, c));
      __builtin_memcpy(ub + 16 * c, &v, 16);
    }
    for (int s = 0; s < 4; s++) {
      uint8_t rb[80];
      for (int i = 0; i < 80; i++) rb[i] = 0;
      if (L.dtype == T_Q5_K) {
        for (int i = 0; i < 16; i++) rb[i] = ub[i];
        for (int i = 0; i < 32; i++) rb[16 + i] = ub[48 + 32 * s + i];
        for (int h = 0; h < 2; h++)
          for (int l = 0; l < 32; l++)  // element 32 h + l of the stage: qh[l] bit 2 s + h
            rb[48 + 4 * (2 * h + (l >> 4)) + ((l & 15) >> 3)] |=
                (uint8_t)(((ub[16 + l] >> (2 * s + h)) & 1) << (l & 7));
        for (int q = 0; q < 4; q++) {
          uint4 v;
          __builtin_memcpy(&v, rb + 16 * q, 16);
          *(uint4 *)(dst + 64 * s + 16 * q) = v;
        }
      } else {
        for (int i = 0; i < 4; i++) rb[i] = ub[256 + 4 * s + i];  // d of blocks 2 s, 2 s + 1
        for (int i = 0; i < 64; i++) rb[16 + i] = ub[64 * s + i];
        for (int q = 0; q < 5; q++) {
          uint4 v;
          __builtin_memcpy(&v, rb + 16 * q, 16);
          *(uint4 *)(dst + 80 * s + 16 * q) = v;
        }
      }
    }
  }
}

// ----------------------------------------------------------- bf16 kernel, ring pipeline
// Block tile TBM rows x TBN tokens, 512 threads.  Waves 0-3 multiply: each
// owns an 80 x 128 tile (5 x 8 MFMA tiles) and reads fragment-major LDS
// operands (MFMA operand (ks, t), 16 rows or tokens x 32 k, is 64 lane slots
// of 16 B: conflict-free 128-bit reads).  Waves 4-7 produce:
//   * each fetches, two stages ahead, the stage records of its own TBM / 4
//     rows into a ring private to the wave and dequantizes them (Q4_K:
//     d*sc*q - dmin*m; Q6_K: d*sc*(q - 32); both rounded to bf16, RNE) into
//     the next A tile, so it waits only for its own loads;
//   * together they fetch the X fragments (bf16, written by a pre-pass in
//     fragment order) into an NXR-slot ring, NXR - 1 stages ahead.
// Loads go straight to LDS (global_load_lds_dwordx4); a producer's LDS
// reads are inline asm with their own waits (a plain LDS read would make
// the compiler first drain every outstanding load to LDS, the ones just
// issued included).  One barrier per stage.
// Blocks: (row tile, token tile, K split).  A launch covers up to
// GEMM_MAX_SEG matrices sharing the input (row tiles numbered across them);
// with ksplit > 1 a block covers stages [S*s/ksplit, S*(s+1)/ksplit) and
// writes a partial product, which gemm_reduce sums in a fixed order.

// Workgroups are dealt to the 8 XCDs round-robin by id (id % 8).  The
// GEMM's block index is renumbered so that each XCD takes a contiguous range
// of it: the token tiles (and K splits) of one row tile then run on one XCD
// and read its W tile through the same L2.
__device__ __forceinline__ int xcd_block(int id, int n) {
  const int x = id & 7, j = id >> 3, q = n >> 3, r = n & 7;
  return x * q + min(x, r) + j;
}

template <int TBM, int TBN, int NXR, int FMT>
struct Ring {
  static constexpr int AT_ = TBM / 16, BT_ = TBN / 16;
  static constexpr int A_FR_ = 2 * AT_, B_FR_ = 2 * BT_;
  static constexpr int C = GemmFmt<FMT>::C;    // 16-byte chunks per stage record
  static constexpr int PROWS = TBM / 4;        // rows per producer wave
  static constexpr int WSLOTS = C * PROWS;     // W chunks per producer wave per stage
  static constexpr int WINS = (WSLOTS + 63) / 64;
  static constexpr int XPW = B_FR_ / 4;        // X fragment loads per producer wave per stage
  static constexpr int WGM = TBM / WM;         // multiply waves along the rows
  static_assert(WGM * (TBN / WN) == 4, "4 multiply waves");
  static constexpr int TASKS = 4 * PROWS;      // 16-element dequant tasks per producer wave
  static constexpr int ROUNDS = (TASKS + 63) / 64;
  static_assert(ROUNDS == 2 || ROUNDS == 3, "2 or 3 dequant rounds");
  // W ring slots: 2 suffice (stage kt + 2 is fetched into the slot stage kt
  // was dequantized from, one iteration earlier); a third where LDS allows
  // keeps a fetch off the slot read in the iteration just before.
  static constexpr size_t LDS2 = (size_t)2 * A_FR_ * FR16 * 2 + (size_t)NXR * B_FR_ * FR16 * 2 +
                                 (size_t)4 * 2 * WSLOTS * 16;
  static constexpr int WR = LDS2 + (size_t)4 * WSLOTS * 16 <= 163840 ? 3 : 2;
};

template <int TBM, int TBN, int NXR, int FMT>
__global__ __launch_bounds__(512) void k_gemm_bf16_ring(GemmArgs a) {
  using R = Ring<TBM, TBN, NXR, FMT>;
  constexpr int AT_ = R::AT_, BT_ = R::BT_, PROWS = R::PROWS, WSLOTS = R::WSLOTS, C = R::C;
  constexpr int WINS = R::WINS, XPW = R::XPW, WR = R::WR;
  __shared__ __align__(16) uint16_t As[2][R::A_FR_ * FR16];
  __shared__ __align__(16) uint16_t Xs[NXR][R::B_FR_ * FR16];
  __shared__ __align__(16) uint8_t Wg[4][WR][WSLOTS * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = xcd_block(blockIdx.x, gridDim.x), split = b % a.ksplit, rest = b / a.ksplit;
  const int ntile = rest % a.ntiles, tile = rest / a.ntiles;
  GemmSeg sg = a.seg[0];
#pragma unroll
  for (int i = 1; i < GEMM_MAX_SEG; i++)
    if (i < a.nseg && tile >= a.seg[i].tile_begin) sg = a.seg[i];
  const int m0 = (tile - sg.tile_begin) * TBM, n0 = ntile * TBN, rows = sg.rows;
  const int stages_all = a.kpad / BK;
  const int s0 = (int)((long)stages_all * split / a.ksplit);
  const int stages = (int)((long)stages_all * (split + 1) / a.ksplit) - s0, last = stages - 1;
  const long row_stride = (long)(stages_all / 4) * gemm_unit_bytes(FMT);
  const bool mma = wave < 4;

  if (!mma) {
    const int pw = wave - 4;
    const int ksteps = a.kpad / 32;
    const uint16_t *xsrc = a.xb + ((long)(n0 / 16) * ksteps * 64 + lane) * 8;
    // W chunk slots of this wave: q = 64 i + lane (q < WSLOTS): row
    // PROWS * pw + q / C, chunk q % C of the stage record.
    const uint8_t *wsrc[WINS];
    int wc[WINS];
#pragma unroll
    for (int i = 0; i < WINS; i++) {
      const int q = min(64 * i + lane, WSLOTS - 1);
      const int row = min(m0 + PROWS * pw + q / C, rows - 1);
      wsrc[i] = sg.rec + (long)row * row_stride;
      wc[i] = q % C;
    }
    auto issue_x = [&](int s) {  // X fragments of local stage s (clamped) into slot s % NXR
      const int sc = s0 + min(s, last);
#pragma unroll
      for (int qd = 0; qd < XPW; qd++) {
        const int f = XPW * pw + qd, nt = f % BT_, ks = f / BT_;
        dma16(xsrc + ((long)nt * ksteps + 2 * sc + ks) * 512, &Xs[s % NXR][f * FR16]);
      }
    };
    auto issue_w = [&](int s) {  // this wave's rows of local stage s (clamped) into slot s % WR
      const int sg_ = s0 + min(s, last);
#pragma unroll
      for (int i = 0; i < WINS; i++)
        if (64 * i + lane < WSLOTS)
          dma16(wsrc[i] + gemm_chunk_off<FMT>(sg_, wc[i]), &Wg[pw][s % WR][1024 * i]);
    };
    // Dequantize local stage s of this wave's rows: task t = 4 rr + 2 h + qq
    // (row rr, half h of the 64 elements, 16-element quarter qq of the half),
    // t = lane + 64 round.
    auto dequant = [&](int s) {
      const int j = (s0 + s) & 3;  // group of the unit (Q4_K scale pick)
      const uint8_t *wg = Wg[pw][s % WR];
      uint4 hd[3], qs[3], qh[3];
      {
        uint32_t ad[3 * 3];
#pragma unroll
        for (int round = 0; round < 3; round++) {
          const int t = min(lane + 64 * round, R::TASKS - 1);
          const int rr = t >> 2, qq = t & 1;
          ad[3 * round] = (uint32_t)(uintptr_t)(lds_void_t *)(wg + 16 * C * rr);
          ad[3 * round + 1] = (uint32_t)(uintptr_t)(lds_void_t *)(wg + 16 * C * rr + 16 + 16 * qq);
          ad[3 * round + 2] = (uint32_t)(uintptr_t)(lds_void_t *)(wg + 16 * C * rr + 48);
        }
        if constexpr (FMT == T_Q4_K) {
          if constexpr (R::ROUNDS == 3) {
            const uint32_t a6[6] = {ad[0], ad[1], ad[3], ad[4], ad[6], ad[7]};
            uint4 v[6];
            lds_read6(a6, v);
            hd[0] = v[0]; qs[0] = v[1]; hd[1] = v[2]; qs[1] = v[3]; hd[2] = v[4]; qs[2] = v[5];
          } else {
            const uint32_t a4[4] = {ad[0], ad[1], ad[3], ad[4]};
            uint4 v[4];
            lds_read4(a4, v);
            hd[0] = v[0]; qs[0] = v[1]; hd[1] = v[2]; qs[1] = v[3];
          }
        } else {
          if constexpr (R::ROUNDS == 3) {
            const uint32_t a6[6] = {ad[0], ad[1], ad[2], ad[3], ad[4], ad[5]};
            uint4 v[6];
            lds_read6(a6, v);
            hd[0] = v[0]; qs[0] = v[1]; qh[0] = v[2]; hd[1] = v[3]; qs[1] = v[4]; qh[1] = v[5];
            const uint32_t a2[2] = {ad[6], ad[7]};
            uint4 w[2];
            lds_read2_a(a2, w);
            hd[2] = w[0]; qs[2] = w[1];
            const uint32_t a1[2] = {ad[8], ad[8]};
            lds_read2_a(a1, w);
            qh[2] = w[0];
          } else {
            const uint32_t a6[6] = {ad[0], ad[1], ad[2], ad[3], ad[4], ad[5]};
            uint4 v[6];
            lds_read6(a6, v);
            hd[0] = v[0]; qs[0] = v[1]; qh[0] = v[2]; hd[1] = v[3]; qs[1] = v[4]; qh[1] = v[5];
          }
        }
      }
#pragma unroll
      for (int round = 0; round < R::ROUNDS; round++) {
        const int t = lane + 64 * round;
        if (round < R::ROUNDS - 1 || t < R::TASKS) {
          const int rr = t >> 2, h = (t >> 1) & 1, qq = t & 1;
          const int r = PROWS * pw + rr;
          const bool ok = m0 + r < rows;
          const uint32_t qw[4] = {qs[round].x, qs[round].y, qs[round].z, qs[round].w};
          const uint32_t sh = 4u * (uint32_t)h;
          uint32_t o[8];
          if constexpr (FMT == T_Q4_K) {
            uint32_t sc, mn;
            scale_min_k4_sel(2 * j + h, hd[round].y, hd[round].z, hd[round].w, sc, mn);
            const float ds = ok ? h2f(hd[round].x) * (float)sc : 0.f;
            const float nm = ok ? -(h2f(hd[round].x >> 16) * (float)mn) : 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const uint32_t qv = (qw[i] >> sh) & 0x0F0F0F0Fu;
              o[2 * i] = pack_bf16(fmaf(ds, cvt_ubyte<0>(qv), nm), fmaf(ds, cvt_ubyte<1>(qv), nm));
              o[2 * i + 1] = pack_bf16(fmaf(ds, cvt_ubyte<2>(qv), nm), fmaf(ds, cvt_ubyte<3>(qv), nm));
            }
          } else {
            // dequant_q6_k: (d * sc) * (q - 32), one rounding: fma(ds, q, -32 ds)
            const int g = 2 * h + qq;
            const int sc8 = (int)(int8_t)(hd[round].x >> (8 * g));
            const float ds = ok ? h2f(hd[round].y) * (float)sc8 : 0.f;
            const float nm = -32.0f * ds;
            const uint32_t hw = g == 0 ? qh[round].x : g == 1 ? qh[round].y : g == 2 ? qh[round].z : qh[round].w;
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const uint32_t b2 = (hw >> (8 * i)) & 0xFFu;
              const uint32_t hi = (b2 | (b2 << 6) | (b2 << 12) | (b2 << 18)) & 0x03030303u;
              const uint32_t qv = ((qw[i] >> sh) & 0x0F0F0F0Fu) | (hi << 4);
              o[2 * i] = pack_bf16(fmaf(ds, cvt_ubyte<0>(qv), nm), fmaf(ds, cvt_ubyte<1>(qv), nm));
              o[2 * i + 1] = pack_bf16(fmaf(ds, cvt_ubyte<2>(qv), nm), fmaf(ds, cvt_ubyte<3>(qv), nm));
            }
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
      bf16x8_t av[TM];
#pragma unroll
      for (int i = 0; i < TM; i++)
        av[i] = *(const bf16x8_t *)(A + ((ks * AT_ + TM * wm + i) * 64 + lane) * 8);
#pragma unroll
      for (int jn = 0; jn < TN; jn++) {
        const bf16x8_t bb = *(const bf16x8_t *)(B + ((ks * BT_ + TN * wn + jn) * 64 + lane) * 8);
#pragma unroll
        for (int i = 0; i < TM; i++)
          acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bb, acc[i][jn], 0, 0, 0);
      }
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
  }
  // D layout: lane holds rows 4*(lane/16)+r (weight rows) of column lane%16 (token).
  float *Y = a.ksplit > 1 ? sg.part + (long)split * a.n * rows : sg.y;
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int m = m0 + WM * wm + 16 * i + 4 * (lane >> 4);
#pragma unroll
    for (int jj = 0; jj < TN; jj++) {
      const int t = n0 + WN * wn + 16 * jj + (lane & 15);
      if (t >= a.n) continue;
      float *yp = Y + (long)t * rows + m;
      if (m + 3 < rows && (rows & 3) == 0) {
        *(float4 *)yp = make_float4(acc[i][jj][0], acc[i][jj][1], acc[i][jj][2], acc[i][jj][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (m + r < rows) yp[r] = acc[i][jj][r];
      }
    }
  }
}

// ----------------------------------------------------------- bf16 kernel, direct X
// Block tile 160 rows x 256 tokens, 512 threads, K-steps ("stages") of 64.
// Waves 0-3 multiply: wave w owns all 160 rows x tokens 64w .. 64w + 63 of
// the tile, so no X fragment is needed by two waves and X never passes
// through LDS: each multiply wave loads its B fragments (bf16, written in
// fragment order by a pre-pass) from global memory (L2) straight into
// registers, one stage ahead.  The only LDS operand is the dequantized W
// tile (fragment-major, two slots), read once per 4 MFMAs.  Waves 4-7
// produce it as in the ring kernel: each fetches its 40 rows' stage records
// two stages ahead into a ring private to the wave (straight to LDS) and
// dequantizes them to bf16.  One barrier per stage.
// LDS traffic per stage: 20 KiB of A written, 4 x 20 KiB read (the ring
// kernel also moved 2 x 64 KiB of X); load path per stage: 32 KiB of X plus
// the W records.
template <int FMT>
struct Direct {
  static constexpr int TBM = 160, TBN = 256;
  static constexpr int AT_ = TBM / 16;         // row tiles (10)
  static constexpr int A_FR_ = 2 * AT_;        // A fragments per stage
  static constexpr int C = GemmFmt<FMT>::C;
  static constexpr int PROWS = TBM / 4;        // rows per producer wave (40)
  static constexpr int WSLOTS = C * PROWS;
  static constexpr int WINS = (WSLOTS + 63) / 64;
  static constexpr int TASKS = 4 * PROWS;      // 16-element dequant tasks per producer wave
  static constexpr int ROUNDS = (TASKS + 63) / 64;
  static_assert(ROUNDS == 3, "3 dequant rounds");
  static constexpr int WR = 3;
};

template <int FMT>
__global__ __launch_bounds__(512) void k_gemm_bf16_direct(GemmArgs a) {
  using R = Direct<FMT>;
  constexpr int AT_ = R::AT_, PROWS = R::PROWS, WSLOTS = R::WSLOTS, C = R::C;
  constexpr int WINS = R::WINS, WR = R::WR, TBM = R::TBM, TBN = R::TBN;
  __shared__ __align__(16) uint16_t As[2][R::A_FR_ * FR16];
  __shared__ __align__(16) uint8_t Wg[4][WR][WSLOTS * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = xcd_block(blockIdx.x, gridDim.x), split = b % a.ksplit, rest = b / a.ksplit;
  const int ntile = rest % a.ntiles, tile = rest / a.ntiles;
  GemmSeg sg = a.seg[0];
#pragma unroll
  for (int i = 1; i < GEMM_MAX_SEG; i++)
    if (i < a.nseg && tile >= a.seg[i].tile_begin) sg = a.seg[i];
  // pair: tile rows 0-79 are gate rows m0 .. m0 + 79, 80-159 the same up rows
  const bool pair = a.pair != 0;
  const int m0 = (tile - sg.tile_begin) * (pair ? TBM / 2 : TBM), n0 = ntile * TBN, rows = sg.rows;
  const int stages_all = a.kpad / BK;
  const int s0 = (int)((long)stages_all * split / a.ksplit);
  const int stages = (int)((long)stages_all * (split + 1) / a.ksplit) - s0, last = stages - 1;
  const long row_stride = (long)(stages_all / 4) * gemm_unit_bytes(FMT);

  if (wave >= 4) {
    const int pw = wave - 4;
    // matrix row of this wave's tile row PROWS * pw + rr (pair: waves 6-7
    // hold the up rows)
    const int mrow0 = m0 + PROWS * (pair ? (pw & 1) : pw);
    const uint8_t *rec = pair && pw >= 2 ? a.seg[1].rec : sg.rec;
    // W chunk slots of this wave: q = 64 i + lane (q < WSLOTS): row
    // PROWS * pw + q / C, chunk q % C of the stage record.
    const uint8_t *wsrc[WINS];
    int wc[WINS];
#pragma unroll
    for (int i = 0; i < WINS; i++) {
      const int q = min(64 * i + lane, WSLOTS - 1);
      const int row = min(mrow0 + q / C, rows - 1);
      wsrc[i] = rec + (long)row * row_stride;
      wc[i] = q % C;
    }
    auto issue_w = [&](int s) {  // this wave's rows of local stage s (clamped) into slot s % WR
      const int sg_ = s0 + min(s, last);
#pragma unroll
      for (int i = 0; i < WINS; i++)
        if (64 * i + lane < WSLOTS)
          dma16(wsrc[i] + gemm_chunk_off<FMT>(sg_, wc[i]), &Wg[pw][s % WR][1024 * i]);
    };
    // Dequantize local stage s of this wave's rows: task t = 4 rr + 2 h + qq
    // (row rr, half h of the 64 elements, 16-element quarter qq of the half),
    // t = lane + 64 round.
    auto dequant = [&](int s) {
      const int j = (s0 + s) & 3;  // group of the unit (Q4_K scale pick)
      const uint8_t *wg = Wg[pw][s % WR];
      uint4 hd[3], qs[3], qh[3];
      {
        uint32_t ad[3 * 3];
#pragma unroll
        for (int round = 0; round < 3; round++) {
          const int t = min(lane + 64 * round, R::TASKS - 1);
          const int rr = t >> 2, h = (t >> 1) & 1, qq = t & 1;
          ad[3 * round] = (uint32_t)(uintptr_t)(lds_void_t *)(wg + 16 * C * rr);
          ad[3 * round + 1] =
              (uint32_t)(uintptr_t)(lds_void_t *)(wg + 16 * C * rr + 16 * gemm_qs_chunk<FMT>(h, qq));
          ad[3 * round + 2] = (uint32_t)(uintptr_t)(lds_void_t *)(wg + 16 * C * rr + 48);
        }
        if constexpr (FMT == T_Q4_K || FMT == T_Q8_0) {
          const uint32_t a6[6] = {ad[0], ad[1], ad[3], ad[4], ad[6], ad[7]};
          uint4 v[6];
          lds_read6(a6, v);
          hd[0] = v[0]; qs[0] = v[1]; hd[1] = v[2]; qs[1] = v[3]; hd[2] = v[4]; qs[2] = v[5];
        } else {
          const uint32_t a6[6] = {ad[0], ad[1], ad[2], ad[3], ad[4], ad[5]};
          uint4 v[6];
          lds_read6(a6, v);
          hd[0] = v[0]; qs[0] = v[1]; qh[0] = v[2]; hd[1] = v[3]; qs[1] = v[4]; qh[1] = v[5];
          const uint32_t a2[2] = {ad[6], ad[7]};
          uint4 w[2];
          lds_read2_a(a2, w);
          hd[2] = w[0]; qs[2] = w[1];
          const uint32_t a1[2] = {ad[8], ad[8]};
          lds_read2_a(a1, w);
          qh[2] = w[0];
        }
      }
#pragma unroll
      for (int round = 0; round < R::ROUNDS; round++) {
        const int t = lane + 64 * round;
        if (round < R::ROUNDS - 1 || t < R::TASKS) {
          const int rr = t >> 2, h = (t >> 1) & 1, qq = t & 1;
          const int r = PROWS * pw + rr;
          const bool ok = mrow0 + rr < rows;
          const uint32_t qw[4] = {qs[round].x, qs[round].y, qs[round].z, qs[round].w};
          const uint32_t sh = 4u * (uint32_t)h;
          uint32_t o[8];
          if constexpr (FMT == T_Q4_K) {
            uint32_t sc, mn;
            scale_min_k4_sel(2 * j + h, hd[round].y, hd[round].z, hd[round].w, sc, mn);
            const float ds = ok ? h2f(hd[round].x) * (float)sc : 0.f;
            const float nm = ok ? -(h2f(hd[round].x >> 16) * (float)mn) : 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const uint32_t qv = (qw[i] >> sh) & 0x0F0F0F0Fu;
              o[2 * i] = pack_bf16(fmaf(ds, cvt_ubyte<0>(qv), nm), fmaf(ds, cvt_ubyte<1>(qv), nm));
              o[2 * i + 1] = pack_bf16(fmaf(ds, cvt_ubyte<2>(qv), nm), fmaf(ds, cvt_ubyte<3>(qv), nm));
            }
          } else if constexpr (FMT == T_Q5_K) {
            // dequant_q5_k: d * sc * q - dmin * m, q = low nibble | fifth bit << 4
            uint32_t sc, mn;
            scale_min_k4_sel(2 * j + h, hd[round].y, hd[round].z, hd[round].w, sc, mn);
            const float ds = ok ? h2f(hd[round].x) * (float)sc : 0.f;
            const float nm = ok ? -(h2f(hd[round].x >> 16) * (float)mn) : 0.f;
            const int g = 2 * h + qq;
            const uint32_t hw = g == 0 ? qh[round].x : g == 1 ? qh[round].y : g == 2 ? qh[round].z : qh[round].w;
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const uint32_t x4 = (hw >> (4 * i)) & 0xFu;
              const uint32_t hi = (x4 & 1u) | ((x4 & 2u) << 7) | ((x4 & 4u) << 14) | ((x4 & 8u) << 21);
              const uint32_t qv = ((qw[i] >> sh) & 0x0F0F0F0Fu) | (hi << 4);
              o[2 * i] = pack_bf16(fmaf(ds, cvt_ubyte<0>(qv), nm), fmaf(ds, cvt_ubyte<1>(qv), nm));
              o[2 * i + 1] = pack_bf16(fmaf(ds, cvt_ubyte<2>(qv), nm), fmaf(ds, cvt_ubyte<3>(qv), nm));
            }
          } else if constexpr (FMT == T_Q8_0) {
            // dequant_q8_0: d * q, exact in fp32, then bf16
            const float d = ok ? h2f(h ? hd[round].x >> 16 : hd[round].x) : 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const uint32_t w = qw[i];
              o[2 * i] = pack_bf16(d * (float)(int8_t)(w & 0xFFu), d * (float)(int8_t)((w >> 8) & 0xFFu));
              o[2 * i + 1] = pack_bf16(d * (float)(int8_t)((w >> 16) & 0xFFu), d * (float)(int8_t)(w >> 24));
            }
          } else {
            // dequant_q6_k: (d * sc) * (q - 32), one rounding: fma(ds, q, -32 ds)
            const int g = 2 * h + qq;
            const int sc8 = (int)(int8_t)(hd[round].x >> (8 * g));
            const float ds = ok ? h2f(hd[round].y) * (float)sc8 : 0.f;
            const float nm = -32.0f * ds;
            const uint32_t hw = g == 0 ? qh[round].x : g == 1 ? qh[round].y : g == 2 ? qh[round].z : qh[round].w;
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const uint32_t b2 = (hw >> (8 * i)) & 0xFFu;
              const uint32_t hi = (b2 | (b2 << 6) | (b2 << 12) | (b2 << 18)) & 0x03030303u;
              const uint32_t qv = ((qw[i] >> sh) & 0x0F0F0F0Fu) | (hi << 4);
              o[2 * i] = pack_bf16(fmaf(ds, cvt_ubyte<0>(qv), nm), fmaf(ds, cvt_ubyte<1>(qv), nm));
              o[2 * i + 1] = pack_bf16(fmaf(ds, cvt_ubyte<2>(qv), nm), fmaf(ds, cvt_ubyte<3>(qv), nm));
            }
          }
          uint16_t *dst = &As[s & 1][((h * AT_ + (r >> 4)) * 64 + (r & 15) + 32 * qq) * 8];
          *(uint4 *)dst = make_uint4(o[0], o[1], o[2], o[3]);
          *(uint4 *)(dst + 128) = make_uint4(o[4], o[5], o[6], o[7]);
        }
      }
    };
    issue_w(0);
    issue_w(1);
    wait_vm<WINS>();  // W of stage 0
    dequant(0);
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    for (int kt = 0; kt < stages; kt++) {
      issue_w(kt + 2);
      wait_vm<WINS>();  // W of stage kt + 1
      if (kt + 1 < stages) dequant(kt + 1);
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
    }
    wait_vm<0>();  // drain the clamped loads before the block ends
    return;
  }

  // ---- multiply waves: 160 rows x 64 tokens each
  const int ksteps = a.kpad / 32;
  // fragment (token tile 4 * wave + jn of the block, k-step ks):
  // xp + (jn * ksteps + ks) * 512
  const uint16_t *xp = a.xb + ((long)((n0 >> 4) + 4 * wave) * ksteps * 64 + lane) * 8;
  // B fragments of the current stage, per 32-k half; a half is reloaded
  // with the next stage's as soon as its MFMAs are issued (half a stage of
  // lead for the L2 latency, 32 registers).
  bf16x8_t bv[2][4];
  auto load_b = [&](int s, int ks) {
    const int kk = 2 * (s0 + s) + ks;
#pragma unroll
    for (int jn = 0; jn < 4; jn++) bv[ks][jn] = *(const bf16x8_t *)(xp + ((long)jn * ksteps + kk) * 512);
  };
  f32x4_t acc[AT_][4];
#pragma unroll
  for (int i = 0; i < AT_; i++)
#pragma unroll
    for (int jn = 0; jn < 4; jn++) acc[i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  load_b(0, 0);
  load_b(0, 1);
  __builtin_amdgcn_s_barrier();  // stage 0 in LDS
  for (int kt = 0; kt < stages; kt++) {
    const uint16_t *A = As[kt & 1];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      // A fragments one ahead: the read of i + 1 is in flight during the
      // 4 MFMAs of i (the scheduler may not hoist more: registers).
      bf16x8_t av[2];
      av[0] = *(const bf16x8_t *)(A + ((ks * AT_) * 64 + lane) * 8);
#pragma unroll
      for (int i = 0; i < AT_; i++) {
        if (i + 1 < AT_) av[(i + 1) & 1] = *(const bf16x8_t *)(A + ((ks * AT_ + i + 1) * 64 + lane) * 8);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jn = 0; jn < 4; jn++)
          acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i & 1], bv[ks][jn], acc[i][jn], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kt + 1 < stages) load_b(kt + 1, ks);
    }
    __builtin_amdgcn_s_barrier();
  }
  // D layout: lane holds rows 4*(lane/16)+r (weight rows) of column lane%16 (token).
  if (pair) {  // h = silu(g) * u (ffn_gate_up, cpu_path.rs:225-227) as bf16 fragments
    const int hks = a.hkpad / 32;
#pragma unroll
    for (int i = 0; i < AT_ / 2; i++) {
      const int m = m0 + 16 * i + 4 * (lane >> 4);
      if (m >= a.hkpad) continue;
#pragma unroll
      for (int jn = 0; jn < 4; jn++) {
        const int t = n0 + 64 * wave + 16 * jn + (lane & 15);
        float h[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float g = acc[i][jn][r], u = acc[i + AT_ / 2][jn][r];
          h[r] = t < a.n && m + r < rows ? g / (1.0f + expf(-g)) * u : 0.f;
        }
        // columns m .. m + 3 of token t: half of a fragment slot of 8
        uint16_t *dst = a.hb + (((long)(t >> 4) * hks + (m >> 5)) * 64 + (t & 15) + 16 * ((m & 31) >> 3)) * 8 + (m & 7);
        *(uint2 *)dst = make_uint2(f2bf(h[0]) | (f2bf(h[1]) << 16), f2bf(h[2]) | (f2bf(h[3]) << 16));
      }
    }
    return;
  }
  float *Y = a.ksplit > 1 ? sg.part + (long)split * a.n * rows : sg.y;
#pragma unroll
  for (int i = 0; i < AT_; i++) {
    const int m = m0 + 16 * i + 4 * (lane >> 4);
#pragma unroll
    for (int jn = 0; jn < 4; jn++) {
      const int t = n0 + 64 * wave + 16 * jn + (lane & 15);
      if (t >= a.n) continue;
      float *yp = Y + (long)t * rows + m;
      if (m + 3 < rows && (rows & 3) == 0) {
        *(float4 *)yp = make_float4(acc[i][jn][0], acc[i][jn][1], acc[i][jn][2], acc[i][jn][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (m + r < rows) yp[r] = acc[i][jn][r];
      }
    }
  }
}

// y[t][r] = (add ? y[t][r] : 0) + sum_s part[s][t][r], s in order, for the
// segments of one launch at once (segment i owns blocks blk0[i] ..
// blk0[i + 1] - 1: one launch instead of one per matrix).
struct ReduceSegs {
  const float *part[GEMM_MAX_SEG];
  float *y[GEMM_MAX_SEG];
  long count[GEMM_MAX_SEG];
  int blk0[GEMM_MAX_SEG + 1];
  int nseg;
};
__global__ void k_gemm_reduce(ReduceSegs r, int ksplit, int add) {
  int si = 0;
#pragma unroll
  for (int j = 1; j < GEMM_MAX_SEG; j++)
    if (j < r.nseg && (int)blockIdx.x >= r.blk0[j]) si = j;
  const float *part = r.part[si];
  float *y = r.y[si];
  const long count = r.count[si];
  const long i = ((long)(blockIdx.x - r.blk0[si]) * blockDim.x + threadIdx.x) * 4;
  if (i >= count) return;
  if (i + 3 < count) {
    float4 s = add ? *(const float4 *)(y + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < ksplit; k++) {
      const float4 p = *(const float4 *)(part + (long)k * count + i);
      s.x += p.x; s.y += p.y; s.z += p.z; s.w += p.w;
    }
    *(float4 *)(y + i) = s;
  } else {
    for (long e = i; e < count; e++) {
      float s = add ? y[e] : 0.f;
      for (int k = 0; k < ksplit; k++) s += part[(long)k * count + e];
      y[e] = s;
    }
  }
}

// ----------------------------------------------------------- int8 kernel
// X fp32 [n][k] -> per-32 Q8 (KvDtype::Q8_0::pack: amax / 127, f16 scale,
// codes from the f32 scale) in MFMA B-operand fragments for
// v_mfma_i32_16x16x32_i8: fragment (token tile nt, 32-k block kb) is 64
// lane slots of 8 codes (lane l: token 16 nt + l % 16, k 32 kb + 8 (l / 16)),
// 512 B, ordered [nt][kb]; beside it, per (nt, kb), 16 records
// (xs, xs * sum(q)) with xs the f16-rounded scale.  Tokens past n get
// zero records.  One thread per 8 consecutive k of one token; the 4
// threads of a 32-block are consecutive lanes.
__global__ void k_x_to_q8_frag(const float *X, int n, int npad, int k, int kpad, int8_t *q,
                               float2 *xr) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int g8 = kpad / 8;
  const bool ok = i < (long)npad * g8;
  const int t = ok ? (int)(i / g8) : 0, c0 = ok ? (int)(i % g8) * 8 : 0;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = ok && t < n && c0 + e < k ? X[(long)t * k + c0 + e] : 0.f;
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  const float s = amax > 0.f ? amax / 127.0f : 1.0f;
  uint32_t w[2] = {0, 0};
  int sum = 0;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    float r = roundf(v[e] / s);
    r = fminf(fmaxf(r, -127.f), 127.f);
    const int qi = (int)r;
    sum += qi;
    w[e >> 2] |= ((uint32_t)qi & 0xFFu) << (8 * (e & 3));
  }
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  if (!ok) return;
  const int nt = t >> 4, kb = c0 >> 5, sub = (c0 & 31) >> 3;
  const long f = (long)nt * (kpad / 32) + kb;
  *(uint2 *)(q + f * 512 + ((t & 15) + 16 * sub) * 8) = make_uint2(w[0], w[1]);
  if (sub == 0) {
    const float xs = t < n ? __half2float(__float2half_rn(s)) : 0.f;
    xr[f * 16 + (t & 15)] = make_float2(xs, xs * (float)sum);
  }
}

// Block tile 160 rows x 256 tokens, 512 threads = 8 waves, each both
// multiplying and scaling: wave w owns rows 80 (w & 1) .. + 79 and tokens
// 64 (w >> 1) .. + 63 (5 x 4 tiles of 16 x 16), so a SIMD's two waves
// overlap one's scaling VALU with the other's MFMAs.  K-steps ("stages")
// of 64 = one Q4_K group = two 32-element sub-blocks.  Per stage:
//   * every thread fetches one 16-byte chunk of the block's W rows (the
//     group's header or one of its two quant chunks, ggml order) a stage
//     ahead and, after the stage's MFMAs, writes it to LDS: quant bytes as
//     int8 A fragments (low nibbles = sub-block 0, high = sub-block 1; no
//     scaling), the header as (d sc, dmin m) per row and sub-block;
//   * each wave loads its X fragments and (xs, xs sum q) records from
//     global memory (L2) straight into registers, a stage ahead;
//   * per sub-block and tile, one v_mfma_i32_16x16x32_i8 gives the exact
//     integer dot D, and y += (d sc) xs D in fp32 (VALU); the min term
//     - (dmin m) xs sum(q) goes through an fp32 MFMA every two stages.
// One barrier per stage.
constexpr int I8M = 160, I8N = 256;
__global__ __launch_bounds__(512) void k_gemm_i8_direct(const uint8_t *rec, int rows, int ntiles,
                                                        const int8_t *xq, const float2 *xr, int n,
                                                        int kpad, float *Y) {
  __shared__ __align__(16) uint8_t Aq[2][2 * 10 * 512];      // [buf][ks][row tile] fragments
  __shared__ __align__(16) float2 Ws[2][2][I8M];              // [buf][ks][row] (d sc, dmin m)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bid = xcd_block(blockIdx.x, gridDim.x), ntile = bid % ntiles, tile = bid / ntiles;
  const int m0 = tile * I8M, n0 = ntile * I8N;
  const int stages = kpad / 64, kb_all = kpad / 32;
  const long row_stride = (long)(stages / 4) * 144;
  // W chunk of this thread: row wr, chunk wc (0 header, 1-2 quants)
  const bool wact = tid < 3 * I8M;
  const int wr = wact ? tid / 3 : 0, wc = wact ? tid % 3 : 0;
  const bool wok = wact && m0 + wr < rows;
  const uint8_t *wsrc = rec + (long)min(m0 + wr, rows - 1) * row_stride;
  auto load_w = [&](int s) -> uint4 {
    const long off = (long)(s >> 2) * 144 + (wc == 0 ? 0 : 16 + 32 * (s & 3) + 16 * (wc - 1));
    return *(const uint4 *)(wsrc + off);
  };
  auto store_w = [&](int s, int buf, uint4 c) {
    if (!wact) return;
    if (wc == 0) {
      const int j = s & 3;
      uint32_t sc0, mn0, sc1, mn1;
      scale_min_k4(2 * j, c.y, c.z, c.w, sc0, mn0);
      scale_min_k4(2 * j + 1, c.y, c.z, c.w, sc1, mn1);
      const float d = h2f(c.x), dmin = h2f(c.x >> 16);
      Ws[buf][0][wr] = wok ? make_float2(d * (float)sc0, dmin * (float)mn0) : make_float2(0.f, 0.f);
      Ws[buf][1][wr] = wok ? make_float2(d * (float)sc1, dmin * (float)mn1) : make_float2(0.f, 0.f);
    } else {
      // bytes 16 (wc - 1) + b: element 16 (wc - 1) + b (low nibble, sub-block 0)
      // and 32 + 16 (wc - 1) + b (high nibble, sub-block 1); k within the
      // sub-block 16 (wc - 1) + b -> lane slot (row % 16) + 16 * (k / 8)
      const uint32_t qw[4] = {c.x, c.y, c.z, c.w};
      const int rt = wr >> 4, slot0 = (wr & 15) + 32 * (wc - 1);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        uint8_t *fr = &Aq[buf][(h * 10 + rt) * 512];
        const uint32_t l0 = (qw[0] >> (4 * h)) & 0x0F0F0F0Fu, l1 = (qw[1] >> (4 * h)) & 0x0F0F0F0Fu;
        const uint32_t l2 = (qw[2] >> (4 * h)) & 0x0F0F0F0Fu, l3 = (qw[3] >> (4 * h)) & 0x0F0F0F0Fu;
        *(uint2 *)(fr + slot0 * 8) = make_uint2(l0, l1);
        *(uint2 *)(fr + (slot0 + 16) * 8) = make_uint2(l2, l3);
      }
    }
  };
  // X: fragments (token tile 16-token nt, 32-k block kb) at xq + (nt * kb_all + kb) * 512
  const int wm = wave & 1, wn = wave >> 1;
  const long nt0 = (n0 >> 4) + 4 * wn;
  struct XReg {
    long b[2][4];
    float2 r[2][4];
  };
  auto load_x = [&](int s, XReg &x) {
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int jn = 0; jn < 4; jn++) {
        const long f = (nt0 + jn) * kb_all + 2 * s + ks;
        x.b[ks][jn] = *(const long *)(xq + f * 512 + lane * 8);
        x.r[ks][jn] = xr[f * 16 + (lane & 15)];
      }
  };
  f32x4_t acc[5][4];
#pragma unroll
  for (int i = 0; i < 5; i++)
#pragma unroll
    for (int jn = 0; jn < 4; jn++) acc[i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Tiles t = 5 ks + i in a software pipeline: the MFMAs of tile t are
  // issued before the scaling of tile t - 1, so the scaling VALU never
  // waits for the integer results it needs.
  auto compute = [&](int buf, const XReg &x) {
    i32x4_t dq[2][4];
    float ws[2][4];
    auto mf = [&](int t) {
      const int ks = t / 5, rt = 5 * wm + t % 5;
      const long a = *(const long *)&Aq[buf][(ks * 10 + rt) * 512 + lane * 8];
      const float4 w01 = *(const float4 *)&Ws[buf][ks][16 * rt + 4 * (lane >> 4)];
      const float4 w23 = *(const float4 *)&Ws[buf][ks][16 * rt + 4 * (lane >> 4) + 2];
      ws[t & 1][0] = w01.x;
      ws[t & 1][1] = w01.z;
      ws[t & 1][2] = w23.x;
      ws[t & 1][3] = w23.z;
#pragma unroll
      for (int jn = 0; jn < 4; jn++) {
        const i32x4_t z = {0, 0, 0, 0};
        dq[t & 1][jn] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, x.b[ks][jn], z, 0, 0, 0);
      }
    };
    auto scale = [&](int t) {
      const int ks = t / 5, i = t % 5;
#pragma unroll
      for (int jn = 0; jn < 4; jn++) {
        const float xs = x.r[ks][jn].x;
#pragma unroll
        for (int r = 0; r < 4; r++)
          acc[i][jn][r] = fmaf(ws[t & 1][r] * xs, (float)dq[t & 1][jn][r], acc[i][jn][r]);
        // keep the update here (not sunk below later tiles' MFMAs, which
        // would keep every tile's integer result live at once)
        asm volatile("" : "+v"(acc[i][jn]));
      }
    };
    mf(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 1; t < 10; t++) {
      mf(t);
      scale(t - 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    scale(9);
  };
  // prologue: stage 0 to LDS; each stage then loads its X and the next
  // stage's W while it computes
  {
    const uint4 c = load_w(0);
    store_w(0, 0, c);
  }
  __syncthreads();
  // The min term -sum_sb (dmin m)[row][sb] (xs sum q)[token][sb] is a small
  // product over the sub-blocks: every two stages (4 sub-blocks, both W
  // slots of LDS still valid) one v_mfma_f32_16x16x4_f32 per tile adds it,
  // lane l giving row l % 16 of -(dmin m) and token l % 16 of xs sum q for
  // sub-block l / 16 (stages is a multiple of 4: kpad is whole units).
  // The previous stage's LDS slot is being refilled with the next stage's W
  // by other waves during an odd stage, so its (dmin m) values are taken
  // into registers at the even stage.
  const int sbl = lane >> 4;
  float xmp[2][4];  // xs sum q of the previous stage, per (ks, token tile)
  float amp[5];     // -(dmin m) of the previous stage, per row tile (lanes sbl < 2)
  auto mins = [&](int kt, const XReg &x) {
    const int mks = sbl & 1;
    float bq[4];
#pragma unroll
    for (int jn = 0; jn < 4; jn++) {
      const float p0 = mks ? xmp[1][jn] : xmp[0][jn];
      const float c0 = mks ? x.r[1][jn].y : x.r[0][jn].y;
      bq[jn] = sbl < 2 ? p0 : c0;
    }
#pragma unroll
    for (int i = 0; i < 5; i++) {
      const float am = sbl < 2 ? amp[i] : -Ws[kt & 1][mks][16 * (5 * wm + i) + (lane & 15)].y;
#pragma unroll
      for (int jn = 0; jn < 4; jn++)
        acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x4f32(am, bq[jn], acc[i][jn], 0, 0, 0);
    }
  };
  // X of stage kt + 1 is loaded while stage kt computes (two register sets,
  // the loop unrolled by two).
  auto stage = [&](int kt, const XReg &x, XReg &xn) {
    uint4 c = make_uint4(0, 0, 0, 0);
    if (kt + 1 < stages) {
      c = load_w(kt + 1);
      load_x(kt + 1, xn);
    }
    __builtin_amdgcn_sched_barrier(0);
    compute(kt & 1, x);
    if (kt & 1) {
      mins(kt, x);
    } else {
#pragma unroll
      for (int jn = 0; jn < 4; jn++) {
        xmp[0][jn] = x.r[0][jn].y;
        xmp[1][jn] = x.r[1][jn].y;
      }
#pragma unroll
      for (int i = 0; i < 5; i++) amp[i] = -Ws[kt & 1][sbl & 1][16 * (5 * wm + i) + (lane & 15)].y;
    }
    if (kt + 1 < stages) store_w(kt + 1, (kt + 1) & 1, c);
    __syncthreads();
  };
  XReg x0, x1;
  load_x(0, x0);
  for (int kt = 0; kt < stages; kt += 2) {  // stages is even (a multiple of 4)
    stage(kt, x0, x1);
    stage(kt + 1, x1, x0);
  }
  // D layout: lane holds rows 4 (lane / 16) + r of token column lane % 16.
#pragma unroll
  for (int i = 0; i < 5; i++) {
    const int m = m0 + 80 * wm + 16 * i + 4 * (lane >> 4);
#pragma unroll
    for (int jn = 0; jn < 4; jn++) {
      const int t = n0 + 64 * wn + 16 * jn + (lane & 15);
      if (t >= n) continue;
      float *yp = Y + (long)t * rows + m;
      if (m + 3 < rows && (rows & 3) == 0) {
        *(float4 *)yp = make_float4(acc[i][jn][0], acc[i][jn][1], acc[i][jn][2], acc[i][jn][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (m + r < rows) yp[r] = acc[i][jn][r];
      }
    }
  }
}

// ----------------------------------------------------------- int8 kernel, Q6_K
// Q6_K weights against the same per-32 Q8 activation fragments.  A Q6_K
// code minus 32 is an int8 (-32..31), so the A operand is the codes
// themselves.  Its scales change every 16 elements, half a 32-deep MFMA
// step: each step runs twice with the other group's half of A zeroed
// (lanes 0-31 hold k 0..15, lanes 32-63 k 16..31), and the two integer dots
// are combined exactly, sc_a * D_a + sc_b * D_b (|D| <= 16 * 32 * 127),
// before y += (d xs) * that in fp32.
// Block tile 64 rows x 64 tokens, 256 threads; wave w owns rows 16 w ..
// 16 w + 15 and all 64 tokens (4 MFMA tiles).  Per 64-element stage, a
// stage ahead, every operand goes through LDS:
//   * threads 0-127 (row tid / 2, half tid % 2) fetch the stage record's
//     quant chunks of their row and write the half's 32 codes as int8 A
//     fragments; threads 128-191 fetch the row's 4 group scales and d;
//   * every thread fetches 16 bytes of the stage's X fragments (4 KiB) and
//     threads 0-127 its 128 X scales.
// One barrier per stage.
constexpr int Q6M = 64, Q6N = 64, Q6J = Q6N / 16;
__global__ __launch_bounds__(256) void k_gemm_i8_q6k(const uint8_t *rec, int rows, const int8_t *xq,
                                                     const float2 *xr, int n, int kpad, float *Y) {
  __shared__ __align__(16) uint8_t Aq[2][2][4][512];  // [buf][half][row tile][lane slot x 8 codes]
  __shared__ __align__(16) int Sc[2][4][Q6M];         // [buf][group][row] int8 scale
  __shared__ __align__(16) float Dd[2][Q6M];          // [buf][row] f16 d
  __shared__ __align__(16) float Xs[2][2][Q6J][16];   // [buf][half][token tile][token] f16 xs
  __shared__ __align__(16) uint8_t Xb[2][2][Q6J][512];  // [buf][half][token tile] B fragments
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = blockIdx.x * Q6M, n0 = blockIdx.y * Q6N;
  const int stages = kpad / 64, kb_all = kpad / 32;
  const long row_stride = (long)stages * 64;
  // staging role of this thread
  const int sr = tid < 128 ? tid >> 1 : tid - 128, sh = tid & 1;
  const bool sq = tid < 128, ss = tid >= 128 && tid < 192;
  const bool sok = m0 + sr < rows;
  const uint8_t *srow = rec + (long)min(m0 + min(sr, Q6M - 1), rows - 1) * row_stride;
  // the next stage's staged loads: the row's quant chunks (c1, c2, hb) or
  // its scales and d (c0), one X scale (xsv), 16 bytes of X fragments (xf)
  uint4 c1 = make_uint4(0, 0, 0, 0), c2 = c1, c0 = c1, xf = c1;
  uint2 hb = make_uint2(0, 0);
  float xsv = 0.f;
  auto load_w = [&](int s) {
    const uint8_t *rp = srow + (long)s * 64;
    if (sq) {
      c1 = *(const uint4 *)(rp + 16);
      c2 = *(const uint4 *)(rp + 32);
      hb = *(const uint2 *)(rp + 48 + 8 * sh);
    } else if (ss) {
      c0 = *(const uint4 *)rp;
    }
    if (tid < 32 * Q6J) {
      const long f = ((n0 >> 4) + ((tid >> 4) % Q6J)) * kb_all + 2 * s + tid / (16 * Q6J);
      xsv = xr[f * 16 + (tid & 15)].x;
    }
    if (tid < 64 * Q6J) {  // fragment (half, token tile) = tid / 32 (half-major), bytes 16 (tid % 32)
      const int fi = tid >> 5, h = fi / Q6J, jn = fi % Q6J;
      const long f = ((n0 >> 4) + jn) * kb_all + 2 * s + h;
      xf = *(const uint4 *)(xq + f * 512 + 16 * (tid & 31));
    }
  };
  auto store_w = [&](int buf) {
    if (sq) {
      // element e = 16 qq + i of half sh: low 4 bits = nibble sh of byte i
      // of chunk 1 + qq, high 2 bits = bits 2i, 2i + 1 of dword 2 sh + qq
      const uint32_t lw[2][4] = {{c1.x, c1.y, c1.z, c1.w}, {c2.x, c2.y, c2.z, c2.w}};
      const uint32_t hw[2] = {hb.x, hb.y};
      uint8_t *fr = &Aq[buf][sh][sr >> 4][0];
#pragma unroll
      for (int j = 0; j < 4; j++) {  // codes 8 j .. 8 j + 7: lane slot (row % 16) + 16 j
        const int qq = j >> 1;
        uint32_t out[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
          const int i0 = 8 * (j & 1) + 4 * e;  // first of 4 elements within the 16
          const uint32_t lo = (lw[qq][i0 >> 2] >> (4 * sh)) & 0x0F0F0F0Fu;
          const uint32_t b2 = (hw[qq] >> (2 * i0)) & 0xFFu;
          const uint32_t hi = (b2 | (b2 << 6) | (b2 << 12) | (b2 << 18)) & 0x03030303u;
          const uint32_t q6 = lo | (hi << 4);
          out[e] = sok ? (((q6 | 0x80808080u) - 0x20202020u) ^ 0x80808080u) : 0u;  // q - 32
        }
        *(uint2 *)(fr + ((sr & 15) + 16 * j) * 8) = make_uint2(out[0], out[1]);
      }
    } else if (ss) {
#pragma unroll
      for (int g = 0; g < 4; g++) Sc[buf][g][sr] = (int)(int8_t)((c0.x >> (8 * g)) & 0xFFu);
      Dd[buf][sr] = sok ? h2f(c0.y) : 0.f;
    }
    if (tid < 32 * Q6J) Xs[buf][tid / (16 * Q6J)][(tid >> 4) % Q6J][tid & 15] = xsv;
    if (tid < 64 * Q6J) {
      const int fi = tid >> 5;
      *(uint4 *)&Xb[buf][fi / Q6J][fi % Q6J][16 * (tid & 31)] = xf;
    }
  };
  f32x4_t acc[Q6J];
#pragma unroll
  for (int jn = 0; jn < Q6J; jn++) acc[jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int rr0 = 16 * wave + 4 * (lane >> 4);  // this lane's output rows rr0 .. rr0 + 3 (block-local)
  auto compute = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const long a = *(const long *)&Aq[buf][h][wave][lane * 8];
      const long aa = lane < 32 ? a : 0, ab = lane < 32 ? 0 : a;  // groups 2h and 2h + 1
      int sca[4], scb[4];
      float dd[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        sca[r] = Sc[buf][2 * h][rr0 + r];
        scb[r] = Sc[buf][2 * h + 1][rr0 + r];
        dd[r] = Dd[buf][rr0 + r];
      }
#pragma unroll
      for (int jn = 0; jn < Q6J; jn++) {
        const long bx = *(const long *)&Xb[buf][h][jn][lane * 8];
        const i32x4_t z = {0, 0, 0, 0};
        const i32x4_t da = __builtin_amdgcn_mfma_i32_16x16x32_i8(aa, bx, z, 0, 0, 0);
        const i32x4_t db = __builtin_amdgcn_mfma_i32_16x16x32_i8(ab, bx, z, 0, 0, 0);
        const float xs = Xs[buf][h][jn][lane & 15];
#pragma unroll
        for (int r = 0; r < 4; r++)
          acc[jn][r] = fmaf(dd[r] * xs, (float)(sca[r] * da[r] + scb[r] * db[r]), acc[jn][r]);
      }
    }
  };
  load_w(0);
  store_w(0);
  __syncthreads();
  for (int s = 0; s < stages; s++) {
    const bool more = s + 1 < stages;
    if (more) load_w(s + 1);  // a stage ahead
    compute(s & 1);
    if (more) store_w((s & 1) ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int jn = 0; jn < Q6J; jn++) {
    const int t = n0 + 16 * jn + (lane & 15);
    if (t >= n) continue;
#pragma unroll
    for (int r = 0; r < 4; r++)
      if (m0 + rr0 + r < rows) Y[(long)t * rows + m0 + rr0 + r] = acc[jn][r];
  }
}

// ----------------------------------------------------------- host side
size_t gemm_records_bytes(const Layout &L) {
  return (size_t)L.rows * L.units * gemm_unit_bytes(L.dtype);
}

hipError_t launch_gemm_records(const gq_weight *w, uint8_t *out, hipStream_t st) {
  const Layout &L = w->L;
  const long n = (long)L.rows * L.units;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_gemm_records, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, st, L,
                     w->body, w->d, out);
  return hipGetLastError();
}

int gemm_ksplit(int tiles, int stages, int num_cus) {
  // The split with the least time per unit of work, rounds / ks (a block
  // per CU per round; 45 tiles x 6 = 270 blocks would run a second round
  // of 14), the smaller on ties; at most 8, at least 4 stages per split.
  if (tiles >= num_cus) return 1;
  const int kmax = std::max(1, std::min(8, stages / 4));
  int best = 1;
  double best_t = 1.0;
  for (int ks = 2; ks <= kmax; ks++) {
    const double t = (double)((tiles * ks + num_cus - 1) / num_cus) / ks;
    if (t < best_t - 1e-9) {
      best_t = t;
      best = ks;
    }
  }
  return best;
}

namespace {
struct GemmPlan {
  bool direct;
  int tbm, tbn, ntiles, tiles, ksplit;
};
// Kernel choice: the direct-X kernel (160 x 256 tiles, X fragments loaded
// straight into the multiply waves' registers) for batches longer than 128
// tokens; the ring kernel (160 x 256 tiles, X through LDS) for shorter ones.
GemmPlan gemm_plan(const gq_weight *const *ws, int count, int n, int num_cus, bool add) {
  GemmPlan p;
  p.direct = n > 128;
  p.tbm = BM;
  p.tbn = BN;
  p.ntiles = (n + p.tbn - 1) / p.tbn;
  int mt = 0;
  for (int i = 0; i < count; i++) mt += (ws[i]->L.rows + p.tbm - 1) / p.tbm;
  p.tiles = mt * p.ntiles;
  p.ksplit = gemm_ksplit(p.tiles, ws[0]->L.units * 4, num_cus);
  // an accumulating launch adds its product in gemm_reduce
  if (add && p.ksplit == 1) p.ksplit = ws[0]->L.units * 4 >= 2 ? 2 : 1;
  return p;
}
}  // namespace

size_t gemm_part_floats(const gq_weight *const *ws, int count, int n, int num_cus, bool add) {
  const GemmPlan p = gemm_plan(ws, count, n, num_cus, add);
  if (p.ksplit == 1) return 0;
  size_t rows = 0;
  for (int i = 0; i < count; i++) rows += (size_t)ws[i]->L.rows;
  return (size_t)p.ksplit * n * rows;
}

size_t gemm_workspace_bytes(const gq_weight *w, int n, int mode, int num_cus) {
  const size_t kpad = (size_t)w->L.units * 256;
  if (mode == GQ_GEMM_BF16) {
    if (w->L.dtype != T_Q4_K && w->L.dtype != T_Q6_K && w->L.dtype != T_Q5_K && w->L.dtype != T_Q8_0)
      return (size_t)-1;
    const size_t xb = (size_t)((n + GEMM_NPAD - 1) / GEMM_NPAD * GEMM_NPAD) * kpad * 2;
    return ((xb + 255) & ~(size_t)255) + gemm_part_floats(&w, 1, n, num_cus, false) * 4 + 256;
  }
  if (w->L.dtype != T_Q4_K && w->L.dtype != T_Q6_K) return (size_t)-1;
  // int8: fragments [npad/16][kpad/32][512 B] + records [npad/16][kpad/32][16] float2
  const size_t npad = (size_t)(n + I8N - 1) / I8N * I8N;
  return ((npad * kpad + 255) & ~(size_t)255) + npad * (kpad / 32) * 8 + 256;
}

hipError_t launch_x_to_frag(const float *X, int n, int k, uint16_t *xb, hipStream_t st) {
  const int kpad = (k + 255) / 256 * 256;
  const int npad = (n + GEMM_NPAD - 1) / GEMM_NPAD * GEMM_NPAD;
  const long slots = (long)(npad / 16) * (kpad / 32) * 64;
  hipLaunchKernelGGL(k_x_to_bf16_frag, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, st, X,
                     n, npad, k, kpad, xb);
  return hipGetLastError();
}

hipError_t launch_gemm_bf16(const gq_weight *const *ws, float *const *ys, int count,
                            const uint16_t *xb, int n, float *part, bool add, int num_cus,
                            hipStream_t st, int *defer) {
  if (count < 1 || count > GEMM_MAX_SEG || n <= 0) return hipErrorInvalidValue;
  const int fmt = ws[0]->L.dtype;
  const GemmPlan p = gemm_plan(ws, count, n, num_cus, add);
  GemmArgs a{};
  a.nseg = count;
  a.ntiles = p.ntiles;
  a.ksplit = p.ksplit;
  a.n = n;
  a.kpad = ws[0]->L.units * 256;
  a.xb = xb;
  int tb = 0;
  size_t po = 0;
  for (int i = 0; i < count; i++) {
    if (ws[i]->L.dtype != fmt || ws[i]->L.units != ws[0]->L.units || !ws[i]->gemm_raw)
      return hipErrorInvalidValue;
    a.seg[i].rec = ws[i]->gemm_raw;
    a.seg[i].y = ys[i];
    a.seg[i].rows = ws[i]->L.rows;
    a.seg[i].tile_begin = tb;
    a.seg[i].part = p.ksplit > 1 ? part + po : nullptr;
    tb += (ws[i]->L.rows + p.tbm - 1) / p.tbm;
    po += (size_t)p.ksplit * n * ws[i]->L.rows;
  }
  if (p.ksplit > 1 && !part) return hipErrorInvalidValue;
  const long nb = (long)tb * p.ntiles * p.ksplit;
  if (nb > 0x7fffffffL) return hipErrorInvalidValue;
  void (*kern)(GemmArgs);
  // Q5_K and Q8_0 run the direct kernel at every batch size (the ring
  // kernel's LDS has no room for Q8_0's five-chunk records)
  if (fmt == T_Q5_K) kern = k_gemm_bf16_direct<T_Q5_K>;
  else if (fmt == T_Q8_0) kern = k_gemm_bf16_direct<T_Q8_0>;
  else if (p.direct) kern = fmt == T_Q4_K ? k_gemm_bf16_direct<T_Q4_K> : k_gemm_bf16_direct<T_Q6_K>;
  else if (fmt == T_Q4_K) kern = k_gemm_bf16_ring<160, 256, 3, T_Q4_K>;
  else if (fmt == T_Q6_K) kern = k_gemm_bf16_ring<160, 256, 3, T_Q6_K>;
  else return hipErrorInvalidValue;
  hipLaunchKernelGGL(kern, dim3((unsigned)nb), dim3(512), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ksplit == 1) return e;
  if (defer && add) {
    *defer = p.ksplit;
    return hipSuccess;
  }
  ReduceSegs r{};
  r.nseg = count;
  int blocks = 0;
  for (int i = 0; i < count; i++) {
    r.part[i] = a.seg[i].part;
    r.y[i] = a.seg[i].y;
    r.count[i] = (long)n * a.seg[i].rows;
    r.blk0[i] = blocks;
    blocks += (int)((r.count[i] / 4 + 255) / 256 + 1);
  }
  r.blk0[count] = blocks;
  hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)blocks), dim3(256), 0, st, r, p.ksplit, add ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_gemm_bf16_swiglu(const gq_weight *gate, const gq_weight *up, const uint16_t *xb, int n,
                                   uint16_t *hb, int num_cus, hipStream_t st) {
  (void)num_cus;
  if (n <= 128) return hipErrorNotSupported;  // the ring kernel's batches
  const Layout &L = gate->L;
  if (up->L.dtype != L.dtype || up->L.units != L.units || up->L.rows != L.rows || !gate->gemm_raw ||
      !up->gemm_raw)
    return hipErrorNotSupported;
  if (L.dtype != T_Q4_K && L.dtype != T_Q6_K && L.dtype != T_Q5_K && L.dtype != T_Q8_0)
    return hipErrorNotSupported;
  GemmArgs a{};
  a.nseg = 1;
  a.ntiles = (n + BN - 1) / BN;
  a.ksplit = 1;
  a.n = n;
  a.kpad = L.units * 256;
  a.xb = xb;
  a.pair = 1;
  a.hkpad = (L.rows + 255) / 256 * 256;
  a.hb = hb;
  a.seg[0].rec = gate->gemm_raw;
  a.seg[0].rows = L.rows;
  a.seg[0].tile_begin = 0;
  a.seg[1].rec = up->gemm_raw;
  a.seg[1].rows = L.rows;
  // 80 output rows per tile, over every padded column of hb (rows past F
  // give zeros)
  const long nb = (long)((a.hkpad + BM / 2 - 1) / (BM / 2)) * a.ntiles;
  if (nb > 0x7fffffffL) return hipErrorInvalidValue;
  void (*kern)(GemmArgs) = L.dtype == T_Q4_K   ? k_gemm_bf16_direct<T_Q4_K>
                           : L.dtype == T_Q6_K ? k_gemm_bf16_direct<T_Q6_K>
                           : L.dtype == T_Q5_K ? k_gemm_bf16_direct<T_Q5_K>
                                               : k_gemm_bf16_direct<T_Q8_0>;
  hipLaunchKernelGGL(kern, dim3((unsigned)nb), dim3(512), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_gemm(const gq_weight *w, const float *X, int n, float *Y, int mode,
                       void *workspace, size_t ws_bytes, int num_cus, hipStream_t st) {
  (void)ws_bytes;
  const Layout &L = w->L;
  const int kpad = L.units * 256;
  if (mode == GQ_GEMM_BF16) {
    uint16_t *xb = (uint16_t *)workspace;
    const size_t xbb = (size_t)((n + GEMM_NPAD - 1) / GEMM_NPAD * GEMM_NPAD) * kpad * 2;
    float *part = (float *)((char *)workspace + ((xbb + 255) & ~(size_t)255));
    hipError_t e = launch_x_to_frag(X, n, L.k, xb, st);
    if (e != hipSuccess) return e;
    return launch_gemm_bf16(&w, &Y, 1, xb, n, part, false, num_cus, st);
  } else {
    if (!w->gemm_raw) return hipErrorInvalidValue;
    const int npad = (n + I8N - 1) / I8N * I8N;
    int8_t *xq = (int8_t *)workspace;
    float2 *xr = (float2 *)((char *)workspace + (((size_t)npad * kpad + 255) & ~(size_t)255));
    const long threads = (long)npad * (kpad / 8);
    hipLaunchKernelGGL(k_x_to_q8_frag, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, X,
                       n, npad, L.k, kpad, xq, xr);
    if (L.dtype == T_Q6_K) {
      hipLaunchKernelGGL(k_gemm_i8_q6k, dim3((unsigned)((L.rows + Q6M - 1) / Q6M), (unsigned)((n + Q6N - 1) / Q6N)),
                         dim3(256), 0, st, (const uint8_t *)w->gemm_raw, L.rows, (const int8_t *)xq,
                         (const float2 *)xr, n, kpad, Y);
      return hipGetLastError();
    }
    const int ntiles = npad / I8N, mtiles = (L.rows + I8M - 1) / I8M;
    hipLaunchKernelGGL(k_gemm_i8_direct, dim3((unsigned)(mtiles * ntiles)), dim3(512), 0, st,
                       (const uint8_t *)w->gemm_raw, L.rows, ntiles, (const int8_t *)xq,
                       (const float2 *)xr, n, kpad, Y);
  }
  return hipGetLastError();
}

}  // namespace gq
