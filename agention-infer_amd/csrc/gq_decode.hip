// gq_decode.hip -- the non-matmul kernels of a GPU-resident decode step for
// a dense Llama/Qwen2-style decoder and the step's launch sequence (the
// reference's run_gpu_resident, src/model/llama/gpu_resident.rs:427-697,
// restating the arithmetic of LlamaModel::run, src/model/llama/
// cpu_path.rs:695-818).
//
// One step is 6 launches per layer plus 2:
//   qkv matvec   input RMSNorm(x_b) (layer 0: of the embedding row, which
//                block 0 stores as x_b)
//   attention    RoPE of q and of the new k, f16 KV row store, scores,
//                softmax and the weighted V sum for all query heads of one
//                KV head over a chunk of positions
//   merge        the chunk partials of each query head combined
//   o matvec     epilogue x_a = x_b + o (the residual add)
//   gate/up      one matvec over both matrices with input RMSNorm(x_a)
//                and output silu(gate) * up
//   down matvec  epilogue x_b = x_a + down
// then the output head (input RMSNorm(x_b)) and the greedy argmax.
//
// Step state (token, position, step counter) lives in device memory so that
// a captured HIP graph of one step can be replayed for every greedy step:
// the argmax writes the next token and advances the position.  The head's
// per-block maxima are rewritten by every step, so a replay starts from the
// same state.
#include "gq_device.h"
#include "gq_internal.h"

namespace gq {


// ----------------------------------------------------------- attention
// Block (kv head kh, chunk c): positions [c*CH, min((c+1)*CH, n)) for the
// `group` query heads kh*group .. kh*group+group-1 (GQA: each K/V row is
// read once for all of them), ATT_WAVES waves; short chunks so that the
// whole GPU shares the work (a 4096-position context is 4 x 65 blocks).
//   scores  s[g][t] = (q_g . k_t) / sqrt(hd)        (attention_into,
//   softmax m_g = max s, p = exp(s - m_g), l_g = sum p   cpu_path.rs:141-194)
//   values  o[g][d] = sum_t p[g][t] v_t[d]
// Scores run on v_mfma_f32_16x16x32_f16 (rows = query heads, columns =
// positions, depth = head dims): K rows are f16 already and go straight
// from HBM into the B operands; each 32-dim chunk of q is scaled by a power
// of two and split into f16 hi + lo parts, so each product is exact in fp32
// and q is carried to ~22 bits.  The V sum runs on fp32 FMAs: wave w owns a quarter of the
// dims, a lane 2 dims of a group of consecutive positions, and the groups'
// sums are added across lanes with lane swaps.  Everything that does not depend on
// the position (q, the new k and v, the RoPE denominators) is loaded before
// the position is read, and each thread computes the one RoPE angle it
// needs, so the block has three barriers.
// The partial (m, l, o) of each (head, chunk) goes to `part`; the next
// kernel (k_attn_merge) merges the chunks:
//   att[h] = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M).
// (A merge by the last block to finish costs every block a device-scope
// release fence, which writes back its XCD's L2: slower than a launch.)
// The block holding position pos = n - 1 also rotates the new k, rounds k
// and v to f16 (KvDtype::F16::pack) and stores them in the cache; it uses
// the rounded values for position pos itself.  RoPE angles are
// pos / den[i] with den[i] = theta^(2i/hd) from the host (cpu_path.rs:99-133).
constexpr int ATT_MAXG = 8;      // query heads per KV head
constexpr int ATT_WAVES = 4;
constexpr int ATT_THREADS = 64 * ATT_WAVES;
static_assert(ATT_CHUNK == 16 * ATT_WAVES, "16 positions per wave");

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4a_t __attribute__((ext_vector_type(4)));

// Q8 (the Q8_0 KV cache, KvDtype::Q8_0, src/model/mod.rs:540-603): kc / vc
// hold int8 codes [ctx][kvd] and ksc / vsc the f16 scales of each 32-value
// block [ctx][kvd / 32].  A 32-deep MFMA step is exactly one block: it runs
// on the codes (int8 -> f16 is exact) and its result is scaled by the key's
// block scale; V values are code * scale.  The new row is packed like
// KvDtype::Q8_0::pack (scale = max|x| / 127 stored as f16, codes =
// round(x / scale) in [-127, 127]) and used as stored for its position.
// Sum of x over the row groups of LPR lanes (LPR = 8 or 16) of a wave, in
// every lane: pairs of 8-lane halves by a row rotation, then 16-lane rows
// and 32-lane halves by the gfx950 lane swaps (each sum is the same in
// both lanes of a pair, so every lane gets the identical total).
template <int LPR>
__device__ __forceinline__ float row_groups_sum(float x) {
  static_assert(LPR == 8 || LPR == 16, "row groups of 8 or 16 lanes");
  if constexpr (LPR == 8)
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// Max of x over each 32-lane half of a wave, in every lane: row rotations
// by 8, 4, 2, 1 within the 16-lane rows, then the rows of a pair by the
// gfx950 lane swap.
__device__ __forceinline__ float max32(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xF, 0xF, false)));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <int HD, bool Q8>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_gqa(
    const float *q, const float *k, const float *v, uint16_t *kc, uint16_t *vc, uint16_t *ksc,
    uint16_t *vsc, const DecodeState *st, int group, int kvd, const float *rope_den, float *part) {
  constexpr int CH = ATT_CHUNK;
  constexpr int NW = ATT_WAVES;
  constexpr int PW = CH / NW;  // positions per wave in the scores: one 16-column MFMA tile
  constexpr int KS = HD / 32;  // MFMA depth steps
  constexpr int HALF = HD / 2;
  // V sum: wave w owns dims [w*HD/NW, (w+1)*HD/NW), 2 per lane; the lanes
  // of a wave form RG row groups of RPG consecutive positions each.
  constexpr int LPR = HD / (2 * NW);  // lanes per row group
  constexpr int RG = 64 / LPR;
  constexpr int RPG = CH / RG;
  constexpr int QIT = ATT_MAXG * HD / ATT_THREADS;  // q values per thread
  static_assert(ATT_THREADS % HD == 0 && RPG % 4 == 0, "attention layout");
  __shared__ float sp[ATT_MAXG][CH];
  __shared__ __align__(16) _Float16 qhi[ATT_MAXG][HD], qlo[ATT_MAXG][HD];
  __shared__ __align__(16) float qinv[KS][16];  // 2^-e of each (32-dim chunk, head); 16 MFMA rows
  __shared__ __align__(16) uint16_t knew[HD];  // f16 bits (Q8: the code as f16)
  __shared__ __align__(16) uint16_t vnew[HD];
  __shared__ float knew_sc[HD / 32], vnew_sc[HD / 32];  // Q8: the new row's scales
  __shared__ float gm_s[ATT_MAXG], gl_s[ATT_MAXG];

  const int kh = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // The loads that do not depend on the position go out first: this
  // thread's q values (dim d of heads g = (tid + it*ATT_THREADS) / HD, and
  // the NEOX partner dim), the new k / v values and the RoPE denominator.
  const int d = tid % HD, ir = d % HALF, dp = (d + HALF) % HD;
  const float den = rope_den[ir];
  float qown[QIT], qpar[QIT];
#pragma unroll
  for (int it = 0; it < QIT; it++) {
    const int g = (tid + it * ATT_THREADS) / HD;
    const float *qh = q + (long)(kh * group + min(g, group - 1)) * HD;
    qown[it] = qh[d];
    qpar[it] = qh[dp];
  }
  const float kown = k[(long)kh * HD + d], kpar = k[(long)kh * HD + dp];
  const float vv = v[(long)kh * HD + d];

  const int pos = st->pos, n = pos + 1, t0 = c * CH;
  if (t0 >= n) return;
  const int nchunk_grid = gridDim.y;
  const int tw = t0 + wave * PW;  // first scores position of this wave

  // K rows as MFMA B operands (row tw + lane%16, dims 8*(lane/16) + 32*ks);
  // V: dims 2*(lane%LPR) of the wave's dim slice, rows RPG*(lane/LPR) + j.
  // Rows are clamped to n - 1 (unused past n).
  const int8_t *kq8 = (const int8_t *)kc, *vq8 = (const int8_t *)vc;
  const int nbr = kvd / 32;  // Q8 blocks per row
  uint4 kb[KS];
  float kscl[KS];
  {
    const int t = min(tw + (lane & 15), n - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      if constexpr (Q8) {
        const uint2 w = ldw2(kq8 + (long)t * kvd + (long)kh * HD + 8 * (lane >> 4) + 32 * ks);
        kb[ks] = make_uint4(w.x, w.y, 0u, 0u);
        kscl[ks] = h2f(ldh(ksc + (long)t * nbr + (kh * HD) / 32 + ks));
      } else {
        kb[ks] = ldw4(kc + (long)t * kvd + (long)kh * HD + 8 * (lane >> 4) + 32 * ks);
      }
    }
  }
  const int vdim = wave * (HD / NW) + 2 * (lane % LPR);  // first of this lane's 2 dims
  const int vrow = t0 + RPG * (lane / LPR);              // first of its RPG rows
  uint32_t vr[RPG];
  float vscl[RPG];
#pragma unroll
  for (int j = 0; j < RPG; j++) {
    const long row = min(vrow + j, n - 1);
    if constexpr (Q8) {
      vr[j] = ldh((const uint16_t *)(vq8 + row * kvd + (long)kh * HD + vdim));
      vscl[j] = h2f(ldh(vsc + row * nbr + (kh * HD + vdim) / 32));
    } else {
      vr[j] = ldw1(vc + row * kvd + (long)kh * HD + vdim);
      vscl[j] = 1.f;
    }
  }

  // RoPE angle of pair index ir (NEOX pairs d <-> d + hd/2): pos / den.
  float sn, cs;
  sincosf((float)pos / den, &sn, &cs);
  // New K/V row of this KV head: rotate k, round both to f16, store.
  if (pos < t0 + CH && tid < HD) {
    const float rot = d < HALF ? kown * cs - kpar * sn : kpar * sn + kown * cs;
    if constexpr (Q8) {
      // 32-lane groups are the 32-value blocks (HD is a multiple of 64)
      float km = fabsf(rot), vm = fabsf(vv);
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) {
        km = fmaxf(km, __shfl_xor(km, off, 32));
        vm = fmaxf(vm, __shfl_xor(vm, off, 32));
      }
      const float kscale = km > 0.f ? km / 127.0f : 1.0f, vscale = vm > 0.f ? vm / 127.0f : 1.0f;
      const float kcode = fminf(fmaxf(roundf(rot / kscale), -127.f), 127.f);
      const float vcode = fminf(fmaxf(roundf(vv / vscale), -127.f), 127.f);
      const uint16_t ks16 = __half_as_ushort(__float2half_rn(kscale));
      const uint16_t vs16 = __half_as_ushort(__float2half_rn(vscale));
      knew[d] = __half_as_ushort(__float2half_rn(kcode));
      vnew[d] = __half_as_ushort(__float2half_rn(vcode));
      ((int8_t *)kc)[(long)pos * kvd + (long)kh * HD + d] = (int8_t)kcode;
      ((int8_t *)vc)[(long)pos * kvd + (long)kh * HD + d] = (int8_t)vcode;
      if ((d & 31) == 0) {
        knew_sc[d / 32] = h2f(ks16);
        vnew_sc[d / 32] = h2f(vs16);
        ksc[(long)pos * nbr + (kh * HD + d) / 32] = ks16;
        vsc[(long)pos * nbr + (kh * HD + d) / 32] = vs16;
      }
    } else {
      const uint16_t kbits = __half_as_ushort(__float2half_rn(rot));
      const uint16_t vbits = __half_as_ushort(__float2half_rn(vv));
      knew[d] = kbits;
      vnew[d] = vbits;
      kc[(long)pos * kvd + (long)kh * HD + d] = kbits;
      vc[(long)pos * kvd + (long)kh * HD + d] = vbits;
    }
  }
  // Rotated q of the group's heads as MFMA A operands: each 32-dim chunk
  // of a head is scaled by 2^e (its max |q| in [512, 1024); the chunk is 32
  // consecutive lanes) and split into f16 hi + lo, so q is carried to ~22
  // bits and each product with an f16 key is exact in fp32.
#pragma unroll
  for (int it = 0; it < QIT; it++) {
    const int g = (tid + it * ATT_THREADS) / HD;  // uniform per wave
    if (g < group) {
      const float rot = d < HALF ? qown[it] * cs - qpar[it] * sn : qpar[it] * sn + qown[it] * cs;
      const float m32 = max32(fabsf(rot));
      int ex = 0;
      (void)frexpf(m32, &ex);
      const float qscale = m32 > 0.f ? ldexpf(1.0f, 10 - ex) : 1.0f;
      const float x = rot * qscale;  // exact (a power of two)
      const _Float16 h = (_Float16)x;
      qhi[g][d] = h;
      qlo[g][d] = (_Float16)(x - (float)h);
      if ((d & 31) == 0) qinv[d / 32][g] = 1.0f / qscale;  // exact
    }
  }
  __syncthreads();

  // A operands: lane holds head lane%16, dims 8*(lane/16) + 32*ks .. +8.
  f16x8_t ahi[KS], alo[KS];
  {
    const int m = lane & 15;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      if (m < group) {
        ahi[ks] = *(const f16x8_t *)&qhi[m][8 * (lane >> 4) + 32 * ks];
        alo[ks] = *(const f16x8_t *)&qlo[m][8 * (lane >> 4) + 32 * ks];
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++) ahi[ks][j] = alo[ks][j] = (_Float16)0.f;
      }
    }
  }

  // Scores: lane holds S[head 4*(lane/16) + i][position tw + lane%16]; each
  // chunk's product is rescaled by its heads' 2^-e (exactly).
  {
    const float rsq = sqrtf((float)HD);
    const int tcol = tw + (lane & 15);
    const bool isnew = tcol == pos;
    f32x4a_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      // the new row's fragment (read whether used or not)
      const uint4 kn = *(const uint4 *)(knew + 8 * (lane >> 4) + 32 * ks);
      f16x8_t bk;
      if constexpr (Q8) {
        _Float16 h8[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
          h8[e] = (_Float16)(float)(int8_t)(((e < 4 ? kb[ks].x : kb[ks].y) >> (8 * (e & 3))) & 0xffu);
        uint4 raw;
        __builtin_memcpy(&raw, h8, 16);
        raw = make_uint4(isnew ? kn.x : raw.x, isnew ? kn.y : raw.y, isnew ? kn.z : raw.z,
                         isnew ? kn.w : raw.w);
        __builtin_memcpy(&bk, &raw, 16);
        const float sc = isnew ? knew_sc[ks] : kscl[ks];
        f32x4a_t part_acc = {0.f, 0.f, 0.f, 0.f};
        part_acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[ks], bk, part_acc, 0, 0, 0);
        part_acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[ks], bk, part_acc, 0, 0, 0);
        const float4 iv = *(const float4 *)&qinv[ks][4 * (lane >> 4)];
        const float ivs[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(sc * ivs[i], part_acc[i], acc[i]);
      } else {
        const uint4 raw = make_uint4(isnew ? kn.x : kb[ks].x, isnew ? kn.y : kb[ks].y,
                                     isnew ? kn.z : kb[ks].z, isnew ? kn.w : kb[ks].w);
        __builtin_memcpy(&bk, &raw, 16);
        f32x4a_t part_acc = {0.f, 0.f, 0.f, 0.f};
        part_acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[ks], bk, part_acc, 0, 0, 0);
        part_acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[ks], bk, part_acc, 0, 0, 0);
        const float4 iv = *(const float4 *)&qinv[ks][4 * (lane >> 4)];
        const float ivs[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(ivs[i], part_acc[i], acc[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int g = 4 * (lane >> 4) + i;
      if (g < group) sp[g][tcol - t0] = tcol < n ? acc[i] / rsq : -INFINITY;
    }
  }
  __syncthreads();

  // Softmax statistics of the chunk: wave w handles heads w and w + NW;
  // lane = position.
  {
    constexpr int GPW = ATT_MAXG / NW;
    float val[GPW], mh[GPW], p[GPW], lh[GPW];
#pragma unroll
    for (int i = 0; i < GPW; i++) val[i] = wave + NW * i < group ? sp[wave + NW * i][lane] : 0.f;
#pragma unroll
    for (int i = 0; i < GPW; i++) mh[i] = wave_max(val[i]);
#pragma unroll
    for (int i = 0; i < GPW; i++) p[i] = expf(val[i] - mh[i]);  // exp(-inf) = 0 past n
#pragma unroll
    for (int i = 0; i < GPW; i++) lh[i] = wave_sum(p[i]);
#pragma unroll
    for (int i = 0; i < GPW; i++) {
      const int g = wave + NW * i;
      if (g < group) {
        sp[g][lane] = p[i];
        if (lane == 0) {
          gm_s[g] = mh[i];
          gl_s[g] = lh[i];
        }
      }
    }
  }
  __syncthreads();

  // Values: o[g][d] = sum over the row groups of the sums over their rows
  // (in order) of p * v, for this lane's 2 dims.
  {
    const uint32_t vn = *(const uint32_t *)(vnew + vdim);
    float vf[RPG][2];
#pragma unroll
    for (int j = 0; j < RPG; j++) {
      // Rows past pos were clamped to row pos, which this launch is still
      // writing: their p is 0, but 0 * (stale NaN/inf) is not, so they
      // read as 0; row pos itself is the freshly rounded one.
      const int t = vrow + j;
      if constexpr (Q8) {
        // the new row's values were stored as the f16 of its codes
#pragma unroll
        for (int e = 0; e < 2; e++) {
          const float code = t == pos ? h2f(vn >> (16 * e))
                                      : (float)(int8_t)((vr[j] >> (8 * e)) & 0xffu);
          const float sc = t == pos ? vnew_sc[vdim / 32] : vscl[j];
          vf[j][e] = t > pos ? 0.f : code * sc;
        }
      } else {
        const uint32_t raw = t == pos ? vn : (t > pos ? 0u : vr[j]);
#pragma unroll
        for (int e = 0; e < 2; e++) vf[j][e] = h2f(raw >> (16 * e));
      }
    }
    const int rbase = vrow - t0;
    float *pout = part + ((long)(kh * group) * nchunk_grid + c) * (2 + HD) + 2 + vdim;
#pragma unroll
    for (int g = 0; g < ATT_MAXG; g++) {
      if (g < group) {
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int j = 0; j < RPG; j += 4) {
          const float4 p4 = *(const float4 *)&sp[g][rbase + j];
          const float pr[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
          for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int e = 0; e < 2; e++) acc[e] = fmaf(pr[jj], vf[j + jj][e], acc[e]);
        }
        float o[2];
#pragma unroll
        for (int e = 0; e < 2; e++) o[e] = row_groups_sum<LPR>(acc[e]);
        if (lane < LPR)
          *(float2 *)(pout + (long)g * nchunk_grid * (2 + HD)) = make_float2(o[0], o[1]);
      }
    }
  }
  if (tid < group) {
    float *pm = part + ((long)(kh * group + tid) * nchunk_grid + c) * (2 + HD);
    pm[0] = gm_s[tid];
    pm[1] = gl_s[tid];
  }
}

// Merge of the chunk partials: block (h, y) = query head h, dims
// 16 y .. 16 y + 15, 256 threads; thread (qq, d) (qq < MQ = 16) sums dim d
// over the chunks c = qq, qq + MQ, ..., then the MQ partial sums are added
// in order (small blocks: a head's dims spread over HD / 16 of them; 16
// dims per block measured 0.15% faster decode than 32):
//   att[h][d] = sum_c o_c[d] e^(m_c - M) / sum_c l_c e^(m_c - M),
// M = max_c m_c over the chunks holding positions <= pos.  Every load of
// the first 16 * MQ chunks (m, l and o: 16384 positions) is issued at the
// start; every block of a head computes the head's M and L.
constexpr int ATT_MERGE_THREADS = 256, ATT_MERGE_DIMS = 16;
template <int HD>
__global__ __launch_bounds__(ATT_MERGE_THREADS) void k_attn_merge(const DecodeState *st, int nchunk_grid,
                                                             const float *part, float *att) {
  constexpr int NT = ATT_MERGE_THREADS, DB = ATT_MERGE_DIMS, MQ = NT / DB, NWV = NT / 64, R = 16;
  static_assert(HD % DB == 0, "dims per block");
  __shared__ float fac[ATT_MAX_CTX / ATT_CHUNK];
  __shared__ float red[NWV];
  __shared__ float osum[MQ][DB];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // The first loads go out before the position is known: chunks of the
  // grid past the last one in use are read and then ignored.
  const float *ph = part + (long)h * nchunk_grid * (2 + HD);
  const int qq = tid / DB, dl = tid % DB, d = DB * blockIdx.y + dl;
  const float *po = ph + 2 + d;
  float vals[R];
#pragma unroll
  for (int j = 0; j < R; j++) {
    const int c = qq + MQ * j;
    vals[j] = c < nchunk_grid ? po[(long)c * (2 + HD)] : 0.f;
  }
  float mraw = -INFINITY, lraw = 0.f;
  if (tid < nchunk_grid) {
    mraw = ph[(long)tid * (2 + HD)];
    lraw = ph[(long)tid * (2 + HD) + 1];
  }
  const int nch = (st->pos + ATT_CHUNK) / ATT_CHUNK;
  const float mv = tid < nch ? mraw : -INFINITY, lv = tid < nch ? lraw : 0.f;
  float M = mv;
  for (int c = tid + NT; c < nch; c += NT) M = fmaxf(M, ph[(long)c * (2 + HD)]);
  M = wave_max(M);
  if (lane == 0) red[wave] = M;
  __syncthreads();
  M = red[0];
#pragma unroll
  for (int w = 1; w < NWV; w++) M = fmaxf(M, red[w]);
  __syncthreads();
  float L = 0.f;
  if (tid < nch) {
    const float e = expf(mv - M);
    fac[tid] = e;
    L = lv * e;
  }
  for (int c = tid + NT; c < nch; c += NT) {
    const float e = expf(ph[(long)c * (2 + HD)] - M);
    fac[c] = e;
    L += ph[(long)c * (2 + HD) + 1] * e;
  }
  L = wave_sum(L);
  if (lane == 0) red[wave] = L;
  __syncthreads();
  L = red[0];
#pragma unroll
  for (int w = 1; w < NWV; w++) L += red[w];
  float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < R; j++) {
    const int c = qq + MQ * j;
    s4[j & 3] += c < nch ? vals[j] * fac[c] : 0.f;
  }
  for (int cb = qq + MQ * R; cb < nch; cb += MQ * R) {
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int c = cb + MQ * j;
      vals[j] = c < nch ? po[(long)c * (2 + HD)] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int c = cb + MQ * j;
      s4[j & 3] += c < nch ? vals[j] * fac[c] : 0.f;
    }
  }
  osum[qq][dl] = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  __syncthreads();
  if (qq == 0) {
    float o = osum[0][dl];
#pragma unroll
    for (int i = 1; i < MQ; i++) o += osum[i][dl];
    att[(long)h * HD + d] = o / L;
  }
}

// -------------------------------------------------------------- argmax
// Greedy argmax (first maximum wins, sampler.rs:120-131): the head
// matvec's blocks leave per-block maxima, k_argmax_final merges them.
__device__ __forceinline__ void amax_merge(float &bv, int &bi, float ov, int oi) {
  if (ov > bv || (ov == bv && oi < bi)) {
    bv = ov;
    bi = oi;
  }
}

__device__ __forceinline__ void block_amax(float &bv, int &bi, float *sv, int *si) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    amax_merge(bv, bi, ov, oi);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  bv = sv[0];
  bi = si[0];
  for (int j = 1; j < 4; j++) amax_merge(bv, bi, sv[j], si[j]);
}

// The head matvec's blocks leave the first maximum of their rows in
// pv / pi[0 .. ARGMAX_SLOTS) (slots of blocks that do not exist keep
// -inf / INT_MAX from set-up); one block reduces them and advances the step
// state (the token is recorded and becomes the next input; the position
// advances).  No fences: the kernel boundary
// orders the partials before this read.
__global__ __launch_bounds__(256) void k_argmax_final(const float *pv, const int *pi,
                                                      DecodeState *st, int *tokens,
                                                      int max_tokens) {
  __shared__ float sv[4];
  __shared__ int si[4];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int b = threadIdx.x; b < ARGMAX_SLOTS; b += 256) amax_merge(bv, bi, pv[b], pi[b]);
  block_amax(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    const int idx = bi == 0x7fffffff ? 0 : bi;  // no logit above -inf: index 0
    const int step = st->step;
    if (tokens && step < max_tokens) tokens[step] = idx;
    *st = DecodeState{idx, st->pos + 1, step + 1, 0};
  }
}

// Start a decode sequence: token and position from the host, step 0.
__global__ void k_set_state(DecodeState *st, int token, int pos) {
  if (threadIdx.x == 0) *st = DecodeState{token, pos, 0, 0};
}

// ------------------------------------------------------------------ host
hipError_t launch_set_state(DecodeState *st, int token, int pos, hipStream_t s) {
  hipLaunchKernelGGL(k_set_state, dim3(1), dim3(64), 0, s, st, token, pos);
  return hipGetLastError();
}

hipError_t launch_decode_step(const DecodeLaunch &m, hipStream_t s) {
  const int hd = m.head_dim, nh = m.n_heads, nkv = m.n_kv_heads;
  const int kvd = nkv * hd, group = nh / nkv;
  hipError_t e;
  // The down projections split their K range over two sets of blocks
  // (MvIn::y2): x_b = (x_a + down_0) and proj = down_1, added by the next
  // norm, which stores x_c = x_b + proj as the residual stream.
  for (int L = 0; L < m.n_layers; L++) {
    // q, k, v of RMSNorm(x), x the residual stream
    MvIn in;
    in.src = MV_NORM;
    // (layer 0 stores the embedding row as the residual stream x_b; later
    // layers store x_c = x_b + proj from the previous down launch's halves,
    // or read x_b = x_a + down when it did not split)
    const bool split_in = L && mv_ksplit_ok(m.wdown[L - 1]->L.units);
    float *xres = split_in ? m.xc : m.xb;  // the stream the o projection adds to
    in.x = L ? m.xb : m.embd;
    in.r = split_in ? m.proj : nullptr;
    in.tok = L ? nullptr : &m.state->token;
    in.nw = m.attn_norm[L];
    in.xo = !L || split_in ? xres : nullptr;
    in.eps = m.eps;
    in.q8k = true;  // matmul_qkv_into -> matmul_into (cpu_path.rs:319-321)
    // One launch per distinct dtype among q/k/v (GGUF Q4_K_M files carry
    // attn_v in Q6_K on some layers); each launch recomputes the norm and
    // stores the same x_b.
    const gq_weight *qkv[3] = {m.wq[L], m.wk[L], m.wv[L]};
    float *qkv_out[3] = {m.q, m.k, m.v};
    bool done[3] = {false, false, false};
    for (int i = 0; i < 3; i++) {
      if (done[i]) continue;
      const gq_weight *grp[3];
      float *gout[3];
      int n = 0;
      for (int j = i; j < 3; j++)
        if (!done[j] && qkv[j]->L.dtype == qkv[i]->L.dtype) {
          grp[n] = qkv[j];
          gout[n++] = qkv_out[j];
          done[j] = true;
        }
      if ((e = matvec_launch(grp, n, in, gout, s)) != hipSuccess) return e;
    }
    // F16: [layer][ctx][kvd] f16; Q8: [layer][ctx][kvd] int8 codes (in the
    // same allocation) and [layer][ctx][kvd / 32] f16 scales
    const long lo = (long)L * m.ctx * kvd;
    uint16_t *kc = m.kv_q8 ? (uint16_t *)((int8_t *)m.kcache + lo) : m.kcache + lo;
    uint16_t *vc = m.kv_q8 ? (uint16_t *)((int8_t *)m.vcache + lo) : m.vcache + lo;
    uint16_t *ksc = m.kv_q8 ? m.kscale + (long)L * m.ctx * (kvd / 32) : nullptr;
    uint16_t *vsc = m.kv_q8 ? m.vscale + (long)L * m.ctx * (kvd / 32) : nullptr;
    const dim3 ag(nkv, m.att_chunks), at(ATT_THREADS);
    if (hd == 128 && m.kv_q8)
      hipLaunchKernelGGL((k_attn_gqa<128, true>), ag, at, 0, s, m.q, m.k, m.v, kc, vc, ksc, vsc, m.state,
                         group, kvd, m.rope_den, m.att_part);
    else if (hd == 128)
      hipLaunchKernelGGL((k_attn_gqa<128, false>), ag, at, 0, s, m.q, m.k, m.v, kc, vc, ksc, vsc, m.state,
                         group, kvd, m.rope_den, m.att_part);
    else if (m.kv_q8)
      hipLaunchKernelGGL((k_attn_gqa<64, true>), ag, at, 0, s, m.q, m.k, m.v, kc, vc, ksc, vsc, m.state,
                         group, kvd, m.rope_den, m.att_part);
    else
      hipLaunchKernelGGL((k_attn_gqa<64, false>), ag, at, 0, s, m.q, m.k, m.v, kc, vc, ksc, vsc, m.state,
                         group, kvd, m.rope_den, m.att_part);
    if (hd == 128)
      hipLaunchKernelGGL(k_attn_merge<128>, dim3(m.n_heads, 128 / ATT_MERGE_DIMS), dim3(ATT_MERGE_THREADS), 0, s, m.state, m.att_chunks,
                         m.att_part, m.att);
    else
      hipLaunchKernelGGL(k_attn_merge<64>, dim3(m.n_heads, 64 / ATT_MERGE_DIMS), dim3(ATT_MERGE_THREADS), 0, s, m.state, m.att_chunks,
                         m.att_part, m.att);
    MvIn ain;
    ain.x = m.att;
    ain.q8k = true;  // matmul_into (cpu_path.rs:757)
    ain.res = xres;  // x_a = x_b + o (cpu_path.rs:780-782)
    const gq_weight *wo[1] = {m.wo[L]};
    float *xa[1] = {m.xa};
    if ((e = matvec_launch(wo, 1, ain, xa, s)) != hipSuccess) return e;
    // h = silu(gate . n) * (up . n), n = RMSNorm(x_a)
    MvIn fin;
    fin.src = MV_NORM;
    fin.x = m.xa;
    fin.nw = m.ffn_norm[L];
    fin.eps = m.eps;
    const gq_weight *gu[2] = {m.wgate[L], m.wup[L]};
    float *hout[2] = {m.h, nullptr};
    if ((e = matvec_launch(gu, 2, fin, hout, s, true)) != hipSuccess) return e;
    MvIn din;
    din.x = m.h;
    din.q8k = true;  // matmul_ffn_into's down: matmul_into (cpu_path.rs:383)
    din.res = m.xa;  // x_b = x_a + down (cpu_path.rs:806-808)
    if (mv_ksplit_ok(m.wdown[L]->L.units)) din.y2 = m.proj;
    const gq_weight *wd[1] = {m.wdown[L]};
    float *xb[1] = {m.xb};
    if ((e = matvec_launch(wd, 1, din, xb, s)) != hipSuccess) return e;
  }
  // logits of RMSNorm(x_a + proj)
  MvIn hin;
  hin.src = MV_NORM;
  hin.x = m.xb;
  hin.r = m.n_layers && mv_ksplit_ok(m.wdown[m.n_layers - 1]->L.units) ? m.proj : nullptr;
  hin.nw = m.output_norm;
  hin.eps = m.eps;
  hin.q8k = true;  // the head: matmul_into (cpu_path.rs:815)
  const gq_weight *hw[1] = {m.lm_head};
  float *lo[1] = {m.logits};
  if (!m.lm_head->L.quad) return hipErrorInvalidValue;  // dense weights are quad-layout
  // argmax partials from the head's blocks, one final block
  hin.amax_v = m.amax_v;
  hin.amax_i = m.amax_i;
  if ((e = matvec_launch(hw, 1, hin, lo, s)) != hipSuccess) return e;
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, m.amax_v, m.amax_i, m.state,
                     m.tokens, m.max_tokens);
  return hipGetLastError();
}

}  // namespace gq
