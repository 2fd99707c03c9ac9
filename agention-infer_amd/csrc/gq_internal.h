// gq_internal.h -- host/device structures shared by the gq translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gq_layout.h"

// The public handle (opaque in gq.h).
struct gq_weight {
  gq::Layout L;      // dtype, rows, k, units, chunks, rt
  uint8_t *body;     // device body in the wave-tiled layout
  uint16_t *d;       // per-unit f16 scales (Q6_K, IQ3_XXS), or nullptr
  size_t ggml_bytes; // size of the tensor in ggml block order
  int device;
  uint8_t *gemm_raw = nullptr;  // per-stage records for the bf16 GEMM (made on first use)
};

namespace gq {

constexpr int MV_MAX_SEG = 4;
constexpr float LIMB_RANGE = 8323072.0f;  // 127 * 65536: |X| <= this

// One matrix of a matvec launch.  Its rows are split into nblk contiguous
// ranges of equal size (+-1 row), one per block, blocks blk_begin ..
// blk_begin + nblk - 1.
struct MvSeg {
  const uint8_t *body;
  const uint16_t *d;
  float *y;
  int rows;
  int blk_begin;
  int nblk;
};

// Threads per matvec block: as many waves as the format's registers allow
// (bytes in flight set the HBM throughput): 4 per SIMD for IQ3_XXS, 3 for
// Q4_K/Q5_K, 2 for the others.
__host__ __device__ constexpr int mv_threads(int fmt) {
  return fmt == 18 ? 1024 : fmt == 12 || fmt == 13 || fmt == 113 ? 768 : 512;
}

// Where the matvec input vector comes from.
enum MvSource {
  MV_X = 0,       // x
  MV_SWIGLU = 1,  // silu(xg) * xu
  MV_NORM = 2,    // RMSNorm(x + r) * nw; block 0 stores x + r to xo
};

struct MvIn {
  int src = MV_X;
  const float *x = nullptr;   // MV_X / MV_NORM residual stream
  const float *xg = nullptr, *xu = nullptr;
  const float *r = nullptr;   // MV_NORM: residual added to x (may be null)
  const float *nw = nullptr;  // MV_NORM: norm weight
  float *xo = nullptr;        // MV_NORM: x + r written here (may be null)
  const int *tok = nullptr;   // MV_NORM: if set, x is row *tok of the table x
  const float *res = nullptr; // one-matrix launches: y = res + W . x (the residual add,
                              // x += proj of cpu_path.rs:780-782 / 806-808, in the producer)
  float eps = 0.f;
  // Q5_K weights: dot against the input quantized to Q8_K (matmul_into's
  // route, src/model/mod.rs:381-394) instead of the float dot (dot_row,
  // the route of CpuBackend::matmul_dequant and ffn_gate_up).
  bool q8k = false;
  // Quad-layout launches of one matrix: each block also writes the first
  // maximum of its rows of y (value, row) to amax_v / amax_i[block]
  // (greedy argmax, sampler.rs:120-131); null: off.
  float *amax_v = nullptr;
  int *amax_i = nullptr;
  // One-matrix MV_X launches with at least two quads per row: if set, the
  // blocks split each row's K range in two (quads [0, ts) and [ts, T)), so
  // that a block stages half of x; half 0 writes res + W_0 . x to y, half 1
  // writes W_1 . x here (no residual) and the consumer adds the two.
  float *y2 = nullptr;
};

// Whether a matvec of this weight can take MvIn::y2 (two quads per row).
inline bool mv_ksplit_ok(int units) { return (units + 3) / 4 >= 2; }

struct MvArgs {
  MvIn in;
  const uint32_t *grid;  // IQ3_XXS codebook (device)
  int fmt, k, units, chunks;
  int part_floats;       // LDS floats of per-unit partial sums per block
  int blocks;
  int pair;              // 1: seg[0] = gate, seg[1] = up (same shape); y0 = silu(g) * u
  int nseg;
  int groups;            // quad layout: 16-row groups of all segments (seg[i].blk_begin
                         // is then the first of segment i)
  int ksplit;            // in.y2: the first quad of half 1 (0: no split)
  int blocks0;           // in.y2: blocks [0, blocks0) run half 0, the rest half 1
  MvSeg seg[MV_MAX_SEG];
};

// MoE expert FFN (router; gate/up with the SwiGLU; down with the combine).
struct MoeArgs {
  int fmt;
  int n_experts, top_k, h, f;       // hidden h, expert intermediate f
  const uint8_t *gate, *up, *down;  // stacked expert matrices, one tile per expert
  const uint16_t *gate_d, *up_d, *down_d;
  int units_h, units_f;
  int cus;                          // compute units (grid sizing)
  int bpp, bpt;                     // blocks per (token, slot) pair / per token
  int part_h, part_f;               // LDS floats of partial sums per block
  const uint32_t *grid;
  const float *logits;              // [T][n_experts]
  const float *x;                   // [T][h]
  int *ids;                         // [T][top_k]
  float *w;                         // [T][top_k]
  float *hbuf;                      // [T*top_k][f] silu(gate . x) * (up . x)
  float *out;                       // [T][h]
  int quad_gu, quad_dn;             // gate/up, down in the quad layout (MFMA kernels)
  int lds_gu, lds_dn;               // dynamic LDS bytes of the two stages' blocks
};

constexpr int MOE_ROUTE_MAX = 1024;  // experts routed inside the gate/up kernel

// LDS bytes of the MoE kernels' blocks for this shape (<= 160 KiB to run).
size_t moe_lds_bytes(int fmt, int h, int f, int top_k, int T, int cus, bool quad_gu, bool quad_dn);
hipError_t launch_moe(const MoeArgs &a, int T, hipStream_t st);

// LDS bytes of a matvec block: x limbs, records, codebook and part_total
// floats of partial sums.
size_t matvec_lds_bytes(int dtype, int units, int part_total);
// The MFMA matvec over quad-layout weights (Q4_K, Q5_K, Q6_K, Q8_0): plan
// (returns the LDS bytes of a block) and launch.
size_t mvq_plan(MvArgs &a, int num_cus);
hipError_t launch_mvq(const MvArgs &a, size_t lds, hipStream_t st);
// Static LDS bytes (a bound) a quad-layout kernel's block adds to the plan's.
size_t mvq_static_lds(int fmt);
// The MFMA MoE stages over quad-layout experts (stage 1: gate/up with the
// SwiGLU, routing inside when route; stage 2: down with the weighted
// combine): plan (sets bpp or bpt, part and lds fields; returns the LDS
// bytes of a block, static included) and launch.
size_t mvq_moe_plan(MoeArgs &a, int T, int stage, int num_cus);
hipError_t launch_mvq_moe(const MoeArgs &a, int T, int stage, bool route, hipStream_t st);

// Decode step state in device memory (advanced by the argmax kernel).
struct DecodeState {
  int token, pos, step, pad;
};

// Everything one decode step launches with (host struct, device pointers).
struct DecodeLaunch {
  int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, ctx;
  int att_chunks, max_tokens;
  float eps, theta;
  const gq_weight *const *wq, *const *wk, *const *wv, *const *wo;
  const gq_weight *const *wgate, *const *wup, *const *wdown;
  const gq_weight *lm_head;
  const float *const *attn_norm, *const *ffn_norm;  // host arrays of device pointers
  const float *output_norm, *embd;
  uint16_t *kcache, *vcache;  // [layer][ctx][kv_dim] f16 (kv_q8: int8 codes)
  int kv_q8;                  // KvDtype::Q8_0 cache
  uint16_t *kscale, *vscale;  // kv_q8: [layer][ctx][kv_dim / 32] f16 block scales
  float *xa, *xb;             // residual stream, ping-pong
  float *xc;                  // residual stream x_b + proj of the split down launch
  float *q, *k, *v, *att, *proj, *h, *logits, *att_part;
  float *rope_den;            // [head_dim / 2] theta^(2i/head_dim), computed on the host
  float *amax_v;              // per-block argmax partials
  int *amax_i;
  DecodeState *state;
  int *tokens;                // [max_tokens] generated tokens
};

hipError_t launch_decode_step(const DecodeLaunch &m, hipStream_t s);

// Batched prefill (gq_prefill.hip): buffers for passes of up to
// PREFILL_MAX tokens.
constexpr int PREFILL_MAX = 512;
struct PrefillBufs {
  float *x;        // [n][hidden] residual stream
  float *q, *k, *v, *g, *u;
  float *part;     // GEMM K-split partials (prefill_part_floats)
  uint16_t *xb;    // GEMM X fragments [512][max(hidden, ffn, q_dim) rounded to 256] bf16
  uint16_t *xh;    // the down GEMM's X from the fused gate/up epilogue [512][ffn rounded to 256]
  int *tokens;     // [PREFILL_MAX]
  uint16_t *kf, *vf;  // Q8_0 KV cache: one layer's rows unpacked to f16 [ctx][kv_dim]
};
size_t prefill_part_floats(const DecodeLaunch &m, int nmax, int num_cus);
hipError_t launch_prefill(const DecodeLaunch &m, const PrefillBufs &b, const int *tokens_dev, int n,
                          int pos0, int num_cus, hipStream_t s);
constexpr int ATT_CHUNK = 64;    // positions per attention block
constexpr int ATT_MAX_CTX = 65536;
constexpr int ARGMAX_SLOTS = 1024;  // per-block partials of the fused head argmax
hipError_t launch_set_state(DecodeState *st, int token, int pos, hipStream_t s);

// Host-side launch of y_i = W_i . in for weights sharing dtype and in_dim;
// no argument checks.  With pair, ws = {gate, up} and ys[0] receives
// silu(gate . in) * (up . in).
hipError_t matvec_launch(const gq_weight *const *ws, int count, const MvIn &in, float *const *ys,
                         hipStream_t st, bool pair = false);
const uint32_t *device_grid();

// Rows per tile for a matrix (chosen at upload).

// Re-lay a ggml tensor already on the device into the wave-tiled layout.
hipError_t launch_repack(const Layout &L, const uint8_t *raw, uint8_t *body, uint16_t *d,
                         hipStream_t st);

// Bit-exact dequant of rows [row0, row0+nrows) into out[nrows][in_dim].
hipError_t launch_dequant(const gq_weight *w, const uint32_t *grid, int row0, int nrows,
                          float *out, hipStream_t st);

// Per-32 Q8 activation pack (KvDtype::Q8_0::pack).
hipError_t launch_quantize_q8_32(const float *x, long n, uint16_t *scale, int8_t *q,
                                 hipStream_t st);

// quantize_row_q8_k of x[n] (bit-identical to the reference).
hipError_t launch_quantize_row_q8k(const float *x, long n, float *d, int8_t *qs, int16_t *bsums,
                                   hipStream_t st);

// Prefill GEMM.
hipError_t launch_gemm(const gq_weight *w, const float *X, int n, float *Y, int mode,
                       void *workspace, size_t ws_bytes, int num_cus, hipStream_t st);
size_t gemm_workspace_bytes(const gq_weight *w, int n, int mode, int num_cus);
// The bf16 GEMM's per-stage weight records (Q4_K, Q6_K): their size, and
// their construction from the device's tiled body.
size_t gemm_records_bytes(const Layout &L);
hipError_t launch_gemm_records(const gq_weight *w, uint8_t *out, hipStream_t st);

// One matrix of a bf16 GEMM launch: Y [n][rows] (token-major), or with a K
// split the partial products part [ksplit][n][rows].
constexpr int GEMM_MAX_SEG = 3;
struct GemmSeg {
  const uint8_t *rec;  // stage records
  float *y;
  float *part;
  int rows;
  int tile_begin;      // first row tile of this matrix in the launch
};
struct GemmArgs {
  GemmSeg seg[GEMM_MAX_SEG];
  int nseg, ntiles, ksplit, n, kpad;
  const uint16_t *xb;  // X as bf16 MFMA fragments [npad/16][kpad/32][64 lanes][8]
  // pair (direct kernel, no K split): seg[0] = gate, seg[1] = up of one
  // shape; a block tile holds 80 rows of each, and the epilogue writes
  // silu(gate . x) * (up . x) as bf16 fragments hb (the next GEMM's X, hkpad
  // columns) instead of Y.
  int pair, hkpad;
  uint16_t *hb;
};
// X fragments must cover n rounded up to GEMM_NPAD (a multiple of the
// 256-token tile).
constexpr int GEMM_NPAD = 512;
// K split of a launch with this many row x token tiles and stages.
int gemm_ksplit(int tiles, int stages, int num_cus);
// Y_i (+)= W_i . X for count <= GEMM_MAX_SEG weights of one dtype (Q4_K or
// Q6_K) and in_dim, on X already in fragment form (xb, n tokens).  add: Y_i
// += (else =; an accumulating launch always splits K and adds in the
// reduction).  part: gemm_part_floats floats.
// defer (accumulating launches only): the reduction is left to the
// caller; *defer receives the K split whose partials part holds.
hipError_t launch_gemm_bf16(const gq_weight *const *ws, float *const *ys, int count,
                            const uint16_t *xb, int n, float *part, bool add, int num_cus,
                            hipStream_t st, int *defer = nullptr);
// The gate/up pair of the SwiGLU on the direct kernel: hb = bf16 fragments
// of silu(gate . X) * (up . X) ([npad/16][round_up(F, 256)/32][64][8], the
// next GEMM's X; zero past n and F).  hipErrorNotSupported when the batch
// takes the ring kernel (n <= 128) or the two differ in type or shape: the
// caller then runs launch_gemm_bf16 and its own SwiGLU.
hipError_t launch_gemm_bf16_swiglu(const gq_weight *gate, const gq_weight *up, const uint16_t *xb, int n,
                                   uint16_t *hb, int num_cus, hipStream_t st);
size_t gemm_part_floats(const gq_weight *const *ws, int count, int n, int num_cus, bool add);
// X fp32 [n][k] -> bf16 fragments (kpad = k rounded up to 256, npad = n
// rounded up to GEMM_NPAD, zero padding).
hipError_t launch_x_to_frag(const float *X, int n, int k, uint16_t *xb, hipStream_t st);

}  // namespace gq
