// gq_internal.h -- host/device structures shared by the gq translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

// The public handle (opaque in gq.h).
struct gq_weight {
  int dtype;
  int in_dim, out_dim;
  int nb;            // blocks per row
  long stride;       // device body bytes per row
  uint8_t *body;     // device body (layout per dtype, see gq_device.h)
  uint16_t *d;       // device per-block f16 scales, or nullptr
  size_t ggml_bytes; // size of the tensor in ggml block order
  int device;
};

namespace gq {

constexpr int MV_MAX_SEG = 4;

struct MvSeg {
  const uint8_t *body;
  const uint16_t *d;
  float *y;
  long stride;
  int row_begin;  // first global row of this segment
};

struct MvArgs {
  const float *x;
  const uint32_t *grid;  // IQ3_XXS codebook (device)
  int k, kpad, nb;
  int total_rows;
  int nseg;
  MvSeg seg[MV_MAX_SEG];
};

size_t matvec_lds_bytes(int kpad);
hipError_t launch_matvec(const MvArgs &a, int fmt, int num_cus, hipStream_t st);

// Re-lay a ggml tensor that is already on the device into the handle's
// device layout.
hipError_t launch_repack(int dtype, const uint8_t *raw, long rows, int nb, uint8_t *body,
                         uint16_t *d, hipStream_t st);

// Bit-exact dequant of rows [row0, row0+nrows) into out[nrows][in_dim].
hipError_t launch_dequant(const gq_weight *w, const uint32_t *grid, int row0, int nrows,
                          float *out, hipStream_t st);

// Per-32 Q8 activation pack (KvDtype::Q8_0::pack).
hipError_t launch_quantize_q8_32(const float *x, long n, uint16_t *scale, int8_t *q,
                                 hipStream_t st);

// Prefill GEMM.
hipError_t launch_gemm(const gq_weight *w, const float *X, int n, float *Y, int mode,
                       void *workspace, size_t ws_bytes, int num_cus, hipStream_t st);
size_t gemm_workspace_bytes(const gq_weight *w, int n, int mode);

}  // namespace gq
