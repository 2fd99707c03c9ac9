// gq_api.hip -- the C ABI of libgq.so (declared in include/gq.h).
//
// Host-side runtime of the HIP backend: device selection, resident weight
// handles (upload once, re-laid-out on the device), launch shims and the
// synchronous Backend::matmul_dequant mirror.  Errors are negative codes
// plus a per-thread message, mirroring GgufError::BackendError(String)
// (src/error.rs:4-42).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <algorithm>
#include <vector>

#include "../../include/gq.h"
#include "gq_device.h"
#include "gq_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIP_TRY(expr)                                                                \
  do {                                                                               \
    hipError_t e_ = (expr);                                                          \
    if (e_ != hipSuccess)                                                            \
      return fail(GQ_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));           \
  } while (0)

struct DeviceState {
  bool ready = false;
  int device = -1;
  int num_cus = 0;
  uint32_t *grid = nullptr;  // IQ3_XXS codebook, 256 u32 on the device
  uint32_t grid_host[256];
  // IQ3_XXS weights are accepted only once a codebook has been installed
  // with gq_set_iq3xxs_grid: the library does not ship ggml's iq3xxs_grid,
  // and a real IQ3_XXS tensor decoded with any other table is garbage.
  bool grid_installed = false;
};

std::mutex g_mu;
DeviceState g_dev;

// Workspace of gq_moe_ffn_noalloc: a file-scope device array (each GPU holds
// its own copy for the life of the process).  Host code never uses the
// array's name as an address: init_locked fetches the device address with
// hipGetSymbolAddress, once per device, into g_scratch_dev.
constexpr int MAX_DEVICES = 64;
static __device__ __align__(256) unsigned char scratch[GQ_MOE_NOALLOC_MAX_BYTES];
void *g_scratch_dev[MAX_DEVICES] = {};

// Placeholder IQ3_XXS codebook: ggml's magnitude alphabet
// {4,12,20,28,36,44,52,62}, four magnitudes per entry chosen by a fixed
// integer hash of the entry index.  Replaced by gq_set_iq3xxs_grid.
void default_grid(uint32_t *g) {
  static const uint8_t mags[8] = {4, 12, 20, 28, 36, 44, 52, 62};
  for (uint32_t i = 0; i < 256; i++) {
    uint32_t h = i * 0x9E3779B1u;
    h ^= h >> 15;
    uint32_t e = 0;
    for (int k = 0; k < 4; k++) e |= (uint32_t)mags[(h >> (3 * k)) & 7] << (8 * k);
    g[i] = e;
  }
}

int init_locked(int device) {
  if (g_dev.ready && g_dev.device == device) return GQ_OK;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
    return fail(GQ_ENODEV, "no HIP device available");
  if (device < 0 || device >= n) return fail(GQ_ENODEV, "device %d out of range (%d)", device, n);
  HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t p;
  HIP_TRY(hipGetDeviceProperties(&p, device));
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
    return fail(GQ_ENODEV, "device %d is %s, this library is built for gfx950", device,
                p.gcnArchName);
  if (device < MAX_DEVICES && !g_scratch_dev[device]) {
    void *ptr = nullptr;
    HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    g_scratch_dev[device] = ptr;
  }
  g_dev.device = device;
  g_dev.num_cus = p.multiProcessorCount;
  if (!g_dev.grid_installed) default_grid(g_dev.grid_host);
  if (!g_dev.grid) HIP_TRY(hipMalloc(&g_dev.grid, 1024));
  HIP_TRY(hipMemcpy(g_dev.grid, g_dev.grid_host, 1024, hipMemcpyHostToDevice));
  g_dev.ready = true;
  return GQ_OK;
}

int ensure_init() {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_dev.ready) return GQ_OK;
  int dev = 0;
  (void)hipGetDevice(&dev);
  return init_locked(dev);
}

bool supported(int t) {
  return t == gq::T_Q8_0 || t == gq::T_Q4_K || t == gq::T_Q5_K || t == gq::T_Q6_K ||
         t == gq::T_IQ3_XXS;
}

const char *type_name(int t) {
  switch (t) {
  case 0: return "F32";
  case 1: return "F16";
  case 8: return "Q8_0";
  case 12: return "Q4_K";
  case 13: return "Q5_K";
  case 14: return "Q6_K";
  case 18: return "IQ3_XXS";
  case 30: return "BF16";
  default: return "unknown";
  }
}

// LDS a matvec block over w (with pair, over w and a second matrix of its
// shape) needs.
size_t matvec_block_lds(const gq_weight *w, bool pair) {
  gq::MvArgs a{};
  a.fmt = w->L.dtype;
  a.units = w->L.units;
  a.pair = pair;
  a.nseg = 1;
  a.seg[0].rows = std::max(w->L.rows, 1);
  if (!w->L.quad) return SIZE_MAX;  // stacked experts (wave-tiled) take gq_moe_ffn
  a.nseg = pair ? 2 : 1;
  a.seg[1].rows = a.seg[0].rows;
  return gq::mvq_plan(a, g_dev.num_cus) + gq::mvq_static_lds(a.fmt);
}

int check_matvec(const gq_weight *w) {
  if (!w) return fail(GQ_EINVAL, "null weight handle");
  if (w->L.rt != std::max(w->L.rows, 1))
    return fail(GQ_EINVAL, "stacked expert tensors take gq_moe_ffn, not a matvec");
  if (matvec_block_lds(w, false) > 160 * 1024)
    return fail(GQ_EINVAL, "in_dim %d too large for the LDS-staged matvec", w->L.k);
  return GQ_OK;
}

int upload_common(int dtype, const void *src, bool src_on_device, size_t nbytes, int in_dim,
                  int out_dim, gq_weight **out, int rows_per_group = 0) {
  if (!out) return fail(GQ_EINVAL, "null output handle pointer");
  *out = nullptr;
  int rc = ensure_init();
  if (rc) return rc;
  if (!supported(dtype))
    return fail(GQ_EDTYPE, "matmul_dequant: unsupported dtype %s", type_name(dtype));
  if (dtype == gq::T_IQ3_XXS && !g_dev.grid_installed)
    return fail(GQ_EDTYPE,
                "IQ3_XXS: no codebook installed; call gq_set_iq3xxs_grid with ggml's iq3xxs_grid "
                "(or NULL for the built-in test codebook) before uploading IQ3_XXS tensors");
  if (in_dim <= 0 || out_dim < 0) return fail(GQ_EINVAL, "bad shape %d x %d", out_dim, in_dim);
  const int be = gq::block_elems(dtype);
  const int nb = (in_dim + be - 1) / be;
  const size_t row_bytes = (size_t)nb * gq::ggml_block_bytes(dtype);
  const size_t need = row_bytes * (size_t)out_dim;
  if (nbytes < need)
    return fail(GQ_ESHORT, "%s upload: need %zu bytes, have %zu", type_name(dtype), need, nbytes);
  if (out_dim > 0 && !src) return fail(GQ_EINVAL, "null weight data");

  gq_weight *w = new gq_weight();
  w->L.dtype = dtype;
  w->L.rows = out_dim;
  w->L.k = in_dim;
  w->L.units = (in_dim + 255) / 256;
  w->L.chunks = gq::unit_chunks(dtype);
  w->L.rt = std::max(out_dim, 1);  // one tile: the whole matrix
  // Dense matrices, and stacked expert tensors whose experts are whole row
  // groups of 16, take the quad layout of the MFMA kernels; other stacked
  // tensors the wave-tiled one.
  w->L.quad = rows_per_group == 0 || rows_per_group % gq::QROWS == 0;
  // Stacked expert tensors: one tile per expert.
  if (rows_per_group > 0) w->L.rt = rows_per_group;
  w->ggml_bytes = need;
  w->device = g_dev.device;
  const size_t body = (size_t)gq::body_bytes(w->L);
  const bool has_d = dtype == gq::T_Q6_K || dtype == gq::T_IQ3_XXS;
  const size_t d_bytes = has_d ? (size_t)w->L.rows * w->L.units * 2 : 0;
  const size_t d_off = (body + 255) & ~(size_t)255;
  uint8_t *mem = nullptr;
  if (hipMalloc(&mem, d_off + d_bytes + 256) != hipSuccess) {
    delete w;
    return fail(GQ_ENOMEM, "hipMalloc of %zu bytes failed", d_off + d_bytes);
  }
  w->body = mem;
  w->d = d_bytes ? (uint16_t *)(mem + d_off) : nullptr;
  hipError_t e = hipSuccess;
  if (need) {
    const uint8_t *raw = (const uint8_t *)src;
    uint8_t *tmp = nullptr;
    if (!src_on_device) {
      e = hipMalloc(&tmp, need);
      if (e == hipSuccess) e = hipMemcpy(tmp, src, need, hipMemcpyHostToDevice);
      raw = tmp;
    }
    if (e == hipSuccess) e = gq::launch_repack(w->L, raw, w->body, w->d, 0);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (tmp) (void)hipFree(tmp);
  }
  if (e != hipSuccess) {
    (void)hipFree(mem);
    delete w;
    return fail(GQ_EHIP, "weight upload failed: %s", hipGetErrorString(e));
  }
  *out = w;
  return GQ_OK;
}

}  // namespace

namespace gq {
// Launch y_i = W_i . x for weights sharing dtype and in_dim (4 per launch).
// With xu != nullptr the input is silu(xg) * xu instead of x.
hipError_t matvec_launch(const gq_weight *const *ws, int count, const MvIn &in, float *const *ys,
                         hipStream_t st, bool pair) {
  const gq_weight *w0 = ws[0];
  if (pair) {  // {gate, up}: gate rows split over the blocks, up streamed alongside
    if (count != 2) return hipErrorInvalidValue;
    if (w0->L.rows == 0) return hipSuccess;
    MvArgs a{};
    a.in = in;
    a.grid = g_dev.grid;
    a.fmt = w0->L.dtype;
    a.k = w0->L.k;
    a.units = w0->L.units;
    a.chunks = w0->L.chunks;
    a.pair = 1;
    a.nseg = 2;
    a.seg[0] = MvSeg{w0->body, w0->d, ys[0], w0->L.rows, 0, 0};
    a.seg[1] = MvSeg{ws[1]->body, ws[1]->d, nullptr, ws[1]->L.rows, 0, 0};
    if (!w0->L.quad) return hipErrorInvalidValue;  // matvec weights are quad-layout
    return launch_mvq(a, mvq_plan(a, g_dev.num_cus), st);
  }
  for (int base = 0; base < count; base += MV_MAX_SEG) {
    MvArgs a{};
    a.in = in;
    a.grid = g_dev.grid;
    a.fmt = w0->L.dtype;
    a.k = w0->L.k;
    a.units = w0->L.units;
    a.chunks = w0->L.chunks;
    int ns = 0;
    for (int i = base; i < count && i < base + MV_MAX_SEG; i++) {
      const gq_weight *w = ws[i];
      if (w->L.rows == 0) continue;
      a.seg[ns++] = MvSeg{w->body, w->d, ys[i], w->L.rows, 0, 0};
    }
    if (ns == 0) continue;
    a.nseg = ns;
    if (!w0->L.quad) return hipErrorInvalidValue;  // matvec weights are quad-layout
    const hipError_t e = launch_mvq(a, mvq_plan(a, g_dev.num_cus), st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

const uint32_t *device_grid() { return g_dev.grid; }
}  // namespace gq

extern "C" {

int gq_init(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  return init_locked(device);
}

const char *gq_backend_name(void) { return "hip"; }

const char *gq_last_error(void) { return g_err.c_str(); }

size_t gq_type_size(int dtype, size_t n) {
  const int bb = gq::ggml_block_bytes(dtype);
  if (!bb) return 0;
  const size_t be = gq::block_elems(dtype);
  return ((n + be - 1) / be) * bb;
}

int gq_upload(int dtype, const void *w_host, size_t nbytes, int in_dim, int out_dim,
              gq_weight **out) {
  return upload_common(dtype, w_host, false, nbytes, in_dim, out_dim, out);
}

int gq_upload_device(int dtype, const void *w_dev, size_t nbytes, int in_dim, int out_dim,
                     gq_weight **out) {
  return upload_common(dtype, w_dev, true, nbytes, in_dim, out_dim, out);
}

int gq_upload_experts(int dtype, const void *w_host, size_t nbytes, int in_dim,
                      int rows_per_expert, int n_experts, gq_weight **out) {
  if (rows_per_expert <= 0 || n_experts <= 0)
    return fail(GQ_EINVAL, "bad expert shape %d x %d", n_experts, rows_per_expert);
  return upload_common(dtype, w_host, false, nbytes, in_dim, rows_per_expert * n_experts, out,
                       rows_per_expert);
}

}  // extern "C"

namespace {
// True while st is recording a HIP graph: nothing may allocate, free or
// synchronize on it then.
bool stream_capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// The workspace of gq_gemm (the packed X) and gq_moe_ffn (the SwiGLU
// outputs and routing), kept per (device, stream) and grown on demand:
// calls on one stream are ordered, so they can share it.  A buffer that a
// larger call supersedes is never freed (a graph captured earlier may still
// address it), so every workspace is held until the process ends.  Under
// stream capture the workspace cannot grow: the call is refused.
struct StreamWs {
  int dev;
  hipStream_t st;
  void *p;
  size_t bytes;
};
std::vector<StreamWs> g_stream_ws;  // guarded by g_mu
std::vector<void *> g_retired_ws;   // superseded workspaces, guarded by g_mu

int stream_workspace(hipStream_t st, size_t bytes, void **out) {
  std::lock_guard<std::mutex> lk(g_mu);
  int dev = 0;
  (void)hipGetDevice(&dev);
  StreamWs *ws = nullptr;
  for (StreamWs &w : g_stream_ws)
    if (w.dev == dev && w.st == st) ws = &w;
  if (ws && ws->bytes >= bytes) {
    *out = ws->p;
    return GQ_OK;
  }
  if (stream_capturing(st))
    return fail(GQ_EINVAL,
                "stream workspace of %zu bytes needed under graph capture (the stream holds %zu): "
                "make one call of at least this size on the stream before capturing",
                bytes, ws ? ws->bytes : (size_t)0);
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess)
    return fail(GQ_ENOMEM, "workspace of %zu bytes: hipMalloc failed", bytes);
  if (ws) {
    g_retired_ws.push_back(ws->p);
    ws->p = p;
    ws->bytes = bytes;
  } else {
    g_stream_ws.push_back(StreamWs{dev, st, p, bytes});
  }
  *out = p;
  return GQ_OK;
}
}  // namespace

namespace {
// gq_moe_ffn and its no-allocation variant: with noalloc the workspace is
// the device's scratch array (sizes above GQ_MOE_NOALLOC_MAX_BYTES are
// refused), otherwise the stream's cached workspace.
int moe_ffn(const gq_weight *gate, const gq_weight *up, const gq_weight *down, int n_experts,
            const float *logits_dev, int T, int top_k, const float *x_dev, float *out_dev,
            int *ids_dev, float *w_dev, void *stream, bool noalloc) {
  int rc = ensure_init();
  if (rc) return rc;
  if (!gate || !up || !down) return fail(GQ_EINVAL, "null expert weight handle");
  if (T < 0 || n_experts <= 0 || n_experts > 4096 || top_k <= 0 || top_k > n_experts || top_k > 64)
    return fail(GQ_EINVAL, "bad MoE shape T=%d experts=%d top_k=%d", T, n_experts, top_k);
  if (T == 0) return GQ_OK;
  const int h = gate->L.k, f = down->L.k;
  if (gate->L.dtype != up->L.dtype || gate->L.dtype != down->L.dtype)
    return fail(GQ_EINVAL, "expert tensors must share one dtype");
  if (up->L.k != h || gate->L.rows != n_experts * f || up->L.rows != n_experts * f ||
      down->L.rows != n_experts * h)
    return fail(GQ_EINVAL, "expert shapes disagree: gate %dx%d up %dx%d down %dx%d, experts %d",
                gate->L.rows, gate->L.k, up->L.rows, up->L.k, down->L.rows, down->L.k, n_experts);
  if (gate->L.rt != f || up->L.rt != f || down->L.rt != h)
    return fail(GQ_EINVAL, "expert tensors must be uploaded with gq_upload_experts");
  if (!logits_dev || !x_dev || !out_dev) return fail(GQ_EINVAL, "null MoE buffer");
  if (gate->L.quad != up->L.quad)
    return fail(GQ_EINVAL, "gate and up expert tensors must share one layout");
  if (gq::moe_lds_bytes(gate->L.dtype, h, f, top_k, T, g_dev.num_cus, gate->L.quad, down->L.quad) >
      160 * 1024)
    return fail(GQ_EINVAL, "MoE shape h %d f %d top_k %d too large for the LDS-staged kernels", h, f,
                top_k);
  const int pairs = T * top_k;
  const size_t ws = (size_t)pairs * (size_t)f * 4 + (size_t)pairs * 8 + 1024;
  char *wsp = nullptr;
  if (noalloc) {
    if (ws > GQ_MOE_NOALLOC_MAX_BYTES)
      return fail(GQ_EINVAL,
                  "gq_moe_ffn_noalloc: workspace of %zu bytes (T=%d top_k=%d f=%d) exceeds the %d-byte "
                  "scratch; use gq_moe_ffn",
                  ws, T, top_k, f, GQ_MOE_NOALLOC_MAX_BYTES);
    if (g_dev.device < 0 || g_dev.device >= MAX_DEVICES || !g_scratch_dev[g_dev.device])
      return fail(GQ_ENODEV, "gq_moe_ffn_noalloc: no scratch on device %d", g_dev.device);
    wsp = (char *)g_scratch_dev[g_dev.device];
  } else if ((rc = stream_workspace((hipStream_t)stream, ws, (void **)&wsp))) {
    return rc;
  }
  gq::MoeArgs a{};
  a.fmt = gate->L.dtype;
  a.n_experts = n_experts;
  a.top_k = top_k;
  a.h = h;
  a.f = f;
  a.gate = gate->body; a.up = up->body; a.down = down->body;
  a.gate_d = gate->d; a.up_d = up->d; a.down_d = down->d;
  a.units_h = gate->L.units;
  a.units_f = down->L.units;
  a.cus = g_dev.num_cus;
  a.grid = g_dev.grid;
  a.logits = logits_dev;
  a.x = x_dev;
  a.hbuf = (float *)wsp;
  a.ids = ids_dev ? ids_dev : (int *)(a.hbuf + (size_t)pairs * f);
  a.w = w_dev ? w_dev : (float *)((int *)(a.hbuf + (size_t)pairs * f) + pairs);
  a.out = out_dev;
  a.quad_gu = gate->L.quad;
  a.quad_dn = down->L.quad;
  hipError_t e = gq::launch_moe(a, T, (hipStream_t)stream);
  if (e != hipSuccess) return fail(GQ_EHIP, "MoE launch failed: %s", hipGetErrorString(e));
  return GQ_OK;
}
}  // namespace

extern "C" {
int gq_moe_ffn(const gq_weight *gate, const gq_weight *up, const gq_weight *down, int n_experts,
               const float *logits_dev, int T, int top_k, const float *x_dev, float *out_dev,
               int *ids_dev, float *w_dev, void *stream) {
  return moe_ffn(gate, up, down, n_experts, logits_dev, T, top_k, x_dev, out_dev, ids_dev, w_dev,
                 stream, false);
}

int gq_moe_ffn_noalloc(const gq_weight *gate, const gq_weight *up, const gq_weight *down,
                       int n_experts, const float *logits_dev, int T, int top_k, const float *x_dev,
                       float *out_dev, int *ids_dev, float *w_dev, void *stream) {
  return moe_ffn(gate, up, down, n_experts, logits_dev, T, top_k, x_dev, out_dev, ids_dev, w_dev,
                 stream, true);
}

int gq_weight_free(gq_weight *w) {
  if (!w) return GQ_OK;
  if (w->body) (void)hipFree(w->body);
  if (w->gemm_raw) (void)hipFree(w->gemm_raw);
  delete w;
  return GQ_OK;
}

int gq_weight_shape(const gq_weight *w, int *dtype, int *in_dim, int *out_dim) {
  if (!w) return fail(GQ_EINVAL, "null weight handle");
  if (dtype) *dtype = w->L.dtype;
  if (in_dim) *in_dim = w->L.k;
  if (out_dim) *out_dim = w->L.rows;
  return GQ_OK;
}

size_t gq_weight_bytes(const gq_weight *w) { return w ? w->ggml_bytes : 0; }

}  // extern "C"

namespace {
// y_i = W_i . x for weights sharing dtype and in_dim; q8k selects the
// Q8_K route for Q5_K weights.
int matvec_multi(const gq_weight *const *ws, int count, const float *x_dev, float *const *y_dev,
                 void *stream, bool q8k) {
  int rc = ensure_init();
  if (rc) return rc;
  if (count <= 0 || !ws || !y_dev) return fail(GQ_EINVAL, "empty weight list");
  for (int i = 0; i < count; i++) {
    if ((rc = check_matvec(ws[i]))) return rc;
    if (ws[i]->L.dtype != ws[0]->L.dtype || ws[i]->L.k != ws[0]->L.k)
      return fail(GQ_EINVAL, "gq_matvec_multi: weights must share dtype and in_dim");
    if (ws[i]->L.rows > 0 && !y_dev[i]) return fail(GQ_EINVAL, "null output %d", i);
  }
  if (!x_dev) return fail(GQ_EINVAL, "null x");
  gq::MvIn in;
  in.x = x_dev;
  in.q8k = q8k;
  hipError_t e = gq::matvec_launch(ws, count, in, y_dev, (hipStream_t)stream);
  if (e != hipSuccess) return fail(GQ_EHIP, "matvec launch failed: %s", hipGetErrorString(e));
  return GQ_OK;
}
}  // namespace

extern "C" {
int gq_matvec_multi(const gq_weight *const *ws, int count, const float *x_dev,
                    float *const *y_dev, void *stream) {
  return matvec_multi(ws, count, x_dev, y_dev, stream, true);
}

int gq_matvec(const gq_weight *w, const float *x_dev, float *y_dev, void *stream) {
  const gq_weight *ws[1] = {w};
  float *ys[1] = {y_dev};
  return matvec_multi(ws, 1, x_dev, ys, stream, true);
}

int gq_matmul_dequant_preloaded(const gq_weight *w, const float *x_host, float *out_host) {
  int rc = ensure_init();
  if (rc) return rc;
  if ((rc = check_matvec(w))) return rc;
  if (w->L.rows == 0) return GQ_OK;
  if (!x_host || !out_host) return fail(GQ_EINVAL, "null x or out");
  float *xd = nullptr, *yd = nullptr;
  HIP_TRY(hipMalloc(&xd, (size_t)w->L.k * 4));
  if (hipMalloc(&yd, (size_t)w->L.rows * 4) != hipSuccess) {
    (void)hipFree(xd);
    return fail(GQ_ENOMEM, "hipMalloc failed");
  }
  hipError_t e = hipMemcpy(xd, x_host, (size_t)w->L.k * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    // the float dot of every type, Q5_K included (matmul_dequant_preloaded
    // runs the per-format dequant-dot kernels, wgpu_backend/mod.rs:642-696,
    // like CpuBackend::matmul_dequant's dot_row)
    const gq_weight *ws[1] = {w};
    float *ys[1] = {yd};
    rc = matvec_multi(ws, 1, xd, ys, nullptr, false);
    if (!rc) e = hipMemcpy(out_host, yd, (size_t)w->L.rows * 4, hipMemcpyDeviceToHost);
  }
  (void)hipFree(xd);
  (void)hipFree(yd);
  if (rc) return rc;
  if (e != hipSuccess) return fail(GQ_EHIP, "copy failed: %s", hipGetErrorString(e));
  return GQ_OK;
}

int gq_matmul_dequant_host(int dtype, const void *w_host, size_t nbytes, const float *x_host,
                           size_t in_dim, float *out_host, size_t out_dim) {
  if (!supported(dtype) || dtype == gq::T_IQ3_XXS)
    // Backend::matmul_dequant accepts the GPU_DEQUANT_DTYPES (ops/mod.rs:27-28).
    return fail(GQ_EDTYPE, "matmul_dequant: unsupported dtype %s", type_name(dtype));
  if (out_dim == 0) return GQ_OK;
  gq_weight *w = nullptr;
  int rc = gq_upload(dtype, w_host, nbytes, (int)in_dim, (int)out_dim, &w);
  if (rc) return rc;
  rc = gq_matmul_dequant_preloaded(w, x_host, out_host);
  gq_weight_free(w);
  return rc;
}

int gq_dequant_rows(const gq_weight *w, int row0, int nrows, float *out_dev, void *stream) {
  int rc = ensure_init();
  if (rc) return rc;
  if (!w) return fail(GQ_EINVAL, "null weight handle");
  if (row0 < 0 || nrows < 0 || row0 + nrows > w->L.rows)
    return fail(GQ_EINVAL, "row index %d out of range (tensor has %d rows)", row0 + nrows - 1,
                w->L.rows);
  if (nrows == 0) return GQ_OK;
  hipError_t e = gq::launch_dequant(w, g_dev.grid, row0, nrows, out_dev, (hipStream_t)stream);
  if (e != hipSuccess) return fail(GQ_EHIP, "dequant launch failed: %s", hipGetErrorString(e));
  return GQ_OK;
}

int gq_dequant_rows_host(const gq_weight *w, int row0, int nrows, float *out_host) {
  int rc = ensure_init();
  if (rc) return rc;
  if (!w) return fail(GQ_EINVAL, "null weight handle");
  if (row0 < 0 || nrows < 0 || row0 + nrows > w->L.rows)
    return fail(GQ_EINVAL, "row index %d out of range (tensor has %d rows)", row0 + nrows - 1,
                w->L.rows);
  if (nrows == 0) return GQ_OK;
  if (!out_host) return fail(GQ_EINVAL, "null out");
  // Rows in batches of at most 64 MiB of f32 through one device buffer.
  const int per = std::max(1, (int)std::min<long>(nrows, (64l << 20) / (4l * w->L.k)));
  float *buf = nullptr;
  HIP_TRY(hipMalloc(&buf, (size_t)per * w->L.k * 4));
  hipError_t e = hipSuccess;
  for (int r = 0; r < nrows && e == hipSuccess; r += per) {
    const int n = std::min(per, nrows - r);
    e = gq::launch_dequant(w, g_dev.grid, row0 + r, n, buf, nullptr);
    if (e == hipSuccess)
      e = hipMemcpy(out_host + (size_t)r * w->L.k, buf, (size_t)n * w->L.k * 4,
                    hipMemcpyDeviceToHost);
  }
  (void)hipFree(buf);
  if (e != hipSuccess) return fail(GQ_EHIP, "dequant failed: %s", hipGetErrorString(e));
  return GQ_OK;
}

int gq_quantize_q8_32(const float *x_dev, int n, uint16_t *scale_dev, int8_t *q_dev,
                      void *stream) {
  int rc = ensure_init();
  if (rc) return rc;
  if (n < 0 || n % 32) return fail(GQ_EINVAL, "n=%d must be a multiple of 32", n);
  hipError_t e = gq::launch_quantize_q8_32(x_dev, n, scale_dev, q_dev, (hipStream_t)stream);
  if (e != hipSuccess) return fail(GQ_EHIP, "quantize launch failed: %s", hipGetErrorString(e));
  return GQ_OK;
}

int gq_quantize_row_q8k(const float *x_dev, int n, float *d_dev, int8_t *qs_dev,
                        int16_t *bsums_dev, void *stream) {
  int rc = ensure_init();
  if (rc) return rc;
  if (n < 0) return fail(GQ_EINVAL, "negative length %d", n);
  if (n == 0) return GQ_OK;
  if (!x_dev || !d_dev || !qs_dev || !bsums_dev) return fail(GQ_EINVAL, "null Q8_K buffer");
  hipError_t e = gq::launch_quantize_row_q8k(x_dev, n, d_dev, qs_dev, bsums_dev, (hipStream_t)stream);
  if (e != hipSuccess) return fail(GQ_EHIP, "quantize launch failed: %s", hipGetErrorString(e));
  return GQ_OK;
}

int gq_set_iq3xxs_grid(const uint32_t *grid_host) {
  int rc = ensure_init();
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  if (grid_host) {
    // magnitudes enter signed 8-bit dot products, negated bytewise:
    // each byte must be in 1..127 (ggml's codebook uses 4..62)
    for (int i = 0; i < 256; i++) {
      const uint32_t g = grid_host[i];
      if ((g & 0x80808080u) || !(g & 0xffu) || !(g & 0xff00u) || !(g & 0xff0000u) ||
          !(g & 0xff000000u))
        return fail(GQ_EINVAL, "IQ3_XXS grid entry %d has a magnitude byte outside 1..127", i);
    }
    memcpy(g_dev.grid_host, grid_host, 1024);
  }
  else default_grid(g_dev.grid_host);
  HIP_TRY(hipMemcpy(g_dev.grid, g_dev.grid_host, 1024, hipMemcpyHostToDevice));
  g_dev.grid_installed = true;
  return GQ_OK;
}

int gq_get_iq3xxs_grid(uint32_t *grid_host) {
  int rc = ensure_init();
  if (rc) return rc;
  if (!grid_host) return fail(GQ_EINVAL, "null grid");
  memcpy(grid_host, g_dev.grid_host, 1024);
  return GQ_OK;
}

// The bf16 GEMM streams per-stage records of a weight (made once, on first
// use, from the tiled body).
static int gq_ensure_gemm_records(const gq_weight *w, hipStream_t stream) {
  if (w->gemm_raw) return GQ_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  if (w->gemm_raw) return GQ_OK;
  if (stream_capturing(stream))
    return fail(GQ_EINVAL,
                "gq_gemm: the first call on a weight builds its GEMM records and must not be "
                "made under graph capture");
  uint8_t *rec = nullptr;
  const size_t bytes = gq::gemm_records_bytes(w->L);
  if (hipMalloc(&rec, bytes) != hipSuccess)
    return fail(GQ_ENOMEM, "hipMalloc of %zu bytes (GEMM weight records) failed", bytes);
  hipError_t e = gq::launch_gemm_records(w, rec, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    (void)hipFree(rec);
    return fail(GQ_EHIP, "GEMM weight records failed: %s", hipGetErrorString(e));
  }
  const_cast<gq_weight *>(w)->gemm_raw = rec;
  return GQ_OK;
}

}  // extern "C"


extern "C" {
int gq_gemm(const gq_weight *w, const float *X_dev, int n, float *Y_dev, int mode,
            void *stream) {
  int rc = ensure_init();
  if (rc) return rc;
  if (!w) return fail(GQ_EINVAL, "null weight handle");
  if (n < 0) return fail(GQ_EINVAL, "negative batch");
  if (n == 0 || w->L.rows == 0) return GQ_OK;
  if (mode != GQ_GEMM_BF16 && mode != GQ_GEMM_INT8) return fail(GQ_EINVAL, "bad gemm mode %d", mode);
  const size_t ws = gq::gemm_workspace_bytes(w, n, mode, g_dev.num_cus);
  if (ws == (size_t)-1)
    return fail(GQ_EDTYPE, "gq_gemm: %s weights not supported in %s mode", type_name(w->L.dtype),
                mode == GQ_GEMM_BF16 ? "bf16" : "int8");
  {
    int rc2 = gq_ensure_gemm_records(w, (hipStream_t)stream);  // both modes read the ggml-order copy
    if (rc2) return rc2;
  }
  void *wsp = nullptr;
  if (ws && (rc = stream_workspace((hipStream_t)stream, ws, &wsp))) return rc;
  hipError_t e = gq::launch_gemm(w, X_dev, n, Y_dev, mode, wsp, ws, g_dev.num_cus,
                                 (hipStream_t)stream);
  if (e != hipSuccess) return fail(GQ_EHIP, "gemm launch failed: %s", hipGetErrorString(e));
  return GQ_OK;
}

// ------------------------------------------------------------ decode model
}  // extern "C"

struct gq_model {
  gq::DecodeLaunch L;
  std::vector<const gq_weight *> wq, wk, wv, wo, wg, wu, wd;
  std::vector<const float *> an, fn;
  std::vector<void *> owned;  // device allocations
  hipGraphExec_t graph = nullptr;
  hipStream_t graph_stream = nullptr;
  gq::PrefillBufs pf{};  // allocated by the first prefill
  ~gq_model() {
    if (graph) (void)hipGraphExecDestroy(graph);
    for (void *p : owned) (void)hipFree(p);
  }
};

namespace {
template <typename T>
int dalloc(gq_model *m, T **p, size_t count) {
  void *q = nullptr;
  if (hipMalloc(&q, count * sizeof(T) + 256) != hipSuccess)
    return fail(GQ_ENOMEM, "hipMalloc of %zu bytes failed", count * sizeof(T));
  m->owned.push_back(q);
  *p = (T *)q;
  return GQ_OK;
}

int check_w(const gq_weight *w, int rows, int k, const char *what, int layer) {
  if (!w) return fail(GQ_EINVAL, "layer %d: null %s", layer, what);
  if (w->L.rows != rows || w->L.k != k)
    return fail(GQ_EINVAL, "layer %d: %s is %dx%d, expected %dx%d", layer, what, w->L.rows,
                w->L.k, rows, k);
  return check_matvec(w);
}
}  // namespace

extern "C" {

int gq_model_create(const gq_model_desc *d, gq_model **out) {
  if (!d || !out) return fail(GQ_EINVAL, "null model descriptor");
  *out = nullptr;
  int rc = ensure_init();
  if (rc) return rc;
  const int H = d->hidden, hd = d->head_dim, nh = d->n_heads, nkv = d->n_kv_heads;
  if (d->n_layers <= 0 || H <= 0 || H % 4 || (hd != 64 && hd != 128) || nh <= 0 || nkv <= 0 ||
      nh % nkv || nh / nkv > 8 || d->ffn <= 0 || d->vocab <= 0 || d->ctx <= 0 ||
      d->ctx > gq::ATT_MAX_CTX ||
      (d->kv_dtype != 0 && d->kv_dtype != GQ_TYPE_F16 && d->kv_dtype != GQ_TYPE_Q8_0) ||
      (d->kv_dtype == GQ_TYPE_Q8_0 && (nkv * hd) % 32))
    return fail(GQ_EINVAL, "bad model shape (hidden a multiple of 4, head_dim 64 or 128, "
                           "n_heads a multiple of n_kv_heads with at most 8 query heads per KV "
                           "head, ctx <= %d, KV type F16 or Q8_0)", gq::ATT_MAX_CTX);
  for (int l = 0; l < d->n_layers; l++) {
    if ((rc = check_w(d->wq[l], nh * hd, H, "wq", l)) || (rc = check_w(d->wk[l], nkv * hd, H, "wk", l)) ||
        (rc = check_w(d->wv[l], nkv * hd, H, "wv", l)) || (rc = check_w(d->wo[l], H, nh * hd, "wo", l)) ||
        (rc = check_w(d->wgate[l], d->ffn, H, "ffn_gate", l)) ||
        (rc = check_w(d->wup[l], d->ffn, H, "ffn_up", l)) ||
        (rc = check_w(d->wdown[l], H, d->ffn, "ffn_down", l)))
      return rc;
    if (d->wgate[l]->L.dtype != d->wup[l]->L.dtype)
      return fail(GQ_EINVAL, "layer %d: ffn_gate and ffn_up must share a dtype", l);
    const gq_weight *g = d->wgate[l];
    if (d->wup[l]->L.rows != g->L.rows || matvec_block_lds(g, true) > 160 * 1024)
      return fail(GQ_EINVAL, "layer %d: ffn_gate/ffn_up layouts do not pair", l);
  }
  if ((rc = check_w(d->lm_head, d->vocab, H, "output", -1))) return rc;
  gq_model *m = new gq_model();
  auto &L = m->L;
  L.n_layers = d->n_layers; L.hidden = H; L.n_heads = nh; L.n_kv_heads = nkv; L.head_dim = hd;
  L.ffn = d->ffn; L.vocab = d->vocab; L.ctx = d->ctx; L.eps = d->eps; L.theta = d->theta;
  L.att_chunks = (d->ctx + gq::ATT_CHUNK - 1) / gq::ATT_CHUNK;
  L.max_tokens = d->max_tokens > 0 ? d->max_tokens : 4096;
  for (int l = 0; l < d->n_layers; l++) {
    m->wq.push_back(d->wq[l]); m->wk.push_back(d->wk[l]); m->wv.push_back(d->wv[l]);
    m->wo.push_back(d->wo[l]); m->wg.push_back(d->wgate[l]); m->wu.push_back(d->wup[l]);
    m->wd.push_back(d->wdown[l]);
  }
  L.wq = m->wq.data(); L.wk = m->wk.data(); L.wv = m->wv.data(); L.wo = m->wo.data();
  L.wgate = m->wg.data(); L.wup = m->wu.data(); L.wdown = m->wd.data(); L.lm_head = d->lm_head;
  const size_t kvd = (size_t)nkv * hd;
  float *norms = nullptr, *embd = nullptr;
  rc = dalloc(m, &norms, (size_t)(2 * d->n_layers + 1) * H);
  if (!rc) rc = dalloc(m, &embd, (size_t)d->vocab * H);
  L.kv_q8 = d->kv_dtype == GQ_TYPE_Q8_0;
  // Q8_0: int8 codes in the first half of the f16-sized allocation
  if (!rc) rc = dalloc(m, &L.kcache, (size_t)d->n_layers * d->ctx * kvd / (L.kv_q8 ? 2 : 1) + 1);
  if (!rc) rc = dalloc(m, &L.vcache, (size_t)d->n_layers * d->ctx * kvd / (L.kv_q8 ? 2 : 1) + 1);
  if (!rc && L.kv_q8) rc = dalloc(m, &L.kscale, (size_t)d->n_layers * d->ctx * (kvd / 32));
  if (!rc && L.kv_q8) rc = dalloc(m, &L.vscale, (size_t)d->n_layers * d->ctx * (kvd / 32));
  float *buf = nullptr;
  const int nb_amax = gq::ARGMAX_SLOTS;
  const size_t nbuf = 4 * ((size_t)H + 16) + 2 * ((size_t)nh * hd + 16) + 2 * (kvd + 16) +
                      ((size_t)d->ffn + 16) + ((size_t)d->vocab + 16) +
                      ((size_t)nh * L.att_chunks * (2 + hd) + 16) + (nb_amax + 16) + (hd / 2 + 16);
  int *ibuf = nullptr;
  const size_t nibuf = (size_t)nb_amax;
  if (!rc) rc = dalloc(m, &buf, nbuf);
  if (!rc) rc = dalloc(m, &ibuf, nibuf);
  if (!rc) rc = dalloc(m, &L.state, 1);
  if (!rc) rc = dalloc(m, &L.tokens, (size_t)L.max_tokens);
  if (rc) { delete m; return rc; }
  size_t o = 0;
  auto take = [&](size_t n) { float *p = buf + o; o += (n + 15) & ~(size_t)15; return p; };
  L.xa = take(H); L.xb = take(H); L.xc = take(H); L.proj = take(H);
  L.q = take((size_t)nh * hd); L.att = take((size_t)nh * hd);
  L.k = take(kvd); L.v = take(kvd); L.h = take(d->ffn);
  L.logits = take(d->vocab); L.att_part = take((size_t)nh * L.att_chunks * (2 + hd));
  L.amax_v = take(nb_amax);
  L.rope_den = take(hd / 2);
  L.amax_i = ibuf;
  hipError_t e = hipSuccess;
  {  // argmax partial slots start neutral (-inf, INT_MAX): the fused head argmax
     // reads all ARGMAX_SLOTS, of which only the head's blocks write
    std::vector<float> nv((size_t)nb_amax, -INFINITY);
    std::vector<int> ni((size_t)nb_amax, 0x7fffffff);
    e = hipMemcpy(L.amax_v, nv.data(), nv.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(L.amax_i, ni.data(), ni.size() * 4, hipMemcpyHostToDevice);
  }
  for (int l = 0; l < d->n_layers && e == hipSuccess; l++) {
    e = hipMemcpy(norms + (size_t)(2 * l) * H, d->attn_norm[l], H * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess)
      e = hipMemcpy(norms + (size_t)(2 * l + 1) * H, d->ffn_norm[l], H * 4, hipMemcpyHostToDevice);
    m->an.push_back(norms + (size_t)(2 * l) * H);
    m->fn.push_back(norms + (size_t)(2 * l + 1) * H);
  }
  if (e == hipSuccess)
    e = hipMemcpy(norms + (size_t)2 * d->n_layers * H, d->output_norm, H * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(embd, d->embd, (size_t)d->vocab * H * 4, hipMemcpyHostToDevice);
  // RoPE: angle(pos, i) = pos / theta^(2i/hd), the divisor as the CPU path
  // computes it (cpu_path.rs:99-133).
  std::vector<float> den(hd / 2);
  for (int i = 0; i < hd / 2; i++) den[i] = powf(d->theta, 2.0f * (float)i / (float)hd);
  // counters of the last-block merges start (and end every launch) at zero
  if (e == hipSuccess) e = hipMemset(ibuf, 0, nibuf * sizeof(int));
  if (e == hipSuccess) e = hipMemset(buf, 0, nbuf * sizeof(float));
  if (e == hipSuccess) e = hipMemcpy(L.rope_den, den.data(), den.size() * 4, hipMemcpyHostToDevice);
  const size_t kv_bytes = (size_t)d->n_layers * d->ctx * kvd * (L.kv_q8 ? 1 : 2);
  if (e == hipSuccess) e = hipMemset(L.kcache, 0, kv_bytes);
  if (e == hipSuccess) e = hipMemset(L.vcache, 0, kv_bytes);
  if (e == hipSuccess && L.kv_q8) e = hipMemset(L.kscale, 0, (size_t)d->n_layers * d->ctx * (kvd / 32) * 2);
  if (e == hipSuccess && L.kv_q8) e = hipMemset(L.vscale, 0, (size_t)d->n_layers * d->ctx * (kvd / 32) * 2);
  if (e != hipSuccess) { delete m; return fail(GQ_EHIP, "model upload failed: %s", hipGetErrorString(e)); }
  L.attn_norm = m->an.data(); L.ffn_norm = m->fn.data();
  L.output_norm = norms + (size_t)2 * d->n_layers * H;
  L.embd = embd;
  *out = m;
  return GQ_OK;
}

int gq_model_free(gq_model *m) {
  delete m;
  return GQ_OK;
}

// KV rows in the cache's KvDtype byte format on the host; the device keeps
// Q8_0 as codes [ctx][kvd] and f16 scales [ctx][kvd / 32].
static int kv_copy(gq_model *m, int layer, void *k, void *v, int n_pos, bool up) {
  if (!m || layer < 0 || layer >= m->L.n_layers || n_pos < 0 || n_pos > m->L.ctx)
    return fail(GQ_EINVAL, "bad KV range (layer %d, %d positions)", layer, n_pos);
  if (n_pos > 0 && (!k || !v)) return fail(GQ_EINVAL, "null KV buffer");
  const size_t kvd = (size_t)m->L.n_kv_heads * m->L.head_dim;
  if (!m->L.kv_q8) {
    const size_t off = (size_t)layer * m->L.ctx * kvd, bytes = (size_t)n_pos * kvd * 2;
    hipError_t e = up ? hipMemcpy(m->L.kcache + off, k, bytes, hipMemcpyHostToDevice)
                      : hipMemcpy(k, m->L.kcache + off, bytes, hipMemcpyDeviceToHost);
    if (e == hipSuccess)
      e = up ? hipMemcpy(m->L.vcache + off, v, bytes, hipMemcpyHostToDevice)
             : hipMemcpy(v, m->L.vcache + off, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return fail(GQ_EHIP, "KV copy failed: %s", hipGetErrorString(e));
    return GQ_OK;
  }
  const size_t nb = kvd / 32, rows = (size_t)n_pos;
  std::vector<int8_t> codes(rows * kvd);
  std::vector<uint16_t> scales(rows * nb);
  void *host[2] = {k, v};
  int8_t *dq[2] = {(int8_t *)m->L.kcache + (size_t)layer * m->L.ctx * kvd,
                   (int8_t *)m->L.vcache + (size_t)layer * m->L.ctx * kvd};
  uint16_t *ds[2] = {m->L.kscale + (size_t)layer * m->L.ctx * nb,
                     m->L.vscale + (size_t)layer * m->L.ctx * nb};
  for (int i = 0; i < 2; i++) {
    uint8_t *hb = (uint8_t *)host[i];
    hipError_t e = hipSuccess;
    if (up) {
      for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < nb; b++) {
          const uint8_t *blk = hb + (r * nb + b) * 34;
          scales[r * nb + b] = (uint16_t)(blk[0] | (blk[1] << 8));
          memcpy(&codes[r * kvd + 32 * b], blk + 2, 32);
        }
      e = hipMemcpy(dq[i], codes.data(), codes.size(), hipMemcpyHostToDevice);
      if (e == hipSuccess) e = hipMemcpy(ds[i], scales.data(), scales.size() * 2, hipMemcpyHostToDevice);
    } else {
      e = hipMemcpy(codes.data(), dq[i], codes.size(), hipMemcpyDeviceToHost);
      if (e == hipSuccess) e = hipMemcpy(scales.data(), ds[i], scales.size() * 2, hipMemcpyDeviceToHost);
      for (size_t r = 0; r < rows && e == hipSuccess; r++)
        for (size_t b = 0; b < nb; b++) {
          uint8_t *blk = hb + (r * nb + b) * 34;
          blk[0] = (uint8_t)scales[r * nb + b];
          blk[1] = (uint8_t)(scales[r * nb + b] >> 8);
          memcpy(blk + 2, &codes[r * kvd + 32 * b], 32);
        }
    }
    if (e != hipSuccess) return fail(GQ_EHIP, "KV copy failed: %s", hipGetErrorString(e));
  }
  return GQ_OK;
}

int gq_model_kv_upload(gq_model *m, int layer, const void *k, const void *v, int n_pos) {
  return kv_copy(m, layer, (void *)k, (void *)v, n_pos, true);
}

int gq_model_kv_download(gq_model *m, int layer, void *k, void *v, int n_pos) {
  return kv_copy(m, layer, k, v, n_pos, false);
}

static int set_state(gq_model *m, int token, int pos, hipStream_t s) {
  if (token < 0 || token >= m->L.vocab) return fail(GQ_EINVAL, "token %d out of range", token);
  if (pos < 0 || pos >= m->L.ctx) return fail(GQ_EINVAL, "position %d outside the context", pos);
  HIP_TRY(gq::launch_set_state(m->L.state, token, pos, s));
  return GQ_OK;
}

int gq_model_decode(gq_model *m, int token, int pos, float *logits_host, int *next_token) {
  if (!m) return fail(GQ_EINVAL, "null model");
  int rc = set_state(m, token, pos, nullptr);
  if (rc) return rc;
  hipError_t e = gq::launch_decode_step(m->L, nullptr);
  if (e != hipSuccess) return fail(GQ_EHIP, "decode launch failed: %s", hipGetErrorString(e));
  if (logits_host)
    HIP_TRY(hipMemcpy(logits_host, m->L.logits, (size_t)m->L.vocab * 4, hipMemcpyDeviceToHost));
  gq::DecodeState st;
  HIP_TRY(hipMemcpy(&st, m->L.state, sizeof st, hipMemcpyDeviceToHost));
  if (next_token) *next_token = st.token;
  return GQ_OK;
}

int gq_model_generate(gq_model *m, int token, int pos, int n_steps, int *tokens_host,
                      void *stream) {
  if (!m) return fail(GQ_EINVAL, "null model");
  if (n_steps < 0 || n_steps > m->L.max_tokens || pos + n_steps > m->L.ctx)
    return fail(GQ_EINVAL, "%d steps from position %d exceed the context or token buffer",
                n_steps, pos);
  hipStream_t s = (hipStream_t)stream;
  int rc = set_state(m, token, pos, s);
  if (rc) return rc;
  if (!m->graph || m->graph_stream != s) {
    // Capture one step (its kernels read token/position from device state).
    if (m->graph) { (void)hipGraphExecDestroy(m->graph); m->graph = nullptr; }
    hipStream_t cap = nullptr;
    HIP_TRY(hipStreamCreateWithFlags(&cap, hipStreamNonBlocking));
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
      hipError_t le = gq::launch_decode_step(m->L, cap);
      e = hipStreamEndCapture(cap, &g);
      if (le != hipSuccess) e = le;
    }
    if (e == hipSuccess) e = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
    if (g) (void)hipGraphDestroy(g);
    (void)hipStreamDestroy(cap);
    if (e != hipSuccess) return fail(GQ_EHIP, "decode graph capture failed: %s", hipGetErrorString(e));
    m->graph_stream = s;
  }
  for (int i = 0; i < n_steps; i++) HIP_TRY(hipGraphLaunch(m->graph, s));
  if (tokens_host && n_steps > 0) {
    HIP_TRY(hipMemcpyAsync(tokens_host, m->L.tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
  }
  return GQ_OK;
}

// LlamaModel::run_batch (src/model/llama/cpu_path.rs:834-991): tokens at
// positions pos .. pos + n - 1 through every layer in passes of up to
// PREFILL_MAX tokens, K/V of every position written to the cache, logits of
// the last position.
int gq_model_prefill(gq_model *m, const int *tokens_host, int n, int pos, float *logits_host,
                     int *next_token, void *stream) {
  if (!m) return fail(GQ_EINVAL, "null model");
  if (!tokens_host || n < 1) return fail(GQ_EINVAL, "prefill needs at least one token");
  if (pos < 0 || (long)pos + n > m->L.ctx)
    return fail(GQ_EINVAL, "%d tokens from position %d exceed the context (%d)", n, pos, m->L.ctx);
  for (int i = 0; i < n; i++)
    if (tokens_host[i] < 0 || tokens_host[i] >= m->L.vocab)
      return fail(GQ_EINVAL, "token %d out of range", tokens_host[i]);
  hipStream_t s = (hipStream_t)stream;
  auto &L = m->L;
  if (L.kv_q8 && (L.n_kv_heads * L.head_dim) % 32)
    return fail(GQ_EINVAL, "a Q8_0 KV cache needs kv_dim a multiple of 32");
  if (L.hidden % 8 || L.hidden > 8 * 256 * 4 || L.ffn % 8 || (L.n_heads * L.head_dim) % 8)
    return fail(GQ_EINVAL, "prefill needs hidden <= 8192 and hidden, ffn multiples of 8");
  for (int l = 0; l < L.n_layers; l++) {
    const gq_weight *ws[7] = {L.wq[l], L.wk[l], L.wv[l], L.wo[l], L.wgate[l], L.wup[l], L.wdown[l]};
    for (const gq_weight *w : ws) {
      if (w->L.dtype != gq::T_Q4_K && w->L.dtype != gq::T_Q6_K && w->L.dtype != gq::T_Q5_K &&
          w->L.dtype != gq::T_Q8_0)
        return fail(GQ_EDTYPE, "layer %d: prefill needs Q4_K, Q5_K, Q6_K or Q8_0 projection weights, not %s", l,
                    type_name(w->L.dtype));
      int rc = gq_ensure_gemm_records(w, s);
      if (rc) return rc;
    }
  }
  if (!m->pf.x) {
    const int H = L.hidden, qd = L.n_heads * L.head_dim, kvd = L.n_kv_heads * L.head_dim;
    const size_t np = gq::PREFILL_MAX;
    const size_t kmax = (size_t)((std::max(std::max(H, L.ffn), qd) + 255) / 256 * 256);
    int rc = dalloc(m, &m->pf.x, np * H);
    if (!rc) rc = dalloc(m, &m->pf.q, np * qd);
    if (!rc) rc = dalloc(m, &m->pf.k, np * kvd);
    if (!rc) rc = dalloc(m, &m->pf.v, np * kvd);
    if (!rc) rc = dalloc(m, &m->pf.g, np * L.ffn);
    if (!rc) rc = dalloc(m, &m->pf.u, np * L.ffn);
    if (!rc) rc = dalloc(m, &m->pf.part, std::max<size_t>(1, gq::prefill_part_floats(L, gq::PREFILL_MAX, g_dev.num_cus)));
    if (!rc) rc = dalloc(m, &m->pf.xb, (size_t)gq::GEMM_NPAD * kmax);
    if (!rc) rc = dalloc(m, &m->pf.xh, (size_t)gq::GEMM_NPAD * ((L.ffn + 255) / 256 * 256));
    if (!rc) rc = dalloc(m, &m->pf.tokens, np);
    if (!rc && L.kv_q8) rc = dalloc(m, &m->pf.kf, (size_t)L.ctx * kvd);
    if (!rc && L.kv_q8) rc = dalloc(m, &m->pf.vf, (size_t)L.ctx * kvd);
    if (rc) { m->pf.x = nullptr; return rc; }
  }
  for (int off = 0; off < n; off += gq::PREFILL_MAX) {
    const int c = std::min(n - off, gq::PREFILL_MAX);
    HIP_TRY(hipMemcpyAsync(m->pf.tokens, tokens_host + off, (size_t)c * 4, hipMemcpyHostToDevice, s));
    hipError_t e = gq::launch_prefill(L, m->pf, m->pf.tokens, c, pos + off, g_dev.num_cus, s);
    if (e != hipSuccess) return fail(GQ_EHIP, "prefill launch failed: %s", hipGetErrorString(e));
    // the token upload of the next pass reuses the buffer
    HIP_TRY(hipStreamSynchronize(s));
  }
  if (logits_host || next_token) {
    std::vector<float> lg((size_t)L.vocab);
    HIP_TRY(hipMemcpy(lg.data(), L.logits, lg.size() * 4, hipMemcpyDeviceToHost));
    if (logits_host) memcpy(logits_host, lg.data(), lg.size() * 4);
    if (next_token) {  // first maximum from -inf, NaN never wins (sampler.rs:120-131)
      int best = 0;
      float bv = -INFINITY;
      for (int i = 0; i < L.vocab; i++)
        if (lg[i] > bv) {
          bv = lg[i];
          best = i;
        }
      *next_token = best;
    }
  }
  return GQ_OK;
}

int gq_sync(void *stream) {
  HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
  return GQ_OK;
}

}  // extern "C"
