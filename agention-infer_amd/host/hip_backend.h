// hip_backend.h -- the HIP backend as the reference's host code sees it
// (host C++ over the C ABI of libgq.so, include/gq.h).
//
// HipBackend mirrors the Backend trait (src/ops/mod.rs:93-106: name(),
// matmul_dequant) and the GPU-resident API of the reference's GPU backend
// (upload_weight / matmul_dequant_preloaded / handle shape accessors,
// src/ops/wgpu_backend/mod.rs:61-92, 642-696, 906-922).  The trait's CubeCL
// associated type (type R: Runtime, client()) has no counterpart: this
// backend is reached through the C ABI.  Failures throw GgufError with kind
// BackendError and libgq's message, as the CPU backend returns
// GgufError::BackendError (src/ops/cpu_backend.rs:57-61).
//
// upload_tensor / upload_gguf take tensors straight out of a mapped GGUF
// file (pre_upload_gpu, src/model/llama/gpu_resident.rs:69-229): the bytes
// go from the mapping to the device once and stay resident.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/gq.h"
#include "gguf.h"

namespace gqh {

// A resident weight (GpuWeightHandle): owns its device memory.
class GpuWeight {
 public:
  GpuWeight() = default;
  explicit GpuWeight(gq_weight *w) : w_(w) {}
  GpuWeight(GpuWeight &&o) noexcept : w_(o.w_) { o.w_ = nullptr; }
  GpuWeight &operator=(GpuWeight &&o) noexcept;
  GpuWeight(const GpuWeight &) = delete;
  GpuWeight &operator=(const GpuWeight &) = delete;
  ~GpuWeight();
  const gq_weight *get() const { return w_; }
  gq_weight *release();
  explicit operator bool() const { return w_ != nullptr; }
  // (in_dim, out_dim) and the GGML type
  std::pair<size_t, size_t> shape() const;
  size_t out_dim() const { return shape().second; }
  GgmlType dtype() const;
  size_t device_bytes() const { return gq_weight_bytes(w_); }

 private:
  gq_weight *w_ = nullptr;
};

class HipBackend {
 public:
  explicit HipBackend(int device = 0);  // throws BackendError without a gfx950 device
  const char *name() const { return "hip"; }

  // Backend::matmul_dequant: w is the whole tensor (out.size() rows of
  // type_size(x.size()) bytes, ggml block order); out is overwritten.
  void matmul_dequant(GgmlType dtype, const uint8_t *w, size_t w_len, const float *x, size_t x_len,
                      float *out, size_t out_len) const;

  // One upload, resident until the handle goes.
  GpuWeight upload_weight(GgmlType dtype, const uint8_t *w, size_t w_len, size_t in_dim) const;
  void matmul_dequant_preloaded(const GpuWeight &h, const float *x, size_t x_len, float *out,
                                size_t out_len) const;

  // A 2-D weight tensor of a GGUF file (dims [in_dim, out_dim]); a tensor of
  // another rank or a type this backend does not multiply is refused.
  GpuWeight upload_tensor(const GgufFile &f, const uint8_t *data, size_t data_len,
                          const TensorInfo &t) const;
  // Every 2-D tensor of a supported type, by name; others are skipped and
  // their names returned in `skipped`.
  std::unordered_map<std::string, GpuWeight> upload_gguf(const GgufFile &f, const Mmap &m,
                                                         std::vector<std::string> *skipped = nullptr) const;
};

// The GGML types this backend multiplies (Q8_0, Q4_K, Q5_K, Q6_K, IQ3_XXS).
bool gpu_dequant_type(GgmlType t);

}  // namespace gqh
