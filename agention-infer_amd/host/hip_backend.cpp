// hip_backend.cpp -- see hip_backend.h.
#include <climits>
#include "hip_backend.h"

namespace gqh {

namespace {
[[noreturn]] void backend_fail() {
  throw GgufError(GgufError::Kind::BackendError, std::string("backend error: ") + gq_last_error());
}
void check(int rc) {
  if (rc != GQ_OK) backend_fail();
}
}  // namespace

bool gpu_dequant_type(GgmlType t) {
  return t == GgmlType::Q8_0 || t == GgmlType::Q4_K || t == GgmlType::Q5_K ||
         t == GgmlType::Q6_K || t == GgmlType::IQ3_XXS;
}

GpuWeight &GpuWeight::operator=(GpuWeight &&o) noexcept {
  if (this != &o) {
    if (w_) gq_weight_free(w_);
    w_ = o.w_;
    o.w_ = nullptr;
  }
  return *this;
}
GpuWeight::~GpuWeight() {
  if (w_) gq_weight_free(w_);
}
gq_weight *GpuWeight::release() {
  gq_weight *w = w_;
  w_ = nullptr;
  return w;
}
std::pair<size_t, size_t> GpuWeight::shape() const {
  int dt = 0, in = 0, out = 0;
  check(gq_weight_shape(w_, &dt, &in, &out));
  return {(size_t)in, (size_t)out};
}
GgmlType GpuWeight::dtype() const {
  int dt = 0, in = 0, out = 0;
  check(gq_weight_shape(w_, &dt, &in, &out));
  return (GgmlType)dt;
}

HipBackend::HipBackend(int device) { check(gq_init(device)); }

void HipBackend::matmul_dequant(GgmlType dtype, const uint8_t *w, size_t w_len, const float *x,
                                size_t x_len, float *out, size_t out_len) const {
  check(gq_matmul_dequant_host((int)dtype, w, w_len, x, x_len, out, out_len));
}

GpuWeight HipBackend::upload_weight(GgmlType dtype, const uint8_t *w, size_t w_len,
                                    size_t in_dim) const {
  if (!gpu_dequant_type(dtype) || in_dim == 0)
    throw GgufError(GgufError::Kind::BackendError,
                    std::string("backend error: upload_weight: unsupported dtype ") + type_name(dtype));
  const size_t row = type_size(dtype, in_dim), out_dim = w_len / row;
  if (out_dim * row != w_len)
    throw GgufError(GgufError::Kind::BackendError,
                    "backend error: upload_weight: " + std::to_string(w_len) +
                        " bytes is not a whole number of rows of " + std::to_string(row));
  if (in_dim > (size_t)INT_MAX || out_dim > (size_t)INT_MAX)
    throw GgufError(GgufError::Kind::BackendError,
                    "backend error: upload_weight: shape " + std::to_string(out_dim) + " x " +
                        std::to_string(in_dim) + " exceeds the backend's 2^31-1 rows/columns");
  gq_weight *h = nullptr;
  check(gq_upload((int)dtype, w, w_len, (int)in_dim, (int)out_dim, &h));
  return GpuWeight(h);
}

void HipBackend::matmul_dequant_preloaded(const GpuWeight &h, const float *x, size_t x_len,
                                          float *out, size_t out_len) const {
  const auto [in, o] = h.shape();
  if (x_len != in || out_len != o)
    throw GgufError(GgufError::Kind::BackendError,
                    "backend error: matmul_dequant_preloaded: x has " + std::to_string(x_len) +
                        " elements for in_dim " + std::to_string(in) + ", out " +
                        std::to_string(out_len) + " for out_dim " + std::to_string(o));
  check(gq_matmul_dequant_preloaded(h.get(), x, out));
}

GpuWeight HipBackend::upload_tensor(const GgufFile &f, const uint8_t *data, size_t data_len,
                                    const TensorInfo &t) const {
  if (t.n_dims != 2 || !gpu_dequant_type(t.ggml_type))
    throw GgufError(GgufError::Kind::BackendError,
                    "backend error: tensor " + t.name + " (" + type_name(t.ggml_type) + ", " +
                        t.shape_str() + ") is not a weight this backend multiplies");
  const uint64_t at = f.data_offset + t.byte_offset, n = t.byte_size();
  if (at > data_len || n > data_len - at)
    throw GgufError(GgufError::Kind::UnexpectedEof,
                    "unexpected end of input at byte " + std::to_string(data_len), data_len);
  return upload_weight(t.ggml_type, data + at, (size_t)n, (size_t)t.dims[0]);
}

std::unordered_map<std::string, GpuWeight> HipBackend::upload_gguf(
    const GgufFile &f, const Mmap &m, std::vector<std::string> *skipped) const {
  std::unordered_map<std::string, GpuWeight> out;
  for (const TensorInfo &t : f.tensors) {
    if (t.n_dims == 2 && gpu_dequant_type(t.ggml_type)) {
      out.emplace(t.name, upload_tensor(f, m.data(), m.size(), t));
    } else if (skipped) {
      skipped->push_back(t.name);
    }
  }
  return out;
}

}  // namespace gqh
