// Decode GEMV (plain mode of the streaming kernel): y = W x (+ bias), and the
// multi-matrix launch (several weights sharing x, e.g. q, k, v).
// Replaces _dequantize + x.astype(f32) @ W.T (draco/format/gguf.py:820-834,
// draco/runtime/cpu/kernels/generic.py:32-33) per _linear call
// (draco/runtime/cpu/executor.py:47-79), and _qkv (:243-271) for the fused
// form, optionally with the _norm before it (:199-206) in the prologue.
#include "gemv_x1.h"

namespace draco {

int gemv_multi_dispatch(int qtype, bool d_last, int n_mats, const void* const* w, const int* n, float* const* y,
                        uint16_t* const* yb, const void* x, bool xbf16, const float* bias, int m, int k,
                        hipStream_t s) {
  StreamJob job{};
  job.n_mats = n_mats;
  for (int i = 0; i < n_mats; ++i) {
    job.w[i] = static_cast<const uint8_t*>(w[i]);
    job.n[i] = n[i];
    job.y[i] = y ? y[i] : nullptr;
    job.yb[i] = yb ? yb[i] : nullptr;
    job.rows += n[i];
  }
  job.row_bytes = row_bytes_of(qtype, k);
  job.k = k;
  job.m = m;
  job.x = x;
  job.bias = bias;
  return gemv_dispatch_mode<kPlain>(qtype, d_last, job, xbf16, s);
}

int gemv_multi_norm_dispatch(int qtype, bool d_last, int n_mats, const void* const* w, const int* n, float* const* y,
                             uint16_t* const* yb, const float* x, const float* norm_w, float eps, uint16_t* x_norm,
                             int m, int k, hipStream_t s) {
  StreamJob job{};
  job.n_mats = n_mats;
  for (int i = 0; i < n_mats; ++i) {
    job.w[i] = static_cast<const uint8_t*>(w[i]);
    job.n[i] = n[i];
    job.y[i] = y ? y[i] : nullptr;
    job.yb[i] = yb ? yb[i] : nullptr;
    job.rows += n[i];
  }
  job.row_bytes = row_bytes_of(qtype, k);
  job.k = k;
  job.m = m;
  job.x = x;
  if (x1p_ok(qtype, job, true)) {
    job.norm_w = norm_w;
    job.norm_eps = eps;
    job.x_norm = x_norm;
    return gemv_dispatch_norm<kPlain>(qtype, d_last, job, s);
  }
  if (int rc = rms_norm_launch(x, norm_w, eps, nullptr, x_norm, m, k, s)) return rc;
  return gemv_multi_dispatch(qtype, d_last, n_mats, w, n, y, yb, x_norm, true, nullptr, m, k, s);
}

int gemv_dispatch(int qtype, bool d_last, const void* w, const void* x, bool x_bf16, const float* bias, float* y,
                  int m, int n, int k, hipStream_t s) {
  const void* ws[1] = {w};
  float* ys[1] = {y};
  const int ns[1] = {n};
  return gemv_multi_dispatch(qtype, d_last, 1, ws, ns, ys, nullptr, x, x_bf16, bias, m, k, s);
}

}  // namespace draco
