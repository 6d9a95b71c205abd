// Fused gate/up GEMV with the SwiGLU epilogue: y = silu(W_gate x) * (W_up x),
// optionally with the post-attention RMSNorm of x in the prologue.
// Replaces the reference executor's _mlp gate/up projections and swiglu
// (draco/runtime/cpu/executor.py:208-224, draco/runtime/cpu/ops.py:19-27) and
// the _norm before them (:199-206, 331-334).
#include "gemv_x1.h"

namespace draco {

int gemv_swiglu_dispatch(int qtype, bool d_last, const void* w_gate, const void* w_up, float* y, uint16_t* yb,
                         const void* x, bool xbf16, int m, int n, int k, hipStream_t s) {
  StreamJob job{};
  job.n_mats = 2;
  job.w[0] = static_cast<const uint8_t*>(w_gate);
  job.w[1] = static_cast<const uint8_t*>(w_up);
  job.n[0] = job.n[1] = n;
  job.y[0] = y;
  job.yb[0] = yb;
  job.rows = n;
  job.row_bytes = row_bytes_of(qtype, k);
  job.k = k;
  job.m = m;
  job.x = x;
  return gemv_dispatch_mode<kSwiGLU>(qtype, d_last, job, xbf16, s);
}

int gemv_swiglu_norm_dispatch(int qtype, bool d_last, const void* w_gate, const void* w_up, float* y, uint16_t* yb,
                              const float* x, const float* norm_w, float eps, uint16_t* x_norm, int m, int n, int k,
                              hipStream_t s) {
  StreamJob job{};
  job.n_mats = 2;
  job.w[0] = static_cast<const uint8_t*>(w_gate);
  job.w[1] = static_cast<const uint8_t*>(w_up);
  job.n[0] = job.n[1] = n;
  job.y[0] = y;
  job.yb[0] = yb;
  job.rows = n;
  job.row_bytes = row_bytes_of(qtype, k);
  job.k = k;
  job.m = m;
  job.x = x;
  if (x1p_ok(qtype, job, true)) {
    job.norm_w = norm_w;
    job.norm_eps = eps;
    job.x_norm = x_norm;
    return gemv_dispatch_norm<kSwiGLU>(qtype, d_last, job, s);
  }
  if (int rc = rms_norm_launch(x, norm_w, eps, nullptr, x_norm, m, k, s)) return rc;
  return gemv_swiglu_dispatch(qtype, d_last, w_gate, w_up, y, yb, x_norm, true, m, n, k, s);
}

}  // namespace draco
