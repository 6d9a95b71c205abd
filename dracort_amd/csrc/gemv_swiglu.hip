// Fused gate/up GEMV with the SwiGLU epilogue: y = silu(W_gate x) * (W_up x).
// Replaces the reference executor's _mlp gate/up projections and swiglu
// (draco/runtime/cpu/executor.py:208-224, draco/runtime/cpu/ops.py:19-27).
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

}  // namespace draco
