// GEMV with the residual-add epilogue: resid += W x (float32, in place) and an
// optional bfloat16 copy of the updated residual for the next projection.
// Replaces _o_proj / the down projection plus the residual adds of
// forward_step (draco/runtime/cpu/executor.py:273-277, 308-329).
#include "gemv_x1.h"

namespace draco {

static StreamJob resid_job(int qtype, int m, int n, int k) {
  StreamJob job{};
  job.n_mats = 1;
  job.n[0] = n;
  job.rows = n;
  job.row_bytes = row_bytes_of(qtype, k);
  job.k = k;
  job.m = m;
  return job;
}

size_t gemv_resid_split_bytes(int qtype, int m, int n, int k) {
  // the launches the matrix-core kernel takes: its types, 8..16 rows
  if ((qtype != kQ4_K && qtype != kQ6_K && qtype != kQ4_0) || m < 8) return 0;
  return gemv_split_bytes(resid_job(qtype, m, n, k));
}

int gemv_resid_dispatch(int qtype, bool d_last, const void* w, const void* x, bool xbf16, float* resid,
                        uint16_t* resid_bf16, int m, int n, int k, void* workspace, size_t workspace_bytes,
                        hipStream_t s) {
  StreamJob job{};
  job.n_mats = 1;
  job.w[0] = static_cast<const uint8_t*>(w);
  job.n[0] = n;
  job.rows = n;
  job.row_bytes = row_bytes_of(qtype, k);
  job.k = k;
  job.m = m;
  job.x = x;
  job.resid = resid;
  job.resid_bf16 = resid_bf16;
  // split K when the caller's workspace holds the partial sums (only the
  // matrix-core kernel reads job.part)
  const size_t need = workspace ? gemv_resid_split_bytes(qtype, m, n, k) : 0;
  if (need > 0 && workspace_bytes >= need) {
    job.part = static_cast<float*>(workspace);
    job.split_chunks = 8;
  }
  return gemv_dispatch_mode<kResid>(qtype, d_last, job, xbf16, s);
}

}  // namespace draco
