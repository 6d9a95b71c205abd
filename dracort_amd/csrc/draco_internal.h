// Internal helpers shared by the HIP translation units of libdraco_gguf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/draco_gguf.h"

namespace draco {

// Records a formatted message in the calling thread's last-error slot and
// returns `code` (one of the DRACO_E* values).
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// hipGetLastError() after a launch -> DRACO_OK or DRACO_EHIP with the HIP message.
int check_launch(const char* what);

int dequant_dispatch(int qtype, bool d_last, const void* w, float* out, int64_t n_rows, int64_t k,
                     hipStream_t s);

// Row gather with dequantization: out[i, :] = dequant(W[ids[i], :]) for
// i < n_rows (ids NULL: row i itself); W has n_src_rows rows; an id outside
// [0, n_src_rows) gives a NaN row.
int dequant_rows_dispatch(int qtype, bool d_last, const void* w, const int32_t* ids, int64_t n_src_rows, float* out,
                          int64_t n_rows, int64_t k, hipStream_t s);

int gemv_dispatch(int qtype, bool d_last, const void* w, const void* x, bool x_bf16, const float* bias,
                  float* y, int m, int n, int k, hipStream_t s);

int gemv_multi_dispatch(int qtype, bool d_last, int n_mats, const void* const* w, const int* n, float* const* y,
                        uint16_t* const* yb, const void* x, bool xbf16, const float* bias, int m, int k,
                        hipStream_t s);

int gemv_swiglu_dispatch(int qtype, bool d_last, const void* w_gate, const void* w_up, float* y, uint16_t* yb,
                         const void* x, bool xbf16, int m, int n, int k, hipStream_t s);

// workspace: NULL, or room for the split-K partial sums (gemv_resid_split_bytes)
size_t gemv_resid_split_bytes(int qtype, int m, int n, int k);
int gemv_resid_dispatch(int qtype, bool d_last, const void* w, const void* x, bool xbf16, float* resid,
                        uint16_t* resid_bf16, int m, int n, int k, void* workspace, size_t workspace_bytes,
                        hipStream_t s);

// RMSNorm of m rows of n float32 values into float32 y and / or bf16 yb.
int rms_norm_launch(const float* x, const float* w, float eps, float* y, uint16_t* yb, int64_t m, int64_t n,
                    hipStream_t s);

// GEMV launches whose input is RMSNorm(x) (x float32 [m, k]): fused into the
// persistent single-token kernel where it runs, else rms_norm_launch into
// x_norm followed by the plain launch.  x_norm [m, k] bf16 always receives the
// normalized input.
int gemv_multi_norm_dispatch(int qtype, bool d_last, int n_mats, const void* const* w, const int* n, float* const* y,
                             uint16_t* const* yb, const float* x, const float* norm_w, float eps, uint16_t* x_norm,
                             int m, int k, hipStream_t s);

int gemv_swiglu_norm_dispatch(int qtype, bool d_last, const void* w_gate, const void* w_up, float* y, uint16_t* yb,
                              const float* x, const float* norm_w, float eps, uint16_t* x_norm, int m, int n, int k,
                              hipStream_t s);

// Workspace bytes of the GEMM of this base type (0: it needs none): the
// minimum its workspace kernels require, and the size that also holds the
// split-K partial sums of the few-tile shapes.
size_t gemm_workspace_min(int qtype, int64_t m, int64_t k);
size_t gemm_workspace_size(int qtype, int64_t m, int64_t k);

// workspace: NULL, or at least gemm_workspace_min(qtype, m, k) bytes (256-byte
// aligned), of which workspace_bytes are usable.
int gemm_dispatch(int qtype, bool d_last, const void* w, const void* x_bf16, const float* bias, float* y,
                  int m, int n, int k, void* workspace, size_t workspace_bytes, hipStream_t s);

}  // namespace draco
