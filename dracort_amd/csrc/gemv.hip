// Fused GGUF dequant + GEMV for decode (M = 1..16 activation rows) on gfx950.
//
//   y[m, n] = sum_k x[m, k] * W[n, k]  (+ bias[n])
//
// Replaces the reference's per-call "dequantize the whole tensor, then
// x.astype(f32) @ W.T" (draco/format/gguf.py:820-834 feeding
// draco/runtime/cpu/kernels/generic.py:32-33 from _linear,
// draco/runtime/cpu/executor.py:47-79).  The weight stays in its packed GGUF
// block layout in HBM and is read exactly once; the math is in gemv_core.h.
#include "draco_internal.h"
#include "gemv_core.h"

namespace draco {

template <int QT, bool DL, int MT, bool XBF16, int R>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* __restrict__ w, const void* __restrict__ x,
                                                   const float* __restrict__ bias, float* __restrict__ y, int m,
                                                   int n, int k, int64_t row_bytes) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int n0 = wave * R;
  if (n0 >= n) return;
  const size_t xstride = XBF16 ? (size_t)k * 2 : (size_t)k * 4;
  const uint8_t* xb = static_cast<const uint8_t*>(x);
  float acc[R][MT];
  gemv_accumulate<QT, DL, MT, XBF16, R>(w, row_bytes, n0, n, k, m,
                                        [&](int mi) { return (const void*)(xb + (size_t)mi * xstride); }, acc);
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      const float v = wave_sum(acc[r][mi]);
      if (lane == 0 && mi < m && n0 + r < n) y[(size_t)mi * n + n0 + r] = v + (bias ? bias[n0 + r] : 0.f);
    }
  }
}

template <int QT, bool DL, int MT, bool XBF16, int R>
static int launch_gemv(const void* w, const void* x, const float* bias, float* y, int m, int n, int k,
                       hipStream_t s) {
  const int64_t row_bytes = (int64_t)(k / Fmt<QT>::QK) * Fmt<QT>::BYTES;
  const int waves = (n + R - 1) / R;
  const int blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((gemv_kernel<QT, DL, MT, XBF16, R>), dim3(blocks), dim3(256), 0, s,
                     static_cast<const uint8_t*>(w), x, bias, y, m, n, k, row_bytes);
  return check_launch("gemv");
}

// Rows per wave: as many as keep >= 2 workgroups per CU on the 256-CU part.
static int pick_rows(int n, int mt) {
  const int target_blocks = 512;
  if (mt <= 4 && (n + 15) / 16 >= target_blocks) return 4;
  if ((n + 7) / 8 >= target_blocks) return 2;
  return 1;
}

template <int QT, bool DL, int MT, bool XBF16>
static int gemv_rows(const void* w, const void* x, const float* bias, float* y, int m, int n, int k,
                     hipStream_t s) {
  const int r = pick_rows(n, MT);
  if constexpr (MT <= 4) {
    if (r == 4) return launch_gemv<QT, DL, MT, XBF16, 4>(w, x, bias, y, m, n, k, s);
  }
  if (r >= 2) return launch_gemv<QT, DL, MT, XBF16, 2>(w, x, bias, y, m, n, k, s);
  return launch_gemv<QT, DL, MT, XBF16, 1>(w, x, bias, y, m, n, k, s);
}

template <int QT, bool DL, bool XBF16>
static int gemv_mt(const void* w, const void* x, const float* bias, float* y, int m, int n, int k,
                   hipStream_t s) {
  if (m <= 1) return gemv_rows<QT, DL, 1, XBF16>(w, x, bias, y, m, n, k, s);
  if (m <= 2) return gemv_rows<QT, DL, 2, XBF16>(w, x, bias, y, m, n, k, s);
  if (m <= 4) return gemv_rows<QT, DL, 4, XBF16>(w, x, bias, y, m, n, k, s);
  if (m <= 8) return gemv_rows<QT, DL, 8, XBF16>(w, x, bias, y, m, n, k, s);
  return gemv_rows<QT, DL, 16, XBF16>(w, x, bias, y, m, n, k, s);
}

template <int QT, bool DL>
static int gemv_x(const void* w, const void* x, bool x_bf16, const float* bias, float* y, int m, int n, int k,
                  hipStream_t s) {
  return x_bf16 ? gemv_mt<QT, DL, true>(w, x, bias, y, m, n, k, s)
                : gemv_mt<QT, DL, false>(w, x, bias, y, m, n, k, s);
}

int gemv_dispatch(int qtype, bool d_last, const void* w, const void* x, bool x_bf16, const float* bias, float* y,
                  int m, int n, int k, hipStream_t s) {
  switch (qtype) {
    case kQ8_0: return gemv_x<kQ8_0, false>(w, x, x_bf16, bias, y, m, n, k, s);
    case kQ4_0: return gemv_x<kQ4_0, false>(w, x, x_bf16, bias, y, m, n, k, s);
    case kQ4_K: return gemv_x<kQ4_K, false>(w, x, x_bf16, bias, y, m, n, k, s);
    case kQ6_K:
      return d_last ? gemv_x<kQ6_K, true>(w, x, x_bf16, bias, y, m, n, k, s)
                    : gemv_x<kQ6_K, false>(w, x, x_bf16, bias, y, m, n, k, s);
    default: return set_error(DRACO_EINVAL_QTYPE, "unsupported ggml type %d", qtype);
  }
}

}  // namespace draco
