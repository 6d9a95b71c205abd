// Float-weight and elementwise pieces of the executor's step on gfx950: the
// tensors of a GGUF file that are not block-quantized (F32 / F16 / BF16
// weights, embeddings), the SwiGLU product of separately computed gate and up
// projections, and the embedding gather for float tables.
//
//  * dense_linear_kernel   y[m, n] (+)= x[m, :] . W[n, :] (+ bias[n]) for a
//    float32 / float16 / bfloat16 weight: the reference's `_linear` on a
//    tensor with quantization=None, get_tensor(dequantize=True) followed by
//    matmul_f32 = x.astype(f32) @ W.T (draco/runtime/cpu/executor.py:47-52,
//    draco/runtime/cpu/kernels/generic.py:32-33), plus the residual add of
//    forward_step (executor.py:324-329) when `accumulate` is set.  One wave per
//    weight row, up to 8 activation rows per workgroup column; lanes stride K
//    with 16-byte loads when every row starts 16-byte aligned, else element
//    by element.  Float32 accumulation, wave-reduced.  These tensors are
//    outside the quantized hot path: the kernel is plain and HBM-bound.
//  * float_rows_kernel     out[i, :] = float(W[ids[i], :]) (NaN row for an id
//    outside the table): embed[token_ids] of _initial_hidden
//    (executor.py:279-288) for float tables; block-quantized tables go through
//    the dequantization kernel's gather.
//  * swiglu_kernel         y = silu(g) * u (draco/runtime/cpu/ops.py:19-27)
//    for gate / up projections that were not fused into one launch.
#include "draco_internal.h"
#include "gemv_core.h"

namespace draco {

enum WDtype { kWF32 = 0, kWF16 = 1, kWBF16 = 2 };

template <int WT>
__device__ __forceinline__ float w_at(const void* __restrict__ w, int64_t i) {
  if constexpr (WT == kWF32) return static_cast<const float*>(w)[i];
  if constexpr (WT == kWF16) return (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(w)[i]);
  return __uint_as_float((uint32_t)static_cast<const uint16_t*>(w)[i] << 16);
}

template <bool XBF16>
__device__ __forceinline__ float x_at(const void* __restrict__ x, int64_t i) {
  if constexpr (XBF16) return __uint_as_float((uint32_t)static_cast<const uint16_t*>(x)[i] << 16);
  return static_cast<const float*>(x)[i];
}

// four consecutive elements starting at element i (16-byte aligned for float32, 8 for 16-bit types)
template <int WT>
__device__ __forceinline__ float4 w4_at(const void* __restrict__ w, int64_t i) {
  if constexpr (WT == kWF32) return *reinterpret_cast<const float4*>(static_cast<const float*>(w) + i);
  const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + i);
  if constexpr (WT == kWF16) {
    return make_float4((float)__builtin_bit_cast(_Float16, (uint16_t)(v.x & 0xFFFFu)),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)(v.x >> 16)),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)(v.y & 0xFFFFu)),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)(v.y >> 16)));
  }
  return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y << 16),
                     __uint_as_float(v.y & 0xFFFF0000u));
}

template <bool XBF16>
__device__ __forceinline__ float4 x4_at(const void* __restrict__ x, int64_t i) {
  if constexpr (!XBF16) return *reinterpret_cast<const float4*>(static_cast<const float*>(x) + i);
  const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(x) + i);
  return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y << 16),
                     __uint_as_float(v.y & 0xFFFF0000u));
}

constexpr int kDenseMT = 8;  // activation rows per workgroup column

// grid (ceil(N / 4), ceil(M / 8)), 256 threads: wave w of workgroup b owns
// weight row 4 b + w and activation rows 8 blockIdx.y .. + 7.
template <int WT, bool XBF16, bool VEC>
__global__ __launch_bounds__(256) void dense_linear_kernel(const void* __restrict__ w, const void* __restrict__ x,
                                                           const float* __restrict__ bias, float* __restrict__ y,
                                                           int M, int N, int K, int accumulate) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int m0 = blockIdx.y * kDenseMT;
  if (n >= N) return;
  const int mt = min(kDenseMT, M - m0);
  float acc[kDenseMT];
#pragma unroll
  for (int i = 0; i < kDenseMT; ++i) acc[i] = 0.f;
  const int64_t wrow = (int64_t)n * K;
  if constexpr (VEC) {
    for (int k4 = 4 * lane; k4 < K; k4 += 256) {
      const float4 wv = w4_at<WT>(w, wrow + k4);
#pragma unroll
      for (int i = 0; i < kDenseMT; ++i) {
        if (i < mt) {
          const float4 xv = x4_at<XBF16>(x, (int64_t)(m0 + i) * K + k4);
          acc[i] = fmaf(wv.x, xv.x, acc[i]);
          acc[i] = fmaf(wv.y, xv.y, acc[i]);
          acc[i] = fmaf(wv.z, xv.z, acc[i]);
          acc[i] = fmaf(wv.w, xv.w, acc[i]);
        }
      }
    }
  } else {
    for (int k = lane; k < K; k += 64) {
      const float wv = w_at<WT>(w, wrow + k);
#pragma unroll
      for (int i = 0; i < kDenseMT; ++i)
        if (i < mt) acc[i] = fmaf(wv, x_at<XBF16>(x, (int64_t)(m0 + i) * K + k), acc[i]);
    }
  }
  const float b = bias ? bias[n] : 0.f;
#pragma unroll
  for (int i = 0; i < kDenseMT; ++i) {
    const float v = wave_sum(acc[i]);
    if (lane == i && i < mt) {
      float* o = y + (int64_t)(m0 + i) * N + n;
      *o = (accumulate ? *o : 0.f) + (v + b);
    }
  }
}

template <int WT>
__global__ __launch_bounds__(256) void float_rows_kernel(const void* __restrict__ w, const int32_t* __restrict__ ids,
                                                         int64_t n_src_rows, float* __restrict__ out, int K) {
  const int row = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= K) return;
  const int64_t src = ids[row];
  const bool bad = src < 0 || src >= n_src_rows;
  out[(int64_t)row * K + c] = bad ? __builtin_nanf("") : w_at<WT>(w, src * K + c);
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ y, uint16_t* __restrict__ yb, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = silu(g[i]) * u[i];
  if (y) y[i] = v;
  if (yb) yb[i] = f32_to_bf16_rne(v);
}

static int wdtype_of(int ggml_type, int* wt, int* elem) {
  switch (ggml_type) {
    case 0: *wt = kWF32; *elem = 4; return DRACO_OK;
    case 1: *wt = kWF16; *elem = 2; return DRACO_OK;
    case 30: *wt = kWBF16; *elem = 2; return DRACO_OK;
    default:
      return set_error(DRACO_EINVAL_QTYPE, "dense weights are F32 (0), F16 (1) or BF16 (30), got ggml type %d",
                       ggml_type);
  }
}

template <int WT, bool XBF16>
static int launch_dense(const void* w, const void* x, const float* bias, float* y, int m, int n, int k, int acc,
                        bool vec, hipStream_t s) {
  const dim3 grid((unsigned)((n + 3) / 4), (unsigned)((m + kDenseMT - 1) / kDenseMT));
  if (vec)
    hipLaunchKernelGGL((dense_linear_kernel<WT, XBF16, true>), grid, dim3(256), 0, s, w, x, bias, y, m, n, k, acc);
  else
    hipLaunchKernelGGL((dense_linear_kernel<WT, XBF16, false>), grid, dim3(256), 0, s, w, x, bias, y, m, n, k, acc);
  return check_launch("dense_linear");
}

}  // namespace draco

using namespace draco;

namespace {

constexpr int64_t kMaxDenseDim = (int64_t)1 << 30;

bool al(const void* p, uintptr_t a) { return p != nullptr && (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

extern "C" {

int draco_gguf_dense_linear(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype,
                            const float* bias, float* y, int64_t m, int64_t n, int64_t k, int accumulate,
                            void* stream) {
  int wt, elem;
  if (int rc = wdtype_of(ggml_type, &wt, &elem)) return rc;
  if (m < 1 || n < 1 || k < 1 || m > kMaxDenseDim || n > kMaxDenseDim || k > kMaxDenseDim ||
      (m + kDenseMT - 1) / kDenseMT > 65535 || n * k > ((int64_t)1 << 40))
    return set_error(DRACO_EINVAL_SHAPE, "invalid dense linear shape m=%lld [%lld, %lld]", (long long)m,
                     (long long)n, (long long)k);
  if ((uint64_t)(n * k * elem) > (uint64_t)w_bytes)
    return set_error(DRACO_EINVAL_SHAPE, "w holds %zu bytes but a [%lld, %lld] weight of ggml type %d needs %lld",
                     w_bytes, (long long)n, (long long)k, ggml_type, (long long)(n * k * elem));
  if (x_dtype != DRACO_DTYPE_F32 && x_dtype != DRACO_DTYPE_BF16)
    return set_error(DRACO_EINVAL_ARG, "unknown activation dtype %d", x_dtype);
  const int xe = x_dtype == DRACO_DTYPE_BF16 ? 2 : 4;
  if (!al(w, elem) || !al(x, xe) || !al(y, 4) || (bias && !al(bias, 4)))
    return set_error(DRACO_EINVAL_ARG, "w, x and y must be non-NULL and aligned to their element size");
  // 16-byte lanes when every weight and activation row starts 16-byte (float32) / 8-byte (16-bit) aligned
  const bool vec = k % 4 == 0 && al(w, elem == 4 ? 16 : 8) && al(x, xe == 4 ? 16 : 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool xb = x_dtype == DRACO_DTYPE_BF16;
  const int M = (int)m, N = (int)n, K = (int)k, A = accumulate ? 1 : 0;
  switch (wt) {
    case kWF32: return xb ? launch_dense<kWF32, true>(w, x, bias, y, M, N, K, A, vec, s)
                          : launch_dense<kWF32, false>(w, x, bias, y, M, N, K, A, vec, s);
    case kWF16: return xb ? launch_dense<kWF16, true>(w, x, bias, y, M, N, K, A, vec, s)
                          : launch_dense<kWF16, false>(w, x, bias, y, M, N, K, A, vec, s);
    default: return xb ? launch_dense<kWBF16, true>(w, x, bias, y, M, N, K, A, vec, s)
                       : launch_dense<kWBF16, false>(w, x, bias, y, M, N, K, A, vec, s);
  }
}

int draco_gguf_get_rows(int ggml_type, const void* w, size_t w_bytes, int64_t n_rows, int64_t k, const int32_t* ids,
                        int64_t n_ids, float* out, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_rows < 1 || k < 1 || n_rows > kMaxDenseDim || k > kMaxDenseDim || n_ids < 1 || n_ids > 65535)
    return set_error(DRACO_EINVAL_SHAPE, "invalid gather: table [%lld, %lld], %lld ids", (long long)n_rows,
                     (long long)k, (long long)n_ids);
  if (!al(ids, 4)) return set_error(DRACO_EINVAL_ARG, "ids must be non-NULL and 4-byte aligned");
  int wt, elem;
  const int base = ggml_type & ~DRACO_GGUF_GGML_ORDER;
  if (base == 0 || base == 1 || base == 30) {
    if (int rc = wdtype_of(base, &wt, &elem)) return rc;
    if ((uint64_t)(n_rows * k * elem) > (uint64_t)w_bytes)
      return set_error(DRACO_EINVAL_SHAPE, "table holds %zu bytes, [%lld, %lld] needs %lld", w_bytes,
                       (long long)n_rows, (long long)k, (long long)(n_rows * k * elem));
    if (!al(w, elem) || !al(out, 4)) return set_error(DRACO_EINVAL_ARG, "w and out must be non-NULL and aligned");
    const dim3 grid((unsigned)((k + 255) / 256), (unsigned)n_ids);
    const int K = (int)k;
    if (wt == kWF32)
      hipLaunchKernelGGL(float_rows_kernel<kWF32>, grid, dim3(256), 0, s, w, ids, n_rows, out, K);
    else if (wt == kWF16)
      hipLaunchKernelGGL(float_rows_kernel<kWF16>, grid, dim3(256), 0, s, w, ids, n_rows, out, K);
    else
      hipLaunchKernelGGL(float_rows_kernel<kWBF16>, grid, dim3(256), 0, s, w, ids, n_rows, out, K);
    return check_launch("get_rows");
  }
  int qk = 0, bb = 0;
  if (int rc = draco_gguf_block_info(ggml_type, &qk, &bb)) return rc;
  if (k % qk != 0)
    return set_error(DRACO_EINVAL_SHAPE, "row gather needs whole blocks per row: K %lld, block size %d",
                     (long long)k, qk);
  if ((uint64_t)(n_rows * (k / qk) * bb) > (uint64_t)w_bytes)
    return set_error(DRACO_EINVAL_SHAPE, "table holds %zu bytes, [%lld, %lld] of ggml type %d needs %lld", w_bytes,
                     (long long)n_rows, (long long)k, base, (long long)(n_rows * (k / qk) * bb));
  if (!al(w, 16) || !al(out, 16)) return set_error(DRACO_EINVAL_ARG, "w and out must be 16-byte aligned");
  return dequant_rows_dispatch(base, (ggml_type & DRACO_GGUF_GGML_ORDER) != 0, w, ids, n_rows, out, n_ids, k, s);
}

int draco_gguf_swiglu(const float* gate, const float* up, float* y, void* y_bf16, int64_t n, void* stream) {
  if (n < 1 || n > ((int64_t)1 << 40)) return set_error(DRACO_EINVAL_SHAPE, "invalid element count %lld", (long long)n);
  if (!al(gate, 4) || !al(up, 4)) return set_error(DRACO_EINVAL_ARG, "gate and up must be non-NULL, 4-byte aligned");
  if (!y && !y_bf16) return set_error(DRACO_EINVAL_ARG, "y and y_bf16 are both NULL");
  if ((y && !al(y, 4)) || (y_bf16 && !al(y_bf16, 2))) return set_error(DRACO_EINVAL_ARG, "y / y_bf16 misaligned");
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     gate, up, y, static_cast<uint16_t*>(y_bf16), n);
  return check_launch("swiglu");
}

}  // extern "C"
