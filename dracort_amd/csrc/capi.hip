// C ABI of libdraco_gguf.so: argument validation, error reporting and
// dispatch to the HIP kernels.  Declarations: include/draco_gguf.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "draco_internal.h"
#include "gguf_common.h"

namespace draco {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DRACO_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return DRACO_OK;
}

namespace {

struct TypeInfo {
  int base;
  bool d_last;
  int qk;
  int bytes;
};

int decode_type(int ggml_type, TypeInfo* t) {
  const int base = ggml_type & ~DRACO_GGUF_GGML_ORDER;
  const bool d_last = (ggml_type & DRACO_GGUF_GGML_ORDER) != 0;
  switch (base) {
    case kQ4_0: *t = {base, false, 32, 18}; break;
    case kQ4_1: *t = {base, false, 32, 20}; break;
    case kQ5_0: *t = {base, false, 32, 22}; break;
    case kQ5_1: *t = {base, false, 32, 24}; break;
    case kQ8_0: *t = {base, false, 32, 34}; break;
    case kQ8_K: *t = {base, false, 256, 258}; break;
    case kQ2_K: *t = {base, d_last, 256, 84}; break;
    case kQ3_K: *t = {base, d_last, 256, 110}; break;
    case kQ4_K: *t = {base, false, 256, 144}; break;
    case kQ5_K: *t = {base, false, 256, 176}; break;
    case kQ6_K: *t = {base, d_last, 256, 210}; break;
    default:
      return set_error(DRACO_EINVAL_QTYPE,
                       "GGUF quantization type %d is not supported by this build (supported: Q4_0=2, Q4_1=3, "
                       "Q5_0=6, Q5_1=7, Q8_0=8, Q2_K=10, Q3_K=11, Q4_K=12, Q5_K=13, Q6_K=14, Q8_K=15)",
                       ggml_type);
  }
  if (d_last && base != kQ2_K && base != kQ3_K && base != kQ6_K)
    return set_error(DRACO_EINVAL_QTYPE,
                     "layout flag DRACO_GGUF_GGML_ORDER only applies to Q2_K, Q3_K and Q6_K (got type %d)",
                     ggml_type);
  return DRACO_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Dimension limits: row and unit indices are 32-bit inside the kernels.
constexpr int64_t kMaxDim = (int64_t)1 << 30;

int check_matrix(const TypeInfo& t, int64_t n, int64_t k) {
  if (n <= 0 || k <= 0 || n > kMaxDim || k > kMaxDim)
    return set_error(DRACO_EINVAL_SHAPE, "invalid weight shape [%lld, %lld]", (long long)n, (long long)k);
  if (k % t.qk != 0)
    return set_error(DRACO_EINVAL_SHAPE, "GGUF row length %lld is not divisible by block size %d for ggml type %d",
                     (long long)k, t.qk, t.base);
  return DRACO_OK;
}

int check_bytes(const TypeInfo& t, int64_t n, int64_t k, size_t have, const char* name) {
  const int64_t need = n * (k / t.qk) * t.bytes;
  if ((uint64_t)need > (uint64_t)have)
    return set_error(DRACO_EINVAL_SHAPE, "%s holds %zu bytes but a [%lld, %lld] ggml type %d tensor needs %lld",
                     name, have, (long long)n, (long long)k, t.base, (long long)need);
  return DRACO_OK;
}

// [a, a + na) and [b, b + nb) overlap (NULL never overlaps)
bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  if (!a || !b) return false;
  const uintptr_t x0 = reinterpret_cast<uintptr_t>(a), y0 = reinterpret_cast<uintptr_t>(b);
  return x0 < y0 + nb && y0 < x0 + na;
}

int check_ptr(const void* p, const char* name) {
  if (p == nullptr) return set_error(DRACO_EINVAL_ARG, "%s is NULL", name);
  if (!aligned16(p)) return set_error(DRACO_EINVAL_ARG, "%s is not 16-byte aligned", name);
  return DRACO_OK;
}

// Scratch of draco_gguf_linear_noalloc: the Q4_K prefill GEMM's workspace
// (float16 activations, sub-block sums, row scales) for callers that cannot
// allocate.  One copy per GPU the library runs on, held until the process
// ends.  Host code never passes `scratch` itself (in host code it names a
// host-side stand-in): it takes each device's address from
// hipGetSymbolAddress once, with that device current, and passes that.
static __device__ __align__(256) unsigned char scratch[DRACO_GGUF_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 256;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];

// The current device's scratch address (looked up on the first call on that device).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(DRACO_EHIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices) return set_error(DRACO_EHIP, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(DRACO_EHIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       e != hipSuccess ? hipGetErrorString(e) : "NULL address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DRACO_OK;
}

}  // namespace
}  // namespace draco

using namespace draco;

extern "C" {

int draco_gguf_abi_version(void) { return 4; }

const char* draco_gguf_last_error(void) { return g_last_error; }

int draco_gguf_block_info(int ggml_type, int* qk, int* block_bytes) {
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (qk) *qk = t.qk;
  if (block_bytes) *block_bytes = t.bytes;
  return DRACO_OK;
}

int draco_gguf_dequant_f32(int ggml_type, const void* blocks, size_t blocks_bytes, float* out, int64_t n_rows,
                           int64_t k, void* stream) {
  g_last_error[0] = 0;
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  // Blocks may run across rows: the reference only needs n_rows * k to be a
  // multiple of the block size (draco/format/gguf.py:292-296).  Such a
  // tensor is one flat row of n_rows * k values (same output layout).
  if (n_rows > 0 && k > 0 && n_rows <= kMaxDim && k <= kMaxDim && k % t.qk != 0 && (n_rows * k) % t.qk == 0) {
    if (n_rows * k > kMaxDim)
      return set_error(DRACO_EINVAL_SHAPE, "a tensor whose blocks run across rows holds at most %lld values",
                       (long long)kMaxDim);
    k *= n_rows;
    n_rows = 1;
  }
  if (int rc = check_matrix(t, n_rows, k)) return rc;
  if (int rc = check_bytes(t, n_rows, k, blocks_bytes, "blocks")) return rc;
  if (int rc = check_ptr(blocks, "blocks")) return rc;
  if (int rc = check_ptr(out, "out")) return rc;
  return dequant_dispatch(t.base, t.d_last, blocks, out, n_rows, k, static_cast<hipStream_t>(stream));
}

int draco_gguf_gemv(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype, const float* bias,
                    float* y, int64_t m, int64_t n, int64_t k, void* stream) {
  g_last_error[0] = 0;
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (int rc = check_matrix(t, n, k)) return rc;
  if (int rc = check_bytes(t, n, k, w_bytes, "w")) return rc;
  if (m < 1 || m > 16)
    return set_error(DRACO_EINVAL_SHAPE, "GEMV takes 1..16 activation rows, got %lld", (long long)m);
  if (x_dtype != DRACO_DTYPE_F32 && x_dtype != DRACO_DTYPE_BF16)
    return set_error(DRACO_EINVAL_ARG, "unknown activation dtype %d", x_dtype);
  if (int rc = check_ptr(w, "w")) return rc;
  if (int rc = check_ptr(x, "x")) return rc;
  if (int rc = check_ptr(y, "y")) return rc;
  return gemv_dispatch(t.base, t.d_last, w, x, x_dtype == DRACO_DTYPE_BF16, bias, y, (int)m, (int)n, (int)k,
                       static_cast<hipStream_t>(stream));
}

int draco_gguf_gemv_multi(int ggml_type, int n_mats, const void* const* w, const size_t* w_bytes,
                          const int64_t* n, float* const* y, void* const* y_bf16, const void* x, int x_dtype,
                          int64_t m, int64_t k, void* stream) {
  g_last_error[0] = 0;
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (n_mats < 1 || n_mats > 4) return set_error(DRACO_EINVAL_ARG, "n_mats must be 1..4, got %d", n_mats);
  if (!w || !w_bytes || !n) return set_error(DRACO_EINVAL_ARG, "w, w_bytes and n must not be NULL");
  if (m < 1 || m > 16)
    return set_error(DRACO_EINVAL_SHAPE, "GEMV takes 1..16 activation rows, got %lld", (long long)m);
  if (x_dtype != DRACO_DTYPE_F32 && x_dtype != DRACO_DTYPE_BF16)
    return set_error(DRACO_EINVAL_ARG, "unknown activation dtype %d", x_dtype);
  if (int rc = check_ptr(x, "x")) return rc;
  const size_t xbytes = (size_t)m * k * (x_dtype == DRACO_DTYPE_BF16 ? 2 : 4);
  int ns[4];
  int64_t total = 0;
  float* ys[4] = {nullptr, nullptr, nullptr, nullptr};
  uint16_t* ybs[4] = {nullptr, nullptr, nullptr, nullptr};
  for (int i = 0; i < n_mats; ++i) {
    if (int rc = check_matrix(t, n[i], k)) return rc;
    if (int rc = check_bytes(t, n[i], k, w_bytes[i], "w[i]")) return rc;
    if (int rc = check_ptr(w[i], "w[i]")) return rc;
    ys[i] = y ? y[i] : nullptr;
    ybs[i] = y_bf16 ? static_cast<uint16_t*>(y_bf16[i]) : nullptr;
    if (!ys[i] && !ybs[i]) return set_error(DRACO_EINVAL_ARG, "matrix %d has neither y nor y_bf16", i);
    if (ys[i] && (reinterpret_cast<uintptr_t>(ys[i]) & 3u)) return set_error(DRACO_EINVAL_ARG, "y[%d] misaligned", i);
    if (ybs[i] && (reinterpret_cast<uintptr_t>(ybs[i]) & 1u))
      return set_error(DRACO_EINVAL_ARG, "y_bf16[%d] misaligned", i);
    if (overlaps(x, xbytes, ys[i], (size_t)m * n[i] * 4) || overlaps(x, xbytes, ybs[i], (size_t)m * n[i] * 2))
      return set_error(DRACO_EINVAL_ARG, "x overlaps an output of matrix %d", i);
    ns[i] = (int)n[i];
    total += n[i];
  }
  if (total > kMaxDim) return set_error(DRACO_EINVAL_SHAPE, "too many rows in one launch");
  return gemv_multi_dispatch(t.base, t.d_last, n_mats, w, ns, ys, ybs, x, x_dtype == DRACO_DTYPE_BF16, nullptr,
                             (int)m, (int)k, static_cast<hipStream_t>(stream));
}

int draco_gguf_gemv_swiglu(int ggml_type, const void* w_gate, const void* w_up, size_t w_bytes, const void* x,
                           int x_dtype, float* y, void* y_bf16, int64_t m, int64_t n, int64_t k, void* stream) {
  g_last_error[0] = 0;
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (int rc = check_matrix(t, n, k)) return rc;
  if (int rc = check_bytes(t, n, k, w_bytes, "w")) return rc;
  if (m < 1 || m > 16)
    return set_error(DRACO_EINVAL_SHAPE, "GEMV takes 1..16 activation rows, got %lld", (long long)m);
  if (x_dtype != DRACO_DTYPE_F32 && x_dtype != DRACO_DTYPE_BF16)
    return set_error(DRACO_EINVAL_ARG, "unknown activation dtype %d", x_dtype);
  if (int rc = check_ptr(w_gate, "w_gate")) return rc;
  if (int rc = check_ptr(w_up, "w_up")) return rc;
  if (int rc = check_ptr(x, "x")) return rc;
  if (!y && !y_bf16) return set_error(DRACO_EINVAL_ARG, "y and y_bf16 are both NULL");
  if ((reinterpret_cast<uintptr_t>(y) & 3u) || (reinterpret_cast<uintptr_t>(y_bf16) & 1u))
    return set_error(DRACO_EINVAL_ARG, "y / y_bf16 misaligned");
  const size_t xbytes = (size_t)m * k * (x_dtype == DRACO_DTYPE_BF16 ? 2 : 4);
  if (overlaps(x, xbytes, y, (size_t)m * n * 4) || overlaps(x, xbytes, y_bf16, (size_t)m * n * 2))
    return set_error(DRACO_EINVAL_ARG, "x overlaps an output");
  return gemv_swiglu_dispatch(t.base, t.d_last, w_gate, w_up, y, static_cast<uint16_t*>(y_bf16), x,
                              x_dtype == DRACO_DTYPE_BF16, (int)m, (int)n, (int)k, static_cast<hipStream_t>(stream));
}

static int gemv_residual_impl(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype, float* resid,
                              void* resid_bf16, int64_t m, int64_t n, int64_t k, void* workspace,
                              size_t workspace_bytes, void* stream) {
  g_last_error[0] = 0;
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (int rc = check_matrix(t, n, k)) return rc;
  if (int rc = check_bytes(t, n, k, w_bytes, "w")) return rc;
  if (m < 1 || m > 16)
    return set_error(DRACO_EINVAL_SHAPE, "GEMV takes 1..16 activation rows, got %lld", (long long)m);
  if (x_dtype != DRACO_DTYPE_F32 && x_dtype != DRACO_DTYPE_BF16)
    return set_error(DRACO_EINVAL_ARG, "unknown activation dtype %d", x_dtype);
  if (int rc = check_ptr(w, "w")) return rc;
  if (int rc = check_ptr(x, "x")) return rc;
  if (!resid || (reinterpret_cast<uintptr_t>(resid) & 3u))
    return set_error(DRACO_EINVAL_ARG, "resid is NULL or misaligned");
  if (reinterpret_cast<uintptr_t>(resid_bf16) & 1u) return set_error(DRACO_EINVAL_ARG, "resid_bf16 misaligned");
  const size_t xbytes = (size_t)m * k * (x_dtype == DRACO_DTYPE_BF16 ? 2 : 4);
  if (overlaps(x, xbytes, resid, (size_t)m * n * 4) || overlaps(x, xbytes, resid_bf16, (size_t)m * n * 2))
    return set_error(DRACO_EINVAL_ARG, "x overlaps resid / resid_bf16");
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return set_error(DRACO_EINVAL_ARG, "GEMV workspace must be 256-byte aligned");
  return gemv_resid_dispatch(t.base, t.d_last, w, x, x_dtype == DRACO_DTYPE_BF16, resid,
                             static_cast<uint16_t*>(resid_bf16), (int)m, (int)n, (int)k, workspace,
                             workspace ? workspace_bytes : 0, static_cast<hipStream_t>(stream));
}

int draco_gguf_gemv_residual(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype, float* resid,
                             void* resid_bf16, int64_t m, int64_t n, int64_t k, void* stream) {
  return gemv_residual_impl(ggml_type, w, w_bytes, x, x_dtype, resid, resid_bf16, m, n, k, nullptr, 0, stream);
}

size_t draco_gguf_gemv_residual_workspace_size(int ggml_type, int64_t m, int64_t n, int64_t k) {
  TypeInfo t;
  if (decode_type(ggml_type, &t) || m < 1 || m > 16 || n < 1 || k < 1 || n > kMaxDim || k > kMaxDim) return 0;
  return gemv_resid_split_bytes(t.base, (int)m, (int)n, (int)k);
}

int draco_gguf_gemv_residual_ws(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype,
                                float* resid, void* resid_bf16, int64_t m, int64_t n, int64_t k, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return gemv_residual_impl(ggml_type, w, w_bytes, x, x_dtype, resid, resid_bf16, m, n, k, workspace,
                            workspace_bytes, stream);
}

// shared checks of the fused-RMSNorm entry points: x [m, k] float32, norm_w [k], x_norm [m, k] bf16
static int check_norm_args(const float* x, const float* norm_w, float eps, const void* x_norm, int64_t m, int64_t k) {
  if (int rc = check_ptr(x, "x")) return rc;
  if (int rc = check_ptr(norm_w, "norm_w")) return rc;
  if (int rc = check_ptr(x_norm, "x_norm")) return rc;
  if (!(eps >= 0.f)) return set_error(DRACO_EINVAL_ARG, "eps must be >= 0");
  if (overlaps(x, (size_t)m * k * 4, x_norm, (size_t)m * k * 2)) return set_error(DRACO_EINVAL_ARG, "x_norm overlaps x");
  return DRACO_OK;
}

int draco_gguf_gemv_multi_rmsnorm(int ggml_type, int n_mats, const void* const* w, const size_t* w_bytes,
                                  const int64_t* n, float* const* y, void* const* y_bf16, const float* x,
                                  const float* norm_w, float eps, void* x_norm, int64_t m, int64_t k, void* stream) {
  g_last_error[0] = 0;
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (n_mats < 1 || n_mats > 4) return set_error(DRACO_EINVAL_ARG, "n_mats must be 1..4, got %d", n_mats);
  if (!w || !w_bytes || !n) return set_error(DRACO_EINVAL_ARG, "w, w_bytes and n must not be NULL");
  if (m < 1 || m > 16)
    return set_error(DRACO_EINVAL_SHAPE, "GEMV takes 1..16 activation rows, got %lld", (long long)m);
  if (int rc = check_norm_args(x, norm_w, eps, x_norm, m, k)) return rc;
  int ns[4];
  int64_t total = 0;
  float* ys[4] = {nullptr, nullptr, nullptr, nullptr};
  uint16_t* ybs[4] = {nullptr, nullptr, nullptr, nullptr};
  for (int i = 0; i < n_mats; ++i) {
    if (int rc = check_matrix(t, n[i], k)) return rc;
    if (int rc = check_bytes(t, n[i], k, w_bytes[i], "w[i]")) return rc;
    if (int rc = check_ptr(w[i], "w[i]")) return rc;
    ys[i] = y ? y[i] : nullptr;
    ybs[i] = y_bf16 ? static_cast<uint16_t*>(y_bf16[i]) : nullptr;
    if (!ys[i] && !ybs[i]) return set_error(DRACO_EINVAL_ARG, "matrix %d has neither y nor y_bf16", i);
    if (ys[i] && (reinterpret_cast<uintptr_t>(ys[i]) & 3u)) return set_error(DRACO_EINVAL_ARG, "y[%d] misaligned", i);
    if (ybs[i] && (reinterpret_cast<uintptr_t>(ybs[i]) & 1u))
      return set_error(DRACO_EINVAL_ARG, "y_bf16[%d] misaligned", i);
    for (const void* in : {static_cast<const void*>(x), static_cast<const void*>(x_norm)}) {
      const size_t nb = in == x ? (size_t)m * k * 4 : (size_t)m * k * 2;
      if (overlaps(in, nb, ys[i], (size_t)m * n[i] * 4) || overlaps(in, nb, ybs[i], (size_t)m * n[i] * 2))
        return set_error(DRACO_EINVAL_ARG, "x or x_norm overlaps an output of matrix %d", i);
    }
    ns[i] = (int)n[i];
    total += n[i];
  }
  if (total > kMaxDim) return set_error(DRACO_EINVAL_SHAPE, "too many rows in one launch");
  return gemv_multi_norm_dispatch(t.base, t.d_last, n_mats, w, ns, ys, ybs, x, norm_w, eps,
                                  static_cast<uint16_t*>(x_norm), (int)m, (int)k, static_cast<hipStream_t>(stream));
}

int draco_gguf_gemv_swiglu_rmsnorm(int ggml_type, const void* w_gate, const void* w_up, size_t w_bytes,
                                   const float* x, const float* norm_w, float eps, void* x_norm, float* y,
                                   void* y_bf16, int64_t m, int64_t n, int64_t k, void* stream) {
  g_last_error[0] = 0;
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (int rc = check_matrix(t, n, k)) return rc;
  if (int rc = check_bytes(t, n, k, w_bytes, "w")) return rc;
  if (m < 1 || m > 16)
    return set_error(DRACO_EINVAL_SHAPE, "GEMV takes 1..16 activation rows, got %lld", (long long)m);
  if (int rc = check_ptr(w_gate, "w_gate")) return rc;
  if (int rc = check_ptr(w_up, "w_up")) return rc;
  if (int rc = check_norm_args(x, norm_w, eps, x_norm, m, k)) return rc;
  if (!y && !y_bf16) return set_error(DRACO_EINVAL_ARG, "y and y_bf16 are both NULL");
  if ((reinterpret_cast<uintptr_t>(y) & 3u) || (reinterpret_cast<uintptr_t>(y_bf16) & 1u))
    return set_error(DRACO_EINVAL_ARG, "y / y_bf16 misaligned");
  for (const void* in : {static_cast<const void*>(x), static_cast<const void*>(x_norm)}) {
    const size_t nb = in == x ? (size_t)m * k * 4 : (size_t)m * k * 2;
    if (overlaps(in, nb, y, (size_t)m * n * 4) || overlaps(in, nb, y_bf16, (size_t)m * n * 2))
      return set_error(DRACO_EINVAL_ARG, "x or x_norm overlaps an output");
  }
  return gemv_swiglu_norm_dispatch(t.base, t.d_last, w_gate, w_up, y, static_cast<uint16_t*>(y_bf16), x, norm_w, eps,
                                   static_cast<uint16_t*>(x_norm), (int)m, (int)n, (int)k,
                                   static_cast<hipStream_t>(stream));
}

size_t draco_gguf_gemm_workspace_size(int ggml_type, int64_t m, int64_t k) {
  TypeInfo t;
  if (decode_type(ggml_type, &t) || m < 1 || k < 1) return 0;
  return gemm_workspace_size(t.base, m, k);
}

int draco_gguf_gemm(int ggml_type, const void* w, size_t w_bytes, const void* x_bf16, const float* bias, float* y,
                    int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error[0] = 0;
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (int rc = check_matrix(t, n, k)) return rc;
  if (int rc = check_bytes(t, n, k, w_bytes, "w")) return rc;
  if (m < 1 || m > kMaxDim) return set_error(DRACO_EINVAL_SHAPE, "invalid token count %lld", (long long)m);
  if (int rc = check_ptr(w, "w")) return rc;
  if (int rc = check_ptr(x_bf16, "x")) return rc;
  if (int rc = check_ptr(y, "y")) return rc;
  if (workspace) {
    const size_t need = gemm_workspace_min(t.base, m, k);
    if (workspace_bytes < need)
      return set_error(DRACO_EWORKSPACE, "GEMM workspace needs %zu bytes, got %zu", need, workspace_bytes);
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
      return set_error(DRACO_EINVAL_ARG, "GEMM workspace must be 256-byte aligned");
  }
  return gemm_dispatch(t.base, t.d_last, w, x_bf16, bias, y, (int)m, (int)n, (int)k, workspace, workspace_bytes,
                       static_cast<hipStream_t>(stream));
}

int draco_gguf_linear(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype, const float* bias,
                      float* y, int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (m >= 1 && m <= 16) return draco_gguf_gemv(ggml_type, w, w_bytes, x, x_dtype, bias, y, m, n, k, stream);
  if (x_dtype == DRACO_DTYPE_BF16)
    return draco_gguf_gemm(ggml_type, w, w_bytes, x, bias, y, m, n, k, workspace, workspace_bytes, stream);
  g_last_error[0] = 0;
  if (m < 1 || m > kMaxDim) return set_error(DRACO_EINVAL_SHAPE, "invalid token count %lld", (long long)m);
  if (x_dtype != DRACO_DTYPE_F32) return set_error(DRACO_EINVAL_ARG, "unknown activation dtype %d", x_dtype);
  // float32 activations, many rows: 16-row GEMV tiles.  Tile row offsets keep x and y 16-byte
  // aligned: m0 is a multiple of 16, so x + m0 k and y + m0 n move by multiples of 64 bytes.
  for (int64_t m0 = 0; m0 < m; m0 += 16) {
    const int64_t mt = m - m0 < 16 ? m - m0 : 16;
    const float* xt = static_cast<const float*>(x) + m0 * k;
    int rc = draco_gguf_gemv(ggml_type, w, w_bytes, xt, x_dtype, bias, y + m0 * n, mt, n, k, stream);
    if (rc) return rc;
  }
  return DRACO_OK;
}

int draco_gguf_linear_noalloc(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype,
                              const float* bias, float* y, int64_t m, int64_t n, int64_t k, void* stream) {
  g_last_error[0] = 0;
  // the GEMV (m <= 16) and the float32 16-row tiles use no workspace
  if ((m >= 1 && m <= 16) || x_dtype != DRACO_DTYPE_BF16)
    return draco_gguf_linear(ggml_type, w, w_bytes, x, x_dtype, bias, y, m, n, k, nullptr, 0, stream);
  TypeInfo t;
  if (int rc = decode_type(ggml_type, &t)) return rc;
  if (m < 1 || m > kMaxDim || k < 1 || k > kMaxDim)
    return set_error(DRACO_EINVAL_SHAPE, "invalid token count %lld or row length %lld", (long long)m, (long long)k);
  const size_t need = gemm_workspace_min(t.base, m, k);
  if (need == 0)  // this type's GEMM needs no workspace
    return draco_gguf_gemm(ggml_type, w, w_bytes, x, bias, y, m, n, k, nullptr, 0, stream);
  if (need > (size_t)DRACO_GGUF_NOALLOC_SCRATCH_BYTES)
    return set_error(DRACO_EWORKSPACE,
                     "draco_gguf_linear_noalloc: %lld rows of length %lld need %zu bytes of scratch, above its %zu-byte "
                     "maximum (split the rows, or call draco_gguf_linear with a workspace)",
                     (long long)m, (long long)k, need, (size_t)DRACO_GGUF_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_for_current_device(&ws)) return rc;
  return draco_gguf_gemm(ggml_type, w, w_bytes, x, bias, y, m, n, k, ws, (size_t)DRACO_GGUF_NOALLOC_SCRATCH_BYTES,
                         stream);
}

}  // extern "C"
