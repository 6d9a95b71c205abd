// Persistent streaming GEMV for decode (1..16 activation rows) on gfx950, plus
// the fused launches of a decode layer.
//
// Grid: sized from the occupancy of the kernel, so every wave is resident from
// the start.  Each wave owns rows r = wave, wave + W, wave + 2W, ... (W = all
// waves) and walks them as one continuous sequence of steps; step s covers
// 64 units (one per lane) of K of one row.  The packed weight bytes of steps
// s + 1 and s + 2 are loaded while step s is multiplied, across row
// boundaries, so a wave keeps ~2 x 2 KB in flight from its first to its last
// row instead of paying a load latency per row.  Activations are staged in
// LDS once per workgroup when they fit (MT * k * sizeof(x) <= 64 KB; their
// reads then do not queue behind the weight loads), else read from global
// memory.  The number of waves is chosen so every wave gets the same number
// of rows (no tail of waves with one extra row).
//
// Modes (one launch each):
//   kPlain   up to 4 matrices sharing x (e.g. q, k, v): their rows are
//            concatenated; y_i = W_i x (+ bias), optional bf16 copy of y_i.
//   kSwiGLU  gate and up: each step multiplies the same row of both;
//            y = silu(W_gate x) * (W_up x), float32 and/or bf16.
//   kResid   resid += W x (float32, in place), optional bf16 copy of resid.
// These replace the reference executor's _qkv, _mlp and _o_proj plus the
// residual adds of forward_step (draco/runtime/cpu/executor.py:208-277,
// 290-342), each of which is one or more _linear calls and numpy glue there.
#pragma once

#include <stdlib.h>

#include <algorithm>

#include "draco_internal.h"
#include "gemv_core.h"

namespace draco {

enum StreamMode : int { kPlain = 0, kSwiGLU = 1, kResid = 2 };

constexpr int kMaxMats = 4;

struct StreamJob {
  const uint8_t* w[kMaxMats];
  float* y[kMaxMats];
  uint16_t* yb[kMaxMats];
  int n[kMaxMats];
  int n_mats;
  int rows;          // rows walked: sum of n (kPlain) or n[0] (kSwiGLU / kResid)
  int64_t row_bytes;
  int k, m;
  const void* x;
  const float* bias;  // kPlain with one matrix only
  float* resid;
  uint16_t* resid_bf16;
  // fused RMSNorm of the input (persistent single-token kernels only): x is
  // float32, normalized with norm_w / norm_eps in the prologue; workgroup 0
  // also stores the normalized bf16 row to x_norm
  const float* norm_w;
  float norm_eps;
  uint16_t* x_norm;
  // bytes between activation rows (0: k elements); set when the launch covers a
  // K window of longer rows (streaming kernel with the activations in LDS only)
  int64_t x_stride;
  // split K (matrix-core kernel, kPlain / kResid with one matrix): grid.y
  // workgroups per tile, split s taking chunks [s split_chunks, (s + 1)
  // split_chunks); each stores its raw 16 x 16 sums to part[s][m][n] and a
  // second launch adds the splits in order (nullptr: no split)
  float* part;
  int split_chunks;
};

// Element i (0..3) of four values by a chain of selects: indexing an array of
// the kernel argument with a run-time index makes the compiler copy the
// argument to scratch memory and load from there.
template <class T>
__device__ __forceinline__ T pick4(int i, T a, T b, T c, T d) {
  T v = a;
  v = i >= 1 ? b : v;
  v = i >= 2 ? c : v;
  v = i >= 3 ? d : v;
  return v;
}

// Row r of this launch -> (matrix, row within it); rows of the matrices of a
// kPlain launch are concatenated.
__device__ __forceinline__ void row_of(const StreamJob& j, int r, int& mat, int& lrow) {
  mat = 0;
  lrow = r;
#pragma unroll
  for (int i = 0; i < kMaxMats - 1; ++i) {
    if (mat == i && i < j.n_mats - 1 && lrow >= j.n[i]) {
      lrow -= j.n[i];
      mat = i + 1;
    }
  }
}

// Bytes of one step (64 units) of a row, and of the part of it before the
// lane's unit: with K / 32 a multiple of 64 a lane always decodes the same
// position inside a step, so its field offsets are per-lane constants.
template <int QT> struct StepGeom {
  static constexpr int STEP_BYTES = 64 * Fmt<QT>::BYTES / Fmt<QT>::UPB;
};

// Walks (row, K-step) steps with two steps of weight loads in flight.
//  * Every wave walks rows_per_wave rows (rows past the end are clamped to
//    the last row and not stored) and every lane loads every step (FULL: the
//    row is a whole number of steps; otherwise lanes past the row end re-read
//    the last unit and add nothing), so loads are never predicated.
//  * Nothing inside the loop writes global memory: row sums are parked in LDS
//    and stored after the loop.
// Both keep the vector-memory wait counts exact: the math of step s waits only
// for step s's own loads.
constexpr int kPrefetch = 4;  // steps of weight loads in flight per wave

template <int QT, bool DL, int MT, bool XBF16, int MODE, bool XLDS, bool FULL>
__global__ __launch_bounds__(256) void gemv_stream_kernel(StreamJob job, int rows_per_wave) {
  constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  constexpr int G = Fmt<QT>::G;
  constexpr int STEP_BYTES = StepGeom<QT>::STEP_BYTES;
  extern __shared__ uint4 smem[];
  const int lane = threadIdx.x & 63;
  // wave-uniform indices kept in scalar registers: the row / matrix selection
  // then uses scalar loads of the pointer table instead of vector loads
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = gridDim.x * (blockDim.x >> 6);
  const int wave = blockIdx.x * (blockDim.x >> 6) + wid;
  const int k = job.k;
  const int units = k >> 5;
  const int iters = (units + 63) >> 6;  // steps per row
  const size_t xstride = job.x_stride ? (size_t)job.x_stride : XBF16 ? (size_t)k * 2 : (size_t)k * 4;
  const uint8_t* xb = static_cast<const uint8_t*>(job.x);

  // LDS: [x rows (XLDS)][group sums (XLDS)][per-wave row results]
  const int x_chunks = XLDS ? MT * k * (XBF16 ? 2 : 4) / 16 : 0;
  float* xsum = reinterpret_cast<float*>(smem + x_chunks);
  const int xsum_floats = XLDS ? (MT * units * G + 3) & ~3 : 0;
  float* res = xsum + xsum_floats + (size_t)wid * rows_per_wave * MT;
  const uint4* xsrc = XLDS ? smem : static_cast<const uint4*>(job.x);
  const bool active = wave < job.rows;

  // matrix base and byte offset of row index i of this wave (clamped to the
  // last row).  Loads compute dword alignment from the offset relative to the
  // 16-byte aligned matrix base: with an odd number of 34 / 18 / 210-byte
  // blocks per row a row start is only 2-byte aligned.
  auto row_at = [&](int i, int r, const uint8_t*& base, int64_t& off) {
    int grow = wave + i * nw;
    grow = grow < job.rows ? grow : job.rows - 1;
    int mat = 0, lrow = grow;
    if constexpr (MODE == kPlain) {
      if (job.n_mats > 1) {
#pragma unroll
        for (int q = 0; q < kMaxMats - 1; ++q) {
          if (mat == q && q < job.n_mats - 1 && lrow >= job.n[q]) {
            lrow -= job.n[q];
            mat = q + 1;
          }
        }
      }
    }
    base = pick4(NR == 2 ? r : mat, job.w[0], job.w[1], job.w[2], job.w[3]);
    off = (int64_t)lrow * job.row_bytes;
  };

  // load cursor
  int l_i = 0, l_it = 0;
  const uint8_t* lbase[NR];
  int64_t loff[NR];
  __amdgpu_buffer_rsrc_t lrsrc[NR];
  auto set_row = [&](int i) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      row_at(i, r, lbase[r], loff[r]);
      if constexpr (FULL) {
        // whole-matrix buffer: byte size from the owning matrix's row count
        int rows_m = job.n[0];
        if constexpr (MODE == kPlain) {
          if (job.n_mats > 1) {
#pragma unroll
            for (int q = 1; q < kMaxMats; ++q)
              if (lbase[r] == job.w[q]) rows_m = job.n[q];
          }
        }
        lrsrc[r] = make_rsrc(lbase[r], (uint32_t)((int64_t)rows_m * job.row_bytes));
      }
    }
  };
  set_row(0);
  auto load_step = [&](Raw<QT>(&dst)[NR]) {
    if constexpr (FULL) {
      // whole steps: the row offset and STEP_BYTES are multiples of 4 and go
      // in the scalar offset; the lane's fields sit at per-lane constant
      // offsets (unit index `lane` inside the step)
#pragma unroll
      for (int r = 0; r < NR; ++r)
        dst[r] = load_unit_l<QT, DL>(BufferLoader{lrsrc[r], (int)(loff[r] + (int64_t)l_it * STEP_BYTES)}, 0, lane);
    } else {
      const int u = min(lane + 64 * l_it, units - 1);
#pragma unroll
      for (int r = 0; r < NR; ++r) dst[r] = load_unit<QT, DL>(lbase[r], loff[r], u);
    }
    if (++l_it == iters) {
      l_it = 0;
      ++l_i;
      set_row(l_i < rows_per_wave ? l_i : rows_per_wave - 1);
    }
  };

  constexpr int NB = kPrefetch + 1;
  Raw<QT> buf[NB][NR];
  float acc[NR][MT];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[r][mi] = 0.f;

  int c_i = 0, c_it = 0;  // compute cursor
  const int steps = rows_per_wave * iters;
  auto compute_step = [&](const Raw<QT>(&cur)[NR]) {
    if (c_i < rows_per_wave) {
      if constexpr (FULL) {
        // the lane's unit index inside the step is `lane`; x offsets move by 2048 per step
        const int u = lane + 64 * c_it;
        unit_math_lds<QT, MT, XBF16, NR, XLDS, XLDS>(cur, u, job.m, k, xsrc, acc, xsum);
      } else {
        const int u = lane + 64 * c_it;
        if (u < units) unit_math_lds<QT, MT, XBF16, NR, XLDS>(cur, u, job.m, k, xsrc, acc, xsum);
      }
      if (c_it == iters - 1) {
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
          float v[NR];
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            v[r] = wave_sum_dpp(acc[r][mi]);
            acc[r][mi] = 0.f;
          }
          float out = v[0];
          if constexpr (MODE == kSwiGLU) out = silu(v[0]) * v[1];
          if (lane == 0) res[c_i * MT + mi] = out;
        }
      }
      if (++c_it == iters) {
        c_it = 0;
        ++c_i;
      }
    }
  };

  // the first weight loads go out before the activations are staged, so the
  // staging latency overlaps theirs instead of preceding it
  if (active) {
#pragma unroll
    for (int b = 0; b < kPrefetch; ++b) load_step(buf[b]);
  }
  if constexpr (XLDS) {
    auto xrow = [&](int mi) { return (const void*)(xb + (size_t)mi * xstride); };
    if constexpr (FULL) {
      stage_x_lds_perm<QT, MT, XBF16>(smem, job.m, k, xrow);
      stage_group_sums_perm<QT, MT, XBF16>(smem, xsum, job.m, k);
    } else {
      stage_x_lds<MT, XBF16>(smem, job.m, k, xrow);
      stage_group_sums<QT, MT, XBF16>(smem, xsum, job.m, k);
    }
  }
  if (!active) return;
  for (int s0 = 0; s0 < steps; s0 += NB) {
    // (fully unrolled: a run-time index into buf would put buf in scratch)
#pragma clang loop unroll(full)
    for (int b = 0; b < NB; ++b) {
      load_step(buf[(b + kPrefetch) % NB]);
      compute_step(buf[b]);
    }
  }

  // epilogue: write this wave's rows (lane t handles (row, m) pairs t, t + 64, ...)
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0);
  for (int t = lane; t < rows_per_wave * MT; t += 64) {
    const int ri = t / MT, mi = t - ri * MT;
    const int grow = wave + ri * nw;
    if (mi >= job.m || grow >= job.rows) continue;
    const float v = res[t];
    int mat = 0, lrow = grow;
    if constexpr (MODE == kPlain) {
#pragma unroll
      for (int q = 0; q < kMaxMats - 1; ++q) {
        if (mat == q && q < job.n_mats - 1 && lrow >= job.n[q]) {
          lrow -= job.n[q];
          mat = q + 1;
        }
      }
    }
    const int n = pick4(mat, job.n[0], job.n[1], job.n[2], job.n[3]);
    const size_t o = (size_t)mi * n + lrow;
    if constexpr (MODE == kResid) {
      const float out = job.resid[o] + v;
      job.resid[o] = out;
      if (job.resid_bf16) job.resid_bf16[o] = f32_to_bf16_rne(out);
    } else {
      const float out = v + ((MODE == kPlain && job.bias) ? job.bias[lrow] : 0.f);
      float* const yp = pick4(mat, job.y[0], job.y[1], job.y[2], job.y[3]);
      uint16_t* const ybp = pick4(mat, job.yb[0], job.yb[1], job.yb[2], job.yb[3]);
      if (yp) yp[o] = out;
      if (ybp) ybp[o] = f32_to_bf16_rne(out);
    }
  }
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------

inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

constexpr size_t kStreamMaxLds = 64 * 1024;

inline int64_t row_bytes_of(int qtype, int k) {
  switch (qtype) {
    case kQ8_0: return (int64_t)(k / 32) * 34;
    case kQ4_0: return (int64_t)(k / 32) * 18;
    case kQ4_1: return (int64_t)(k / 32) * 20;
    case kQ5_0: return (int64_t)(k / 32) * 22;
    case kQ5_1: return (int64_t)(k / 32) * 24;
    case kQ8_K: return (int64_t)(k / 256) * 258;
    case kQ2_K: return (int64_t)(k / 256) * 84;
    case kQ3_K: return (int64_t)(k / 256) * 110;
    case kQ4_K: return (int64_t)(k / 256) * 144;
    case kQ5_K: return (int64_t)(k / 256) * 176;
    default: return (int64_t)(k / 256) * 210;
  }
}

template <int QT, bool DL, int MT, bool XBF16, int MODE, bool XLDS, bool FULL>
static int launch_stream(const StreamJob& job, hipStream_t s) {
  auto kern = gemv_stream_kernel<QT, DL, MT, XBF16, MODE, XLDS, FULL>;
  const int units = job.k / 32;
  const size_t xlds = XLDS ? (size_t)MT * job.k * (XBF16 ? 2 : 4) +
                                 (size_t)((MT * units * Fmt<QT>::G + 3) & ~3) * sizeof(float)
                           : 0;
  static int per_cu[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (per_cu[dev] == 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kern, 256, 0) != hipSuccess || v <= 0) v = 1;
    per_cu[dev] = v;
  }
  // Workgroups per CU: few long-lived waves, each with kPrefetch steps of
  // loads in flight, beat many short ones (the per-wave prologue and first
  // load latency are then paid rarely).  DRACO_GEMV_WGS_PER_CU overrides the
  // default for tuning; the occupancy and LDS bounds always apply.
  static int wgs_target = -1;
  if (wgs_target < 0) {
    const char* e = getenv("DRACO_GEMV_WGS_PER_CU");
    wgs_target = (e && atoi(e) > 0) ? atoi(e) : 2;
  }
  int wgs_per_cu = std::min(per_cu[dev], wgs_target);
  int rows_per_wave = 1;
  size_t lds = 0;
  for (int pass = 0; pass < 2; ++pass) {
    const int cap_waves = device_cus() * std::max(1, wgs_per_cu) * 4;
    rows_per_wave = (job.rows + cap_waves - 1) / cap_waves;
    lds = xlds + (size_t)4 * rows_per_wave * MT * sizeof(float);
    wgs_per_cu = std::max(1, std::min(wgs_per_cu, (int)((160 * 1024) / lds)));
  }
  const int waves = (job.rows + rows_per_wave - 1) / rows_per_wave;
  const int blocks = (waves + 3) / 4;
  if (lds > 160 * 1024) return set_error(DRACO_EINVAL_SHAPE, "GEMV launch needs %zu bytes of LDS", lds);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, s, job, rows_per_wave);
  return check_launch("gemv_stream");
}

template <int QT, bool DL, int MT, bool XBF16, int MODE>
static int launch_stream_x(const StreamJob& job, hipStream_t s) {
  // whole-step fast path: K / 32 a multiple of 64 and every matrix addressable
  // with 32-bit buffer offsets
  bool full = (job.k / 32) % 64 == 0;
  for (int i = 0; i < job.n_mats; ++i)
    if ((int64_t)job.n[i] * job.row_bytes >= ((int64_t)1 << 31)) full = false;
  if ((size_t)MT * job.k * (XBF16 ? 2 : 4) <= kStreamMaxLds) {
    if (full) return launch_stream<QT, DL, MT, XBF16, MODE, true, true>(job, s);
    return launch_stream<QT, DL, MT, XBF16, MODE, true, false>(job, s);
  }
  // the global-memory activation path indexes rows by k: a K window (x_stride
  // set) must fit the LDS image
  if (job.x_stride) return set_error(DRACO_EINVAL_SHAPE, "K window of %d columns does not fit the activation image", job.k);
  if (full) return launch_stream<QT, DL, MT, XBF16, MODE, false, true>(job, s);
  return launch_stream<QT, DL, MT, XBF16, MODE, false, false>(job, s);
}

template <int QT, bool DL, int MODE, bool XBF16>
static int stream_mt(const StreamJob& job, hipStream_t s) {
  if (job.m <= 1) return launch_stream_x<QT, DL, 1, XBF16, MODE>(job, s);
  if (job.m <= 2) return launch_stream_x<QT, DL, 2, XBF16, MODE>(job, s);
  if (job.m <= 4) return launch_stream_x<QT, DL, 4, XBF16, MODE>(job, s);
  if (job.m <= 8) return launch_stream_x<QT, DL, 8, XBF16, MODE>(job, s);
  return launch_stream_x<QT, DL, 16, XBF16, MODE>(job, s);
}

// Q4_1 Q5_0 Q5_1 Q8_K Q2_K Q3_K Q5_K: the same streaming kernel with fewer
// activation-row tiles (1, 4, 16), one translation unit per mode
// (gemv_ext_*.hip) so they compile in parallel with the rest.
int stream_ext_plain(int qtype, bool d_last, const StreamJob& job, bool xbf16, hipStream_t s);
int stream_ext_swiglu(int qtype, bool d_last, const StreamJob& job, bool xbf16, hipStream_t s);
int stream_ext_resid(int qtype, bool d_last, const StreamJob& job, bool xbf16, hipStream_t s);

template <int QT, bool DL, int MODE, bool XBF16>
static int stream_mt_ext(const StreamJob& job, hipStream_t s) {
  if (job.m <= 1) return launch_stream_x<QT, DL, 1, XBF16, MODE>(job, s);
  if (job.m <= 4) return launch_stream_x<QT, DL, 4, XBF16, MODE>(job, s);
  return launch_stream_x<QT, DL, 16, XBF16, MODE>(job, s);
}

template <int MODE>
static int stream_ext_dispatch(int qtype, bool d_last, const StreamJob& job, bool xbf16, hipStream_t s) {
#define DRACO_EXT_CASE(QT)                                                                      \
  case QT:                                                                                      \
    return xbf16 ? stream_mt_ext<QT, false, MODE, true>(job, s) : stream_mt_ext<QT, false, MODE, false>(job, s);
#define DRACO_EXT_CASE_DL(QT)                                                                   \
  case QT:                                                                                      \
    if (d_last)                                                                                 \
      return xbf16 ? stream_mt_ext<QT, true, MODE, true>(job, s) : stream_mt_ext<QT, true, MODE, false>(job, s); \
    return xbf16 ? stream_mt_ext<QT, false, MODE, true>(job, s) : stream_mt_ext<QT, false, MODE, false>(job, s);
  switch (qtype) {
    DRACO_EXT_CASE(kQ4_1)
    DRACO_EXT_CASE(kQ5_0)
    DRACO_EXT_CASE(kQ5_1)
    DRACO_EXT_CASE(kQ8_K)
    DRACO_EXT_CASE(kQ5_K)
    DRACO_EXT_CASE_DL(kQ2_K)
    DRACO_EXT_CASE_DL(kQ3_K)
    default: return set_error(DRACO_EINVAL_QTYPE, "unsupported ggml type %d", qtype);
  }
#undef DRACO_EXT_CASE
#undef DRACO_EXT_CASE_DL
}

template <int MODE>
static int stream_dispatch(int qtype, bool d_last, const StreamJob& job, bool xbf16, hipStream_t s) {
  switch (qtype) {
    case kQ8_0: return xbf16 ? stream_mt<kQ8_0, false, MODE, true>(job, s) : stream_mt<kQ8_0, false, MODE, false>(job, s);
    case kQ4_0: return xbf16 ? stream_mt<kQ4_0, false, MODE, true>(job, s) : stream_mt<kQ4_0, false, MODE, false>(job, s);
    case kQ4_K: return xbf16 ? stream_mt<kQ4_K, false, MODE, true>(job, s) : stream_mt<kQ4_K, false, MODE, false>(job, s);
    case kQ6_K:
      if (d_last)
        return xbf16 ? stream_mt<kQ6_K, true, MODE, true>(job, s) : stream_mt<kQ6_K, true, MODE, false>(job, s);
      return xbf16 ? stream_mt<kQ6_K, false, MODE, true>(job, s) : stream_mt<kQ6_K, false, MODE, false>(job, s);
    default:
      if constexpr (MODE == kPlain) return stream_ext_plain(qtype, d_last, job, xbf16, s);
      if constexpr (MODE == kSwiGLU) return stream_ext_swiglu(qtype, d_last, job, xbf16, s);
      return stream_ext_resid(qtype, d_last, job, xbf16, s);
  }
}

// Activation rows too long for the LDS image (M * K * sizeof(x) > 64 KB, e.g.
// float32 rows of 4 x 14336 or 8 x 4096): without it the streaming kernel
// reads each lane's activations from global memory again for every row.
// Instead the launch is split into K windows of whole 2048-element steps, each
// small enough for the image: window w multiplies columns [k_w, k_w + K_w) of
// every row (the weight base moves by those columns' blocks, the row stride
// stays) with the same columns of x (x_stride keeps the full row).  The first
// window writes y (plain, with the bias) or adds into resid; every later one
// adds into that output through the residual epilogue; the bf16 copy is
// written by the last.  Single-matrix plain launches with a float32 output and
// residual launches only.
// The row tile MT the launch of this type will use (stream_mt / stream_mt_ext).
inline int stream_tile_rows(int qtype, int m) {
  const bool ext = !(qtype == kQ8_0 || qtype == kQ4_0 || qtype == kQ4_K || qtype == kQ6_K);
  if (ext) return m <= 1 ? 1 : m <= 4 ? 4 : 16;
  return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16;
}

inline int stream_window_k(int qtype, const StreamJob& job, bool xbf16) {
  const int mt = stream_tile_rows(qtype, job.m);
  const size_t xb = xbf16 ? 2 : 4;
  if ((size_t)mt * job.k * xb <= kStreamMaxLds || job.k % 2048 != 0) return 0;
  return (int)(kStreamMaxLds / ((size_t)mt * xb)) / 2048 * 2048;
}

template <int MODE>
static int stream_windowed(int qtype, bool d_last, const StreamJob& job, bool xbf16, int kw, hipStream_t s) {
  static_assert(MODE != kSwiGLU, "the SwiGLU epilogue is not additive");
  const size_t xb = xbf16 ? 2 : 4;
  for (int k0 = 0; k0 < job.k; k0 += kw) {
    const bool first = k0 == 0, last = k0 + kw >= job.k;
    StreamJob w = job;
    w.k = std::min(kw, job.k - k0);
    w.x = static_cast<const uint8_t*>(job.x) + (size_t)k0 * xb;
    w.x_stride = (int64_t)job.k * (int64_t)xb;
    w.w[0] = job.w[0] + row_bytes_of(qtype, k0);
    int rc;
    if (MODE == kPlain && first) {
      w.yb[0] = last ? job.yb[0] : nullptr;
      rc = stream_dispatch<kPlain>(qtype, d_last, w, xbf16, s);
    } else {
      w.bias = nullptr;
      w.resid = MODE == kResid ? job.resid : job.y[0];
      w.resid_bf16 = last ? (MODE == kResid ? job.resid_bf16 : job.yb[0]) : nullptr;
      rc = stream_dispatch<kResid>(qtype, d_last, w, xbf16, s);
    }
    if (rc) return rc;
  }
  return DRACO_OK;
}

}  // namespace draco
