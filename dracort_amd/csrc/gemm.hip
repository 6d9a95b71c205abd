// Prefill GEMM with fused GGUF dequantization, bf16 MFMA on gfx950.
//
//   y[m, n] = sum_k x_bf16[m, k] * W[n, k]  (+ bias[n]),  float32 out
//
// Replaces _dequantize + x.astype(f32) @ W.T (draco/format/gguf.py:272-497,
// draco/runtime/cpu/kernels/generic.py:32-33) for prompt-sized M.
//
// Tiling: a 256-thread workgroup owns a 128 (tokens) x 128 (weight rows) output
// tile; its four waves each own 64 x 64 = 4 x 4 tiles of
// v_mfma_f32_16x16x32_bf16.  Per K step of 64 weights the workgroup
//   * copies the x tile into LDS (bf16, 16-byte loads), and
//   * decodes the packed weight tile: each thread unpacks 32-weight units in
//     registers (same decoders as the GEMV; a Q6_K unit spans 128 positions,
//     so a step writes the two of its four groups that fall in the window),
//     forms w = a*code + b in float32 and stores it to LDS as three bf16
//     planes w = hi + mid + lo (each the round-to-nearest bf16 of what the
//     previous ones leave), which represent the float32 weight to ~2^-27.
// Each output tile then takes three MFMAs per 32-wide K slice; a two-term
// split (~2^-18) is not enough for the 1e-3 elementwise bound on outputs near
// zero at K = 4096 with outlier rows.  The activations are bf16 and exact.
// The next K step's global loads are issued before the MFMAs of the current
// one so that HBM latency overlaps the matrix work.
//
// Q4_K with a workspace takes the exact f16 kernels instead: gemm_q4k2.h
// (256 x 128 tiles of 32 x 32 x 16 MFMAs, split along K when there are too
// few tiles and the workspace has room for the partial sums) when its grid
// fills at least three quarters of the CUs, gemm_q4k.h (64 x 128 tiles)
// otherwise.
#include "draco_internal.h"
#include "gemm_q4k.h"
#include "gemm_q4k2.h"
#include "gemv_core.h"

namespace draco {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128;

constexpr int kBK = 64;
constexpr int kLDK = kBK + 8;  // padded LDS row (bf16 elements): 16-byte aligned, conflict-free

template <int QT> struct GemmCfg {
  static constexpr int UR = (Fmt<QT>::FAM == kFamK6) ? 4 : 2;  // 32-weight units touched per row per K step
  static constexpr int UPT = kBN * UR / 256;        // units per thread
  static constexpr int APT = kBM * kBK / 8 / 256;   // 16-byte x pieces per thread
};

// Unit index of the ur-th unit touched by the K window starting at k0.
template <int QT>
__device__ __forceinline__ int window_unit(int k0, int ur) {
  if constexpr (Fmt<QT>::FAM == kFamK6) return 8 * (k0 >> 8) + 4 * ((k0 >> 7) & 1) + ur;
  return (k0 >> 5) + ur;
}

// Whether group g of a unit lies in the 64-wide window starting at k0.
template <int QT>
__device__ __forceinline__ bool group_in_window(int k0, int g) {
  if constexpr (Fmt<QT>::FAM == kFamK6) return (g >> 1) == ((k0 >> 6) & 1);
  return true;
}

__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

template <int QT, bool DL>
__global__ __launch_bounds__(256) void gemm_kernel(const uint8_t* __restrict__ w, const uint16_t* __restrict__ x,
                                                   const float* __restrict__ bias, float* __restrict__ y, int M,
                                                   int N, int K, int64_t row_bytes, int tiles_m) {
  using C = GemmCfg<QT>;
  constexpr int BK = kBK, LDK = kLDK, UR = C::UR, UPT = C::UPT, APT = C::APT;
  constexpr int G = Fmt<QT>::G, GL = Fmt<QT>::GL;
  __shared__ __attribute__((aligned(16))) uint16_t As[kBM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bh[kBN * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bm[kBN * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bl[kBN * LDK];

  const int tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int units_k = K >> 5;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint4 areg[APT];
  Raw<QT> breg[UPT];

  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int p = tid + 256 * i;
      const int row = p / (BK / 8), col = (p % (BK / 8)) * 8;
      const int gm = m0 + row, gk = k0 + col;
      areg[i] = (gm < M && gk < K) ? *reinterpret_cast<const uint4*>(x + (size_t)gm * K + gk) : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int t = tid + 256 * i;
      const int row = t / UR, ur = t % UR;
      const int gn = min(n0 + row, N - 1);
      const int u = min(window_unit<QT>(k0, ur), units_k - 1);
      breg[i] = load_unit<QT, DL>(w, (int64_t)gn * row_bytes, u);
    }
  };

  auto store_lds = [&](int k0) {
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int p = tid + 256 * i;
      const int row = p / (BK / 8), col = (p % (BK / 8)) * 8;
      *reinterpret_cast<uint4*>(&As[row * LDK + col]) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int t = tid + 256 * i;
      const int row = t / UR, ur = t % UR;
      const int u = window_unit<QT>(k0, ur);
      const bool live = (n0 + row < N) && (u < units_k);
      float a[G], b[G];
      unit_coeffs<QT>(breg[i], u, a, b);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (!group_in_window<QT>(k0, g)) continue;
        const int pos = group_pos<QT>(u, g) - k0;
#pragma unroll
        for (int e8 = 0; e8 < GL; e8 += 8) {
          uint32_t hp[4], mp[4], lp[4];
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            uint32_t h[2], md[2], l[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              const float wv = live ? fmaf(a[g], unit_code<QT>(breg[i], g, e8 + e + t, u), b[g]) : 0.f;
              h[t] = bf16_rne_bits(wv);
              const float r1 = wv - __uint_as_float(h[t] << 16);
              md[t] = bf16_rne_bits(r1);
              l[t] = bf16_rne_bits(r1 - __uint_as_float(md[t] << 16));
            }
            hp[e / 2] = h[0] | (h[1] << 16);
            mp[e / 2] = md[0] | (md[1] << 16);
            lp[e / 2] = l[0] | (l[1] << 16);
          }
          *reinterpret_cast<uint4*>(&Bh[row * LDK + pos + e8]) = uint4{hp[0], hp[1], hp[2], hp[3]};
          *reinterpret_cast<uint4*>(&Bm[row * LDK + pos + e8]) = uint4{mp[0], mp[1], mp[2], mp[3]};
          *reinterpret_cast<uint4*>(&Bl[row * LDK + pos + e8]) = uint4{lp[0], lp[1], lp[2], lp[3]};
        }
      }
    }
  };

  load_global(0);
  for (int k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();
    store_lds(k0);
    __syncthreads();
    if (k0 + BK < K) load_global(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      bf16x8 af[4], bh[4], bm[4], bl[4];
      const int kc = kk + 8 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&As[(wm * 64 + 16 * i + (lane & 15)) * LDK + kc]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int bo = (wn * 64 + 16 * j + (lane & 15)) * LDK + kc;
        bh[j] = *reinterpret_cast<const bf16x8*>(&Bh[bo]);
        bm[j] = *reinterpret_cast<const bf16x8*>(&Bm[bo]);
        bl[j] = *reinterpret_cast<const bf16x8*>(&Bl[bo]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bl[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bm[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bh[j], acc[i][j], 0, 0, 0);
        }
    }
  }

  // D layout of v_mfma_f32_16x16x32: lane l holds rows 4*(l/16) + v, column l % 16.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + 16 * j + (lane & 15);
    if (n >= N) continue;
    const float bv = bias ? bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm * 64 + 16 * i + 4 * (lane >> 4) + v;
        if (m < M) y[(size_t)m * N + n] = acc[i][j][v] + bv;
      }
  }
}

template <int QT, bool DL>
static int launch_gemm(const void* w, const void* x, const float* bias, float* y, int m, int n, int k,
                       hipStream_t s) {
  const int64_t row_bytes = (int64_t)(k / Fmt<QT>::QK) * Fmt<QT>::BYTES;
  const int tiles_m = (m + kBM - 1) / kBM, tiles_n = (n + kBN - 1) / kBN;
  const int64_t blocks = (int64_t)tiles_m * tiles_n;
  if (blocks > 0x7FFFFFFF) return set_error(DRACO_EINVAL_SHAPE, "GEMM grid too large");
  hipLaunchKernelGGL((gemm_kernel<QT, DL>), dim3((unsigned)blocks), dim3(256), 0, s,
                     static_cast<const uint8_t*>(w), static_cast<const uint16_t*>(x), bias, y, m, n, k, row_bytes,
                     tiles_m);
  return check_launch("gemm");
}

size_t gemm_workspace_min(int qtype, int64_t m, int64_t k) {
  return qtype == kQ4_K ? gemm_q4k_ws_layout(m, k, nullptr, nullptr) : 0;
}

size_t gemm_workspace_size(int qtype, int64_t m, int64_t k) {
  return qtype == kQ4_K ? gemm_q4k_ws_layout(m, k, nullptr, nullptr) + gemm_q4k2_part_bound(m) : 0;
}

int gemm_dispatch(int qtype, bool d_last, const void* w, const void* x, const float* bias, float* y, int m, int n,
                  int k, void* workspace, size_t workspace_bytes, hipStream_t s) {
  if (qtype == kQ4_K && workspace) {
    if ((int64_t)n * (k / 256) * 144 >= ((int64_t)1 << 31))
      return set_error(DRACO_EINVAL_SHAPE, "Q4_K GEMM weight above 2 GiB");
    const size_t base = gemm_q4k_ws_layout(m, k, nullptr, nullptr);
    const GemmQ4k2Plan plan = gemm_q4k2_plan(m, n, k, workspace_bytes > base ? workspace_bytes - base : 0);
    return plan.splits ? launch_gemm_q4k2(w, x, bias, y, m, n, k, workspace, plan, s)
                       : launch_gemm_q4k(w, x, bias, y, m, n, k, workspace, s);
  }
  switch (qtype) {
    case kQ8_0: return launch_gemm<kQ8_0, false>(w, x, bias, y, m, n, k, s);
    case kQ4_0: return launch_gemm<kQ4_0, false>(w, x, bias, y, m, n, k, s);
    case kQ4_1: return launch_gemm<kQ4_1, false>(w, x, bias, y, m, n, k, s);
    case kQ5_0: return launch_gemm<kQ5_0, false>(w, x, bias, y, m, n, k, s);
    case kQ5_1: return launch_gemm<kQ5_1, false>(w, x, bias, y, m, n, k, s);
    case kQ8_K: return launch_gemm<kQ8_K, false>(w, x, bias, y, m, n, k, s);
    case kQ4_K: return launch_gemm<kQ4_K, false>(w, x, bias, y, m, n, k, s);
    case kQ5_K: return launch_gemm<kQ5_K, false>(w, x, bias, y, m, n, k, s);
    case kQ2_K:
      return d_last ? launch_gemm<kQ2_K, true>(w, x, bias, y, m, n, k, s)
                    : launch_gemm<kQ2_K, false>(w, x, bias, y, m, n, k, s);
    case kQ3_K:
      return d_last ? launch_gemm<kQ3_K, true>(w, x, bias, y, m, n, k, s)
                    : launch_gemm<kQ3_K, false>(w, x, bias, y, m, n, k, s);
    case kQ6_K:
      return d_last ? launch_gemm<kQ6_K, true>(w, x, bias, y, m, n, k, s)
                    : launch_gemm<kQ6_K, false>(w, x, bias, y, m, n, k, s);
    default: return set_error(DRACO_EINVAL_QTYPE, "unsupported ggml type %d", qtype);
  }
}

}  // namespace draco
