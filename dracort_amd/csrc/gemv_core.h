// Register-level GEMV core shared by the decode GEMV and the MoE expert kernels.
//
// A wave64 owns R consecutive weight rows [n0, n0 + R) and walks their K axis
// in 32-weight units (lane l takes units l, l + 64, ...).  For each unit it
// loads the packed bytes of the R rows once, unpacks the codes in registers
// and accumulates, per group g of the unit,
//     acc[r][m] += a_g * sum_i(code_i * x_m[pos_i]) + b_g * sum_i(x_m[pos_i])
// so the block scale and min are applied once per group, not once per weight.
// The activations of a unit serve all R rows.  Accumulation is float32.
#pragma once

#include "gguf_common.h"

namespace draco {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// Load `GL` consecutive activations starting at element `p` of row `xr` as float.
template <int GL, bool XBF16>
__device__ __forceinline__ void load_x(const void* __restrict__ xr, int p, float* dst) {
  if constexpr (XBF16) {
    const uint4* s = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xr) + p);
#pragma unroll
    for (int j = 0; j < GL / 8; ++j) {
      const uint4 v = s[j];
      dst[8 * j + 0] = bf16_lo(v.x); dst[8 * j + 1] = bf16_hi(v.x);
      dst[8 * j + 2] = bf16_lo(v.y); dst[8 * j + 3] = bf16_hi(v.y);
      dst[8 * j + 4] = bf16_lo(v.z); dst[8 * j + 5] = bf16_hi(v.z);
      dst[8 * j + 6] = bf16_lo(v.w); dst[8 * j + 7] = bf16_hi(v.w);
    }
  } else {
    const float4* s = reinterpret_cast<const float4*>(static_cast<const float*>(xr) + p);
#pragma unroll
    for (int j = 0; j < GL / 4; ++j) {
      const float4 v = s[j];
      dst[4 * j + 0] = v.x; dst[4 * j + 1] = v.y; dst[4 * j + 2] = v.z; dst[4 * j + 3] = v.w;
    }
  }
}

// Per-group coefficients a[g], b[g] with w = a*code + b.
template <int QT>
__device__ __forceinline__ void unit_coeffs(const Raw<QT>& r, int u, float* a, float* b) {
  if constexpr (QT == kQ8_0) {
    a[0] = f16_bits_to_f32(r.d);
    b[0] = 0.f;
  } else if constexpr (QT == kQ4_0) {
    a[0] = f16_bits_to_f32(r.d);
    b[0] = -8.f * a[0];
  } else if constexpr (QT == kQ4_K) {
    const float d = f16_bits_to_f32(r.head.x), dmin = f16_bits_to_f32(r.head.x >> 16);
    const int j0 = 2 * ((u & 7) >> 1);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      uint32_t sc, mn;
      q4k_scale_min(r.head, j0 + g, sc, mn);
      a[g] = d * (float)sc;
      b[g] = -(dmin * (float)mn);
    }
  } else {
    const float d = f16_bits_to_f32(r.d);
    const int l16 = ((u & 7) & 3) >> 1;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = l16 + 2 * t;
      const uint32_t scw = j < 4 ? r.sc[0] : r.sc[1];
      a[t] = d * sbyte_f(scw, j & 3);
      b[t] = -32.f * a[t];
    }
  }
}

// Code of element i (0..GL-1) of group g as float.
template <int QT>
__device__ __forceinline__ float unit_code(const Raw<QT>& r, int g, int i) {
  if constexpr (QT == kQ8_0) {
    return sbyte_f(r.q[i >> 2], i & 3);
  } else if constexpr (QT == kQ4_0) {
    return i < 16 ? ubyte_f(nib_lo(r.q[i >> 2]), i & 3) : ubyte_f(nib_hi(r.q[(i - 16) >> 2]), i & 3);
  } else if constexpr (QT == kQ4_K) {
    const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
    return ubyte_f(g == 0 ? nib_lo(q[i >> 2]) : nib_hi(q[i >> 2]), i & 3);
  } else {
    const int h = i >> 2;
    return ubyte_f(q6_codes(g, r.qla[h], r.qlb[h], r.qh[h]), i & 3);
  }
}


// acc[r][mi] (lane partial sums) for rows n0 .. n0+R-1 and activation rows
// 0 .. m-1 (m <= MT); xrow(mi) returns the address of activation row mi.
// Rows past n are clamped to n - 1: they are computed but must not be stored.
template <int QT, bool DL, int MT, bool XBF16, int R, class XRow>
__device__ __forceinline__ void gemv_accumulate(const uint8_t* __restrict__ w, int64_t row_bytes, int n0, int n,
                                                int k, int m, XRow xrow, float (&acc)[R][MT]) {
  using F = Fmt<QT>;
  constexpr int G = F::G, GL = F::GL;
  const int lane = threadIdx.x & 63;
  const int units = k >> 5;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[r][mi] = 0.f;

  for (int u = lane; u < units; u += 64) {
    Raw<QT> raw[R];
    float a[R][G], b[R][G];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = n0 + r < n ? n0 + r : n - 1;
      raw[r] = load_unit<QT, DL>(w, (int64_t)row * row_bytes, u);
      unit_coeffs<QT>(raw[r], u, a[r], b[r]);
    }
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      if (mi < m) {
        const void* xr = xrow(mi);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float xv[GL];
          load_x<GL, XBF16>(xr, group_pos<QT>(u, g), xv);
          float xsum = 0.f;
          if constexpr (QT != kQ8_0) {
#pragma unroll
            for (int i = 0; i < GL; ++i) xsum += xv[i];
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < GL; ++i) dot = fmaf(unit_code<QT>(raw[r], g, i), xv[i], dot);
            acc[r][mi] = fmaf(a[r][g], dot, acc[r][mi]);
            if constexpr (QT != kQ8_0) acc[r][mi] = fmaf(b[r][g], xsum, acc[r][mi]);
          }
        }
      }
    }
  }
}

}  // namespace draco
