// Single-token decode GEMV (M = 1) for the 32-weight block formats Q8_0 and
// Q4_0, float32 or bfloat16 activations, K <= 4096.
//
//   y[n] = sum_k x[k] W[n, k],  w = d q (Q8_0: int8 q; Q4_0: q = nibble - 8)
//
// Lane l of a wave owns elements 64 l .. 64 l + 63 of every row (two blocks:
// 68 bytes of Q8_0, 36 of Q4_0), so its activations are the same for every
// row the wave computes: they are loaded once into 64 float registers, with
// the two block sums.  A wave walks rows gw, gw + waves, ..., requesting
// the next row's two blocks (dwordx4 loads at dword-aligned offsets; Q8_0's
// first block and both of Q4_0's sit two bytes off a dword and are realigned
// with v_alignbyte) before multiplying the current one.  Measured on MI355X:
// Q8_0 4096 x 4096 at f32 x 7.0 us (12.6 on the streaming kernel), four rows
// per wave; sharing the activations through LDS per workgroup, or four rows
// requested at a time, was slower.  Codes are biased to
// non-negative integers (Q8_0: byte ^ 0x80 = q + 128; Q4_0: the nibble =
// q + 8), converted by v_cvt_f32_ubyte and accumulated against x in float32;
// each block contributes d (dot - bias S) with S the block's activation sum.
// The row's 64 lane sums meet through DPP (wave_sum_dpp) and lane 0 stores.
// Replaces _dequantize + x @ W.T for these types at one token
// (draco/format/gguf.py:272-497, draco/runtime/cpu/kernels/generic.py:32-33).
#pragma once

#include <climits>

#include "gemv_stream.h"

namespace draco {

template <int QT> struct X1bFmt;
template <> struct X1bFmt<kQ8_0> { static constexpr int DW = 17; static constexpr float BIAS = 128.f; };  // 68 bytes
template <> struct X1bFmt<kQ4_0> { static constexpr int DW = 9; static constexpr float BIAS = 8.f; };    // 36 bytes

typedef int x1b_v4i __attribute__((ext_vector_type(4)));

// The lane's two blocks of one row (DW dwords from byte offset off).
template <int QT>
__device__ __forceinline__ void x1b_load(__amdgpu_buffer_rsrc_t rs, int off, uint32_t (&w)[X1bFmt<QT>::DW]) {
  constexpr int DW = X1bFmt<QT>::DW;
#pragma unroll
  for (int i = 0; i + 4 <= DW; i += 4) {
    const x1b_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4 * i, 0, 0);
    w[i] = (uint32_t)v.x;
    w[i + 1] = (uint32_t)v.y;
    w[i + 2] = (uint32_t)v.z;
    w[i + 3] = (uint32_t)v.w;
  }
  w[DW - 1] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, off + 4 * (DW - 1), 0, 0);
}

// sum_j x[j] c[j] over the four bytes c of one dword (x: four floats)
__device__ __forceinline__ float x1b_dot4(uint32_t c, const float* x, float acc) {
  acc = fmaf(x[0], ubyte_f(c, 0), acc);
  acc = fmaf(x[1], ubyte_f(c, 1), acc);
  acc = fmaf(x[2], ubyte_f(c, 2), acc);
  acc = fmaf(x[3], ubyte_f(c, 3), acc);
  return acc;
}

// The lane's share of one row: d0 (dot0 - bias S0) + d1 (dot1 - bias S1).
template <int QT>
__device__ __forceinline__ float x1b_row(const uint32_t (&w)[X1bFmt<QT>::DW], const float (&x)[64], float s0,
                                         float s1) {
  constexpr float BIAS = X1bFmt<QT>::BIAS;
  float dot0 = 0.f, dot1 = 0.f;
  float d0, d1;
  if constexpr (QT == kQ8_0) {
    // bytes 0-1 d0, 2-33 block 0's codes, 34-35 d1, 36-67 block 1's codes
    d0 = f16_bits_to_f32(w[0]);
    d1 = f16_bits_to_f32(w[8] >> 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t c0 = __builtin_amdgcn_alignbyte(w[j + 1], w[j], 2) ^ 0x80808080u;  // codes 4j .. 4j + 3
      dot0 = x1b_dot4(c0, &x[4 * j], dot0);
      dot1 = x1b_dot4(w[9 + j] ^ 0x80808080u, &x[32 + 4 * j], dot1);
    }
  } else {
    // bytes 0-1 d0, 2-17 block 0's 16 code bytes, 18-19 d1, 20-35 block 1's;
    // byte i holds element i (low nibble) and element i + 16 (high nibble)
    d0 = f16_bits_to_f32(w[0]);
    d1 = f16_bits_to_f32(w[4] >> 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t q0 = __builtin_amdgcn_alignbyte(w[j + 1], w[j], 2);
      const uint32_t q1 = w[5 + j];
      dot0 = x1b_dot4(q0 & 0x0F0F0F0Fu, &x[4 * j], dot0);
      dot0 = x1b_dot4((q0 >> 4) & 0x0F0F0F0Fu, &x[16 + 4 * j], dot0);
      dot1 = x1b_dot4(q1 & 0x0F0F0F0Fu, &x[32 + 4 * j], dot1);
      dot1 = x1b_dot4((q1 >> 4) & 0x0F0F0F0Fu, &x[48 + 4 * j], dot1);
    }
  }
  // the bias cancels here, once per block, before the block scale
  return fmaf(d0, fmaf(-BIAS, s0, dot0), d1 * fmaf(-BIAS, s1, dot1));
}

template <int QT, bool XBF16, int MODE>
__global__ __launch_bounds__(256) void gemv_x1b_kernel(StreamJob job) {
  static_assert(MODE == kPlain || MODE == kResid, "plain and residual launches only");
  constexpr int DW = X1bFmt<QT>::DW;
  const int lane = threadIdx.x & 63;
  const int gw = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int nw = (int)gridDim.x * 4;
  const int k = job.k, units = k >> 6;
  const bool live = lane < units;

  // the lane's 64 activations (zeros past K)
  float x[64];
  {
    const int u = live ? lane : 0;
    if constexpr (XBF16) {
      const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(job.x) + 64 * u);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint4 v = p[c];
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[8 * c + 2 * i] = live ? __uint_as_float(vw[i] << 16) : 0.f;
          x[8 * c + 2 * i + 1] = live ? __uint_as_float(vw[i] & 0xFFFF0000u) : 0.f;
        }
      }
    } else {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(job.x) + 64 * u);
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float4 v = p[c];
        x[4 * c] = live ? v.x : 0.f;
        x[4 * c + 1] = live ? v.y : 0.f;
        x[4 * c + 2] = live ? v.z : 0.f;
        x[4 * c + 3] = live ? v.w : 0.f;
      }
    }
  }

  // matrices of the launch (kPlain: rows of up to four matrices back to back),
  // picked by chains of selects (an index into the argument would be a table
  // in scratch)
  const uint8_t *w0 = job.w[0], *w1 = job.w[1], *w2 = job.w[2], *w3 = job.w[3];
  const int n0 = job.n[0], n1 = job.n[1], n2 = job.n[2], n3 = job.n[3];
  float *y0 = job.y[0], *y1 = job.y[1], *y2 = job.y[2], *y3 = job.y[3];
  uint16_t *b0 = job.yb[0], *b1 = job.yb[1], *b2 = job.yb[2], *b3 = job.yb[3];
  const int row_bytes = (int)job.row_bytes;
  int c1 = INT_MAX, c2 = INT_MAX, c3 = INT_MAX;
  if constexpr (MODE == kPlain) {
    if (job.n_mats > 1) c1 = n0;
    if (job.n_mats > 2) c2 = c1 + n1;
    if (job.n_mats > 3) c3 = c2 + n2;
  }
  auto pick = [](int mat, auto v0, auto v1, auto v2, auto v3) {
    auto v = v0;
    v = mat >= 1 ? v1 : v;
    v = mat >= 2 ? v2 : v;
    v = mat >= 3 ? v3 : v;
    return v;
  };
  auto locate = [&](int row, int& mat, int& lrow) {
    mat = (row >= c1) + (row >= c2) + (row >= c3);
    int base = row >= c1 ? c1 : 0;
    base = row >= c2 ? c2 : base;
    base = row >= c3 ? c3 : base;
    lrow = row - base;
  };
  const int rows = job.rows;
  // a row's blocks: an empty resource past the wave's last row and an offset
  // past any buffer for lanes beyond K (every wait count stays exact, the
  // resource stays wave-uniform)
  auto fetch = [&](int row, uint32_t (&w)[DW]) {
    int mat, lrow;
    locate(min(row, rows - 1), mat, lrow);
    const uint8_t* wp = pick(mat, w0, w1, w2, w3);
    const int nn = pick(mat, n0, n1, n2, n3);
    const __amdgpu_buffer_rsrc_t rs =
        row < rows ? make_rsrc(wp, (uint32_t)((int64_t)nn * row_bytes)) : make_rsrc(nullptr, 0u);
    x1b_load<QT>(rs, live ? lrow * row_bytes + lane * 4 * DW : (int)0x80000000, w);
  };
  uint32_t wb[2][DW];
  int row = gw;
  fetch(row, wb[0]);
  // the block sums (the first row already requested)
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    s0 += x[i];
    s1 += x[32 + i];
  }
  for (; row < rows; row += 2 * nw) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int r = row + p * nw;
      fetch(r + nw, wb[p ^ 1]);
      if (r < rows) {
        const float part = live ? x1b_row<QT>(wb[p], x, s0, s1) : 0.f;
        const float tot = wave_sum_dpp(part);
        if (lane == 0) {
          int mat, lrow;
          locate(r, mat, lrow);
          if constexpr (MODE == kResid) {
            const float out = job.resid[lrow] + tot;
            job.resid[lrow] = out;
            if (job.resid_bf16) job.resid_bf16[lrow] = f32_to_bf16_rne(out);
          } else {
            float* const yp = pick(mat, y0, y1, y2, y3);
            uint16_t* const ybp = pick(mat, b0, b1, b2, b3);
            const float out = tot + (job.bias ? job.bias[lrow] : 0.f);
            if (yp) yp[lrow] = out;
            if (ybp) ybp[lrow] = f32_to_bf16_rne(out);
          }
        }
      }
    }
  }
}

// Whether the single-token block-format kernel takes this launch.
inline bool x1b_ok(int qtype, const StreamJob& job) {
  if ((qtype != kQ8_0 && qtype != kQ4_0) || job.m != 1 || job.k % 64 != 0 || job.k > 4096) return false;
  for (int i = 0; i < job.n_mats; ++i)
    if ((int64_t)job.n[i] * job.row_bytes >= ((int64_t)1 << 31)) return false;
  return true;
}

template <int QT, bool XBF16, int MODE>
static int launch_x1b(const StreamJob& job, int blocks_per_cu, hipStream_t s) {
  // about a thousand waves, up to four rows each, at most blocks_per_cu
  // workgroups per CU (measured on MI355X: Q8_0 4096 x 4096 7.0 us at 1024
  // waves of four rows, 8.1 us at two rows per wave; Q4_0 1024 x 4096 4.8 us
  // at 512 waves, 6.4 at 256; Q4_0 14336 x 4096 13.2 us at three workgroups
  // per CU, 14.1 at four)
  const int waves = std::min(job.rows, std::max(1024, (job.rows + 3) / 4));
  const int blocks = std::max(1, std::min((waves + 3) / 4, device_cus() * blocks_per_cu));
  hipLaunchKernelGGL((gemv_x1b_kernel<QT, XBF16, MODE>), dim3(blocks), dim3(256), 0, s, job);
  return check_launch("gemv_x1b");
}

template <int MODE>
static int x1b_dispatch(int qtype, const StreamJob& job, bool xbf16, hipStream_t s) {
  constexpr int bpc = 3;
  if (qtype == kQ8_0)
    return xbf16 ? launch_x1b<kQ8_0, true, MODE>(job, bpc, s) : launch_x1b<kQ8_0, false, MODE>(job, bpc, s);
  return xbf16 ? launch_x1b<kQ4_0, true, MODE>(job, bpc, s) : launch_x1b<kQ4_0, false, MODE>(job, bpc, s);
}

}  // namespace draco
