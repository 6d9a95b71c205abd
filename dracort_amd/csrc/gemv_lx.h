// Single-token decode GEMV (M = 1, bfloat16 activations) for Q4_K / Q6_K rows
// of one 4096-weight step (K <= 4096), with row-contiguous weight loads.
//
// The persistent x1p kernel has each lane fetch the fields of its own
// 64-weight unit, so a wave's load instruction covers scattered 16-byte
// pieces of ~2.3 KB and the block heads are fetched four times.  Here a
// wave reads a row as consecutive 1 KB pieces instead (lane l loads bytes
// 1024 c + 16 l .. + 15 of the row, one 16-byte buffer load per lane per
// piece, every byte once; lanes past the row's last byte use an offset past
// the buffer end, which returns zeros without a memory request), parks the
// row in a wave-private LDS slot and then reads its unit's fields from LDS
// (three ds_read_b128 for Q4_K; five-dword reads realigned by two bytes for
// Q6_K's 210-byte blocks).  The unit math, the activation image, the row
// schedule (wave w computes rows w, w + W, ...) and the issue order (row
// i + PF requested before row i is multiplied, results stashed and stored
// every 64 rows) are the x1p kernel's.
#pragma once

#include "gemv_x1.h"

namespace draco {

template <int QT> struct LxGeom {
  static constexpr int ROW_BYTES = 16 * Fmt<QT>::BYTES;   // one 4096-weight step
  static constexpr int LPR = (ROW_BYTES + 1023) / 1024;    // 1 KB pieces per row: Q4_K 3, Q6_K 4
  static constexpr int SLOT = LPR * 1024;                  // bytes of a wave's LDS slot per matrix
};

// 16 bytes at an even LDS byte offset: five dwords from the 4-aligned
// address at or below it, realigned.  The slot is padded so the fifth dword
// stays inside it.
__device__ __forceinline__ uint4 lds_u128_even(const uint32_t* __restrict__ s, int off) {
  const int d = off >> 2;
  const uint32_t sh = (uint32_t)off & 3u;
  const uint32_t a = s[d], b = s[d + 1], c = s[d + 2], e = s[d + 3], f = s[d + 4];
  return uint4{__builtin_amdgcn_alignbyte(b, a, sh), __builtin_amdgcn_alignbyte(c, b, sh),
               __builtin_amdgcn_alignbyte(e, c, sh), __builtin_amdgcn_alignbyte(f, e, sh)};
}

// Unit u (64 weights) of a row parked at LDS slot s (byte offsets as in x1_load).
template <int QT, bool DL>
__device__ __forceinline__ X1Raw<QT> lx_unit(const uint32_t* __restrict__ s, int u) {
  X1Raw<QT> r;
  const int blk = (u >> 2) * Fmt<QT>::BYTES, j = u & 3;
  if constexpr (QT == kQ4_K) {
    const uint4* s4 = reinterpret_cast<const uint4*>(s);
    r.head = s4[blk >> 4];
    r.qs0 = s4[(blk + 16 + 32 * j) >> 4];
    r.qs1 = s4[(blk + 32 + 32 * j) >> 4];
  } else {
    constexpr int QL = DL ? 0 : 2, QH = DL ? 128 : 130, SC = DL ? 192 : 194, D = DL ? 208 : 0;
    const int n = j >> 1, h = j & 1;
    r.qla = lds_u128_even(s, blk + QL + 64 * n + 16 * h);
    r.qlb = lds_u128_even(s, blk + QL + 64 * n + 32 + 16 * h);
    r.qh = lds_u128_even(s, blk + QH + 32 * n + 16 * h);
    const int so = blk + SC + 8 * n, sd = so >> 2;
    const uint32_t ssh = (uint32_t)so & 3u;
    const uint32_t a = s[sd], b = s[sd + 1], c = s[sd + 2];
    r.sc0 = __builtin_amdgcn_alignbyte(b, a, ssh);
    r.sc1 = __builtin_amdgcn_alignbyte(c, b, ssh);
    const int dd = blk + D;
    r.d = (s[dd >> 2] >> (8 * (dd & 3))) & 0xFFFFu;
  }
  return r;
}

// The row's 1 KB pieces for matrix q (kSwiGLU: gate, up) of the wave's row i:
// lane l loads bytes 1024 c + 16 l .. + 15; lanes past the row's last byte
// use an offset past any buffer (zeros, no memory request).
template <int MODE, int NR, int LPR>
__device__ __forceinline__ void lx_load_row(const X1Rows<MODE>& rows, const StreamJob& job, int i, int row_bytes,
                                            uint4 (&dst)[NR][LPR]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int q = 0; q < NR; ++q) {
    const X1Buf b = rows.buf(job, i, q);
#pragma unroll
    for (int c = 0; c < LPR; ++c) {
      const int o = 1024 * c + 16 * lane;
      dst[q][c] = b.b128(o < row_bytes ? o : 0x7FFFFFF0);
    }
  }
}

template <int QT, int MODE>
__host__ __device__ inline size_t lx_lds_bytes(int k) {
  constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  // activation image + sums + pad, then four waves' slots (+16 B so the
  // realigning reads of the last field stay inside)
  return x1p_lds_bytes(QT, k) + 4 * ((size_t)NR * LxGeom<QT>::SLOT + 16);
}

template <int QT, bool DL, int MODE, int PF>
__global__ __launch_bounds__(256) void gemv_lx_kernel(StreamJob job) {
  constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  constexpr int NB = PF + 1;
  constexpr int LPR = LxGeom<QT>::LPR;
  constexpr int SLOTW = (NR * LxGeom<QT>::SLOT + 16) / 4;  // dwords per wave slot
  extern __shared__ uint4 lx_smem[];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const X1Rows<MODE> rows(job);
  const int nrow = rows.nrow;
  const int k = job.k;
  const int units = k >> 6;
  const bool live = lane < units;
  const int row_bytes = (int)job.row_bytes;  // <= ROW_BYTES

  // 1. activations (two 16-byte chunks per thread), then the first rows
  uint4 xr[2];
  x1_fetch_x<2>(job.x, k, xr);
  uint4 buf[NB][NR][LPR];
#pragma unroll
  for (int p = 0; p < PF; ++p) lx_load_row<MODE, NR, LPR>(rows, job, p, row_bytes, buf[p]);

  // 2. the LDS image and group sums; the lane's activations into registers
  x1_stage_regs<QT, 2>(lx_smem, xr, k);
  if (nrow == 0) return;
  const X1Lane lc = x1_lane<QT>(lane);
  X1Act xa;
  x1_read_lds<QT>(lx_smem, k, 0, lane, live, xa);
  uint32_t* slot = reinterpret_cast<uint32_t*>(lx_smem + x1p_lds_bytes(QT, k) / 16) + wid * SLOTW;
  const int ul = live ? lane : units - 1;

  // 3. rows
  float res = 0.f;
  for (int i0 = 0; i0 < nrow; i0 += NB) {
#pragma unroll
    for (int p = 0; p < NB; ++p) {
      const int i = i0 + p;
      lx_load_row<MODE, NR, LPR>(rows, job, i + PF, row_bytes, buf[(p + PF) % NB]);
      __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the math
      if (i < nrow) {
#pragma unroll
        for (int q = 0; q < NR; ++q)
#pragma unroll
          for (int c = 0; c < LPR; ++c)
            reinterpret_cast<uint4*>(slot + q * (LxGeom<QT>::SLOT / 4))[c * 64 + lane] = buf[p][q][c];
        float v[NR];
#pragma unroll
        for (int q = 0; q < NR; ++q) {
          const X1Raw<QT> raw = lx_unit<QT, DL>(slot + q * (LxGeom<QT>::SLOT / 4), ul);
          v[q] = wave_sum_dpp(x1_unit_dot<QT>(raw, lc, xa));
        }
        float out = v[0];
        if constexpr (MODE == kSwiGLU) out = silu(v[0]) * v[1];
        res = (lane == (i & 63)) ? out : res;
        if ((i & 63) == 63) rows.flush(job, i - 63, 64, res);
      }
    }
  }
  if (nrow & 63) rows.flush(job, nrow & ~63, nrow & 63, res);
}

template <int QT, bool DL, int MODE, int PF>
static int launch_lx(const StreamJob& job, int blocks_per_cu, hipStream_t s) {
  if (job.k > 4096 || job.k % 256 != 0 || job.row_bytes > LxGeom<QT>::ROW_BYTES)
    return set_error(DRACO_EINVAL_SHAPE, "row-streaming GEMV takes K <= 4096");
  const size_t lds = lx_lds_bytes<QT, MODE>(job.k);
  const int need = (job.rows + 3) / 4;
  const int blocks = std::max(1, std::min(need, device_cus() * blocks_per_cu));
  hipLaunchKernelGGL((gemv_lx_kernel<QT, DL, MODE, PF>), dim3(blocks), dim3(256), lds, s, job);
  return check_launch("gemv_lx");
}

}  // namespace draco
