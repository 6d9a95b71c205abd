// Decode GEMV with float32 activations and 1..8 activation rows, Q4_0 / Q8_0
// weights, on the float32 matrix cores (v_mfma_f32_4x4x1_16b_f32).
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  m < M <= 8
//
// One v_mfma_f32_4x4x1_16b_f32 is sixteen independent 4 x 4 outer products
// (A: 4 activation rows at one k, B: 4 weight rows at one k), so with M <= 4
// it is exactly the GEMV's work for 64 weights: no padding rows, and float32
// activations go in as they are (no bf16 planes, no conversion).  B carries
// the codes as small integers (exact in float32); the block scale d is
// applied once per 32-weight block on the VALU:
//   sum_k x (code - off) d = d (D - off S),  D = sum_k x code, S = sum_k x,
// with the -off S term added by two more MFMA steps (A = -off * the lane's
// partial sum of x, B = 1).  M 5..8 takes a second MFMA per step on
// activation rows 4..7.
//
// Lane roles (l = 16 s + 4 g + j):
//   * B / D: MFMA block 4 s + g, column j = weight row 4 g + j of a 16-row
//     tile; the lane holds that row's blocks 2 s, 2 s + 1 of a 256-element
//     K range (one contiguous 2-block load) and their 64 codes.
//   * A: the four blocks 4 s .. 4 s + 3 take their A operand from one of
//     them (CBSZ = 2, ABID = a), so lane (s, a, i) holds activation row i at
//     elements 64 s + 16 a .. + 16 of the range, one per register: step v of
//     the 64 multiplies element 16 a + v (ABID a, register v).  Every
//     activation value is held by exactly one lane.
// Elements 0..31 of a lane's pair (ABID 0, 1) are block 2 s, 32..63 (ABID
// 2, 3) block 2 s + 1: two accumulators, each scaled by its block's d.
//
// Grid: a workgroup owns T consecutive tiles and all of K; its waves split
// the K ranges (wave w of nw takes ranges w, w + nw, ...).  Per range a wave
// loads its activations once (the next range's while this one is used) and
// multiplies the T tiles, each tile's next-range weights requested as soon as
// its current ones are used (T items in flight, one accumulator per tile in
// registers).  At the end the tiles' sums (added over s) meet in LDS and the
// wave partials are added in wave order, so results do not depend on timing.
// Modes: kPlain (up to 4 matrices, each row count a multiple of 16 when
// there are several; bias with one) and kResid.
#pragma once

#include "gemv_stream.h"

namespace draco {

typedef float mf32_f32x4 __attribute__((ext_vector_type(4)));

// Dwords of one lane's two blocks, and the code offset taken out through S.
template <int QT> struct Mf32Fmt;
template <> struct Mf32Fmt<kQ4_0> { static constexpr int PD = 9;  static constexpr float OFF = 8.f; };
template <> struct Mf32Fmt<kQ8_0> { static constexpr int PD = 17; static constexpr float OFF = 128.f; };

constexpr int kMf32Oob = (int)0x80000000;  // buffer offset past any resource: loads return 0

template <int QT>
__device__ __forceinline__ void mf32_load_w(__amdgpu_buffer_rsrc_t rs, int off, uint32_t (&w)[Mf32Fmt<QT>::PD]) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  constexpr int PD = Mf32Fmt<QT>::PD;
#pragma unroll
  for (int i = 0; i < PD / 4; ++i) {
    const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * i, 0, 0);
    w[4 * i] = (uint32_t)v.x;
    w[4 * i + 1] = (uint32_t)v.y;
    w[4 * i + 2] = (uint32_t)v.z;
    w[4 * i + 3] = (uint32_t)v.w;
  }
  w[PD - 1] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, off + 16 * (PD / 4), 0, 0);
}

template <int MS>
__device__ __forceinline__ void mf32_load_x(__amdgpu_buffer_rsrc_t rs, const int (&off)[MS], float (&x)[MS][16]) {
  typedef float v4f __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int st = 0; st < MS; ++st)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v4f v = __builtin_amdgcn_raw_buffer_load_b128(rs, off[st] + 16 * i, 0, 0);
      x[st][4 * i] = v.x;
      x[st][4 * i + 1] = v.y;
      x[st][4 * i + 2] = v.z;
      x[st][4 * i + 3] = v.w;
    }
}

// w & c through an opaque instruction: the byte conversions below then stay
// single v_cvt_f32_ubyte{0..3} of the masked word (instead of being folded
// into a bit-field extract plus a conversion per code).
__device__ __forceinline__ uint32_t mf32_and(uint32_t w, uint32_t c) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(c), "v"(w));
  return r;
}
__device__ __forceinline__ uint32_t mf32_xor(uint32_t w, uint32_t c) {
  uint32_t r;
  asm("v_xor_b32 %0, %1, %2" : "=v"(r) : "s"(c), "v"(w));
  return r;
}

// The lane's codes as bytes: Q4_0 the low (lo) and high (hi) nibbles of every
// dword, Q8_0 every dword with the sign bits flipped (code + 128).
template <int QT> struct Mf32Codes {
  uint32_t lo[Mf32Fmt<QT>::PD], hi[QT == kQ4_0 ? Mf32Fmt<QT>::PD : 1];
};

template <int QT>
__device__ __forceinline__ Mf32Codes<QT> mf32_codes(const uint32_t (&w)[Mf32Fmt<QT>::PD]) {
  Mf32Codes<QT> c;
#pragma unroll
  for (int i = 0; i < Mf32Fmt<QT>::PD; ++i) {
    if constexpr (QT == kQ4_0) {
      c.lo[i] = mf32_and(w[i], 0x0F0F0F0Fu);
      c.hi[i] = mf32_and(w[i] >> 4, 0x0F0F0F0Fu);
    } else {
      c.lo[i] = mf32_xor(w[i], 0x80808080u);
    }
  }
  return c;
}

// Code of element 16 h + v of block b (0, 1) of the lane's pair, as float
// (b, h, v constants after unrolling).
template <int QT>
__device__ __forceinline__ float mf32_code(const Mf32Codes<QT>& c, int b, int h, int v) {
  if constexpr (QT == kQ4_0) {
    // block b: f16 d at byte 18 b, qs at 18 b + 2; element 16 h + v is nibble h of qs byte v
    const int pos = 18 * b + 2 + v;
    return ubyte_f(h ? c.hi[pos >> 2] : c.lo[pos >> 2], pos & 3);
  } else {
    // block b: f16 d at byte 34 b, int8 codes at 34 b + 2
    const int pos = 34 * b + 2 + 16 * h + v;
    return ubyte_f(c.lo[pos >> 2], pos & 3);
  }
}

template <int QT, int B>
__device__ __forceinline__ float mf32_d(const uint32_t (&w)[Mf32Fmt<QT>::PD]) {
  constexpr int pos = (QT == kQ4_0 ? 18 : 34) * B;
  return f16_bits_to_f32(pos & 2 ? w[pos >> 2] >> 16 : w[pos >> 2]);
}

// acc += the products of one item: the lane's two blocks (weights w, block
// scales zeroed past the row end) against the activations x; sn = -off *
// the lane's sum of its 16 activations per row set.
template <int QT, int MS>
__device__ __forceinline__ void mf32_item(const uint32_t (&w)[Mf32Fmt<QT>::PD], const float (&x)[MS][16],
                                          const float (&sn)[MS], bool live, mf32_f32x4 (&acc)[MS]) {
  const mf32_f32x4 z = {0.f, 0.f, 0.f, 0.f};
  const Mf32Codes<QT> c = mf32_codes<QT>(w);
  mf32_f32x4 da[MS], db[MS];
#pragma unroll
  for (int st = 0; st < MS; ++st) {
    da[st] = z;
    db[st] = z;
  }
  // ABID order 0, 2, 1, 3: the two accumulators alternate
#pragma clang loop unroll(full)
  for (int v = 0; v < 16; ++v) {
    const float c0 = mf32_code<QT>(c, 0, 0, v), c2 = mf32_code<QT>(c, 1, 0, v);
    const float c1 = mf32_code<QT>(c, 0, 1, v), c3 = mf32_code<QT>(c, 1, 1, v);
#pragma unroll
    for (int st = 0; st < MS; ++st) {
      da[st] = __builtin_amdgcn_mfma_f32_4x4x1f32(x[st][v], c0, da[st], 2, 0, 0);
      db[st] = __builtin_amdgcn_mfma_f32_4x4x1f32(x[st][v], c2, db[st], 2, 2, 0);
      da[st] = __builtin_amdgcn_mfma_f32_4x4x1f32(x[st][v], c1, da[st], 2, 1, 0);
      db[st] = __builtin_amdgcn_mfma_f32_4x4x1f32(x[st][v], c3, db[st], 2, 3, 0);
    }
  }
#pragma unroll
  for (int st = 0; st < MS; ++st) {
    da[st] = __builtin_amdgcn_mfma_f32_4x4x1f32(sn[st], 1.f, da[st], 2, 0, 0);
    db[st] = __builtin_amdgcn_mfma_f32_4x4x1f32(sn[st], 1.f, db[st], 2, 2, 0);
    da[st] = __builtin_amdgcn_mfma_f32_4x4x1f32(sn[st], 1.f, da[st], 2, 1, 0);
    db[st] = __builtin_amdgcn_mfma_f32_4x4x1f32(sn[st], 1.f, db[st], 2, 3, 0);
  }
  const float dA = live ? mf32_d<QT, 0>(w) : 0.f;
  const float dB = live ? mf32_d<QT, 1>(w) : 0.f;
#pragma unroll
  for (int st = 0; st < MS; ++st)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[st][i] = fmaf(dA, da[st][i], acc[st][i]);
      acc[st][i] = fmaf(dB, db[st][i], acc[st][i]);
    }
}

// Waves per workgroup (register budget: 16 waves leave 128 registers a lane,
// enough for Q4_0 with four activation rows and one or two tiles).
template <int QT, int MS, int T> struct Mf32Waves {
  static constexpr int value = QT == kQ4_0 && MS == 1 && T <= 2 ? 16 : 8;
};

// Weight loads in flight per wave (items ahead; divides T).
template <int T> struct Mf32Ahead { static constexpr int value = T == 4 ? 2 : T; };

template <int QT, int MS, int MODE, int W, int T>
__global__ __launch_bounds__(W * 64) void gemv_mf32_kernel(StreamJob job) {
  constexpr int PD = Mf32Fmt<QT>::PD;
  constexpr int BYTES = Fmt<QT>::BYTES;
  constexpr int RB = 8 * BYTES;                  // bytes of one 256-element range of a row
  constexpr int NPR = RB / 16;                   // 16-byte pieces of a row's range: 9 / 17
  constexpr int NQ = (16 * NPR + 63) / 64;       // piece loads per lane and item: 3 / 5
  constexpr int WS = (RB + 16 + 15) / 16 * 16;   // LDS bytes per staged row: 160 / 288
  constexpr int XS = 1040;                       // LDS bytes per staged activation row
  constexpr int REGION = (16 * WS > 4 * MS * XS ? 16 * WS : 4 * MS * XS) / 16;  // uint4 per wave
  constexpr int PF = Mf32Ahead<T>::value;
  __shared__ uint4 stage[W][REGION];
  __shared__ mf32_f32x4 red[W][T][MS][16];
  typedef int v4i __attribute__((ext_vector_type(4)));
  typedef float v4f __attribute__((ext_vector_type(4)));

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;  // waves of the launch (<= W), each with at least one range
  const int s = lane >> 4, g = (lane >> 2) & 3, j = lane & 3;
  const int k = job.k, M = job.m;
  const int nranges = (k + 255) >> 8;
  const int nblk = k >> 5;
  const int tiles = (job.rows + 15) >> 4;
  const int tile0 = blockIdx.x * T;
  const int rw = (nranges - wid + nw - 1) / nw;  // ranges wid, wid + nw, ... of this wave
  uint8_t* const reg = reinterpret_cast<uint8_t*>(stage[wid]);

  // per tile: a weight resource from the tile's first row to its matrix's
  // end (rows past the end read as zeros and are not stored; tiles past the
  // last repeat it and are not stored)
  __amdgpu_buffer_rsrc_t wr[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int tt = min(tile0 + t, tiles - 1);
    int mat = 0, lrow = tt * 16;
    if constexpr (MODE == kPlain) row_of(job, tt * 16, mat, lrow);
    const int n = pick4(mat, job.n[0], job.n[1], job.n[2], job.n[3]);
    wr[t] = make_rsrc(pick4(mat, job.w[0], job.w[1], job.w[2], job.w[3]) + (int64_t)lrow * job.row_bytes,
                      (uint32_t)((int64_t)(n - lrow) * job.row_bytes));
  }
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(job.x, (uint32_t)((int64_t)M * k * 4));

  // Loads are coalesced (lane l takes 16-byte pieces l, l + 64, ... of a
  // tile's 16 x RB bytes, or of each activation row's 1 KB) and staged in the
  // wave's LDS region; the MFMA layout is read back from there.  Lane
  // constants: each piece's byte offset in the tile (at range 0) and in LDS.
  int poff[NQ], pst[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int p = lane + 64 * q, pr = p / NPR, pc = p - pr * NPR;
    poff[q] = p < 16 * NPR ? (int)(pr * job.row_bytes) + 16 * pc : kMf32Oob;
    pst[q] = pr * WS + 16 * pc;
  }
  v4i wraw[PF][NQ];
  v4f xraw[4 * MS];
  // offsets of a range's pieces (the last range again past the wave's end:
  // those loads are never used)
  auto range_off = [&](int ri, int (&vo)[NQ]) {
    const int r = wid + nw * min(ri, rw - 1);
#pragma unroll
    for (int q = 0; q < NQ; ++q) vo[q] = poff[q] + r * RB;
  };
  auto wload = [&](const int (&vo)[NQ], int t, int b) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) wraw[b][q] = __builtin_amdgcn_raw_buffer_load_b128(wr[t], vo[q], 0, 0);
  };
  auto xload = [&](int ri) {
    const int r = wid + nw * ri;
    const bool in = ri < rw && r * 256 + 4 * lane < k;
#pragma unroll
    for (int q = 0; q < 4 * MS; ++q)
      xraw[q] = __builtin_amdgcn_raw_buffer_load_b128(xr, in && q < M ? q * k * 4 + r * 1024 + 16 * lane : kMf32Oob,
                                                      0, 0);
  };
  // activations in the A layout: lane (s, a = g, i = j), row 4 st + j,
  // elements 64 s + 16 g .. + 16 of the range; sn = -off * their sum
  auto xstage = [&](float (&xd)[MS][16], float (&sn)[MS]) {
#pragma unroll
    for (int q = 0; q < 4 * MS; ++q) *reinterpret_cast<v4f*>(reg + q * XS + 16 * lane) = xraw[q];
#pragma unroll
    for (int st = 0; st < MS; ++st) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const v4f v = *reinterpret_cast<const v4f*>(reg + (4 * st + j) * XS + 256 * s + 64 * g + 16 * h);
        xd[st][4 * h] = v.x;
        xd[st][4 * h + 1] = v.y;
        xd[st][4 * h + 2] = v.z;
        xd[st][4 * h + 3] = v.w;
      }
      float sum = xd[st][0];
#pragma unroll
      for (int v = 1; v < 16; ++v) sum += xd[st][v];
      sn[st] = -Mf32Fmt<QT>::OFF * sum;
    }
  };
  auto wstage = [&](int b) {
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      if (lane + 64 * q < 16 * NPR) *reinterpret_cast<v4i*>(reg + pst[q]) = wraw[b][q];
  };
  auto wread = [&](uint32_t (&w)[PD]) {
    const uint8_t* src = reg + (4 * g + j) * WS + 2 * BYTES * s;
#pragma unroll
    for (int d = 0; d < PD; ++d) w[d] = *reinterpret_cast<const uint32_t*>(src + 4 * d);
  };
  // the lane's two blocks exist (K is a multiple of 64, so both or neither)
  auto live = [&](int ri) { return (wid + nw * ri) * 8 + 2 * s < nblk; };

  float xb[MS][16], sn[MS];
  mf32_f32x4 acc[T][MS];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int st = 0; st < MS; ++st) acc[t][st] = mf32_f32x4{0.f, 0.f, 0.f, 0.f};

  // Scheduling barriers keep the load groups in program order (activations
  // of a range before its weights), so every wait is for the oldest group.
  int vcur[NQ], vnext[NQ];
  range_off(0, vcur);
  xload(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < PF; ++t) wload(vcur, t, t);
  __builtin_amdgcn_sched_barrier(0);
  for (int ri = 0; ri < rw; ++ri) {
    xstage(xb, sn);
    __builtin_amdgcn_sched_barrier(0);
    xload(ri + 1);
    __builtin_amdgcn_sched_barrier(0);
    range_off(ri + 1, vnext);
    const bool lv = live(ri);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int b = t % PF;
      wstage(b);
      // the buffer is free again: request the item PF ahead
      if (t + PF < T)
        wload(vcur, t + PF, b);
      else
        wload(vnext, t + PF - T, b);
      __builtin_amdgcn_sched_barrier(0);
      uint32_t w[PD];
      wread(w);
      mf32_item<QT, MS>(w, xb, sn, lv, acc[t]);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) vcur[q] = vnext[q];
  }

  // sums over the four lane groups s, parked per wave; then added in wave order
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int st = 0; st < MS; ++st) {
      mf32_f32x4 v = acc[t][st];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += __shfl_xor(v[q], 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += __shfl_xor(v[q], 32);
      if (s == 0) red[wid][t][st][lane] = v;
    }
  __syncthreads();

  const float* const redf = reinterpret_cast<const float*>(red);
  for (int o = threadIdx.x; o < T * MS * 64; o += nw * 64) {
    const int t = o / (MS * 64), st = (o / 64) % MS, rr = (o / 4) % 16, i = o % 4;
    const int m = 4 * st + i, orow = (tile0 + t) * 16 + rr;
    if (tile0 + t >= tiles || m >= M || orow >= job.rows) continue;
    float part[W];
#pragma unroll
    for (int w = 0; w < W; ++w) part[w] = w < nw ? redf[w * (T * MS * 64) + o] : 0.f;
    float tot = part[0];
#pragma unroll
    for (int w = 1; w < W; ++w)
      if (w < nw) tot += part[w];
    int omat = 0, olrow = orow;
    if constexpr (MODE == kPlain) row_of(job, orow, omat, olrow);
    const int n = pick4(omat, job.n[0], job.n[1], job.n[2], job.n[3]);
    const size_t oi = (size_t)m * n + olrow;
    if constexpr (MODE == kResid) {
      const float out = job.resid[oi] + tot;
      job.resid[oi] = out;
      if (job.resid_bf16) job.resid_bf16[oi] = f32_to_bf16_rne(out);
    } else {
      float* const yp = pick4(omat, job.y[0], job.y[1], job.y[2], job.y[3]);
      uint16_t* const ybp = pick4(omat, job.yb[0], job.yb[1], job.yb[2], job.yb[3]);
      const float out = tot + (job.bias ? job.bias[olrow] : 0.f);
      if (yp) yp[oi] = out;
      if (ybp) ybp[oi] = f32_to_bf16_rne(out);
    }
  }
}

// Whether the float32 matrix-core GEMV takes this launch.
inline bool mf32_ok(int qtype, const StreamJob& job, bool xbf16) {
  if (xbf16 || (qtype != kQ4_0 && qtype != kQ8_0) || job.m < 1 || job.m > 8 || job.k % 64 != 0 || job.x_stride)
    return false;
  if ((int64_t)job.m * job.k * 4 >= ((int64_t)1 << 31)) return false;
  for (int i = 0; i < job.n_mats; ++i) {
    if (job.n_mats > 1 && job.n[i] % 16 != 0) return false;
    if ((int64_t)job.n[i] * job.row_bytes >= ((int64_t)1 << 31)) return false;
  }
  return true;
}

// Waves per workgroup: at most W, at most one per K range, and the count in
// [3W/4, W] that leaves the fewest idle range slots (K = 14336: 56 ranges on
// 14 waves, four each).
inline int mf32_waves(int nranges, int wmax) {
  if (nranges <= wmax) return nranges;
  int best = wmax, waste = (nranges + wmax - 1) / wmax * wmax - nranges;
  for (int w = wmax - 1; w >= (3 * wmax + 3) / 4; --w) {
    const int ws = (nranges + w - 1) / w * w - nranges;
    if (ws < waste) best = w, waste = ws;
  }
  return best;
}

template <int QT, int MS, int MODE, int T>
static int launch_mf32(const StreamJob& job, hipStream_t s) {
  constexpr int W = Mf32Waves<QT, MS, T>::value;
  const int tiles = (job.rows + 15) / 16;
  const int waves = mf32_waves((job.k + 255) / 256, W);
  hipLaunchKernelGGL((gemv_mf32_kernel<QT, MS, MODE, W, T>), dim3((unsigned)((tiles + T - 1) / T)), dim3(waves * 64), 0,
                     s, job);
  return check_launch("gemv_mf32");
}

template <int QT, int MS, int MODE>
static int mf32_tiles(const StreamJob& job, hipStream_t s) {
  // tiles per workgroup: one workgroup per CU while the tiles last, up to four
  const int tiles = (job.rows + 15) / 16;
  const int t = std::min(4, std::max(1, (tiles + device_cus() - 1) / device_cus()));
  if (t == 1) return launch_mf32<QT, MS, MODE, 1>(job, s);
  if (t == 2) return launch_mf32<QT, MS, MODE, 2>(job, s);
  if (t == 3) return launch_mf32<QT, MS, MODE, 3>(job, s);
  return launch_mf32<QT, MS, MODE, 4>(job, s);
}

template <int MODE>
static int mf32_dispatch(int qtype, const StreamJob& job, hipStream_t s) {
  if (qtype == kQ4_0)
    return job.m <= 4 ? mf32_tiles<kQ4_0, 1, MODE>(job, s) : mf32_tiles<kQ4_0, 2, MODE>(job, s);
  return job.m <= 4 ? mf32_tiles<kQ8_0, 1, MODE>(job, s) : mf32_tiles<kQ8_0, 2, MODE>(job, s);
}

}  // namespace draco
