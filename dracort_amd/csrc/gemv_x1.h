// Single-token decode GEMV (M = 1, bfloat16 activations) for the K-quants,
// the shape of every projection of a batch-1 decode step.
//
// Each lane decodes 64-weight units: a Q4_K unit is a quarter super-block
// (32 qs bytes = sub-blocks 2j and 2j + 1, one scale and min each), a Q6_K
// unit is a quarter super-block too (16 l values of one half, all four t
// rows, one int8 scale per t).  The per-unit fields are fetched with one
// vector load each: Q4_K's are 16-byte aligned; Q6_K's sit at even offsets
// (210-byte blocks) and use the unaligned dwordx4 / dwordx2 loads that the
// gfx9 HSA memory model allows, so a 64-weight Q6_K unit costs five load
// instructions instead of thirteen dword loads.
//
// Lane l of a wave owns unit l, l + 64, ... of every row the wave computes
// ("step" s covers units 64 s .. 64 s + 63), so the activations a lane needs
// are the same for all of its rows: the wave loads them into registers once
// per step (64 bfloat16 = 32 VGPRs), sums them per group, and reuses them for
// its R rows.  No LDS and no workgroup barriers: a wave issues the loads of a
// step for all R rows right after the activation loads and starts
// multiplying as soon as its first row has landed.
//
// Codes are turned into exact bfloat16 pairs (128 + code, one v_perm_b32 per
// pair) and multiplied with v_dot2_f32_bf16; scale and min are applied once
// per 32- (Q4_K) or 16-weight (Q6_K) group:
//   Q4_K  sum_i w_i x_i = a * (dot - 128 xs) + b * xs,   a = d sc, b = -dmin m
//   Q6_K  sum_i w_i x_i = a * (dot - 160 xs),            a = d sc  (codes - 32)
// with dot = sum (128 + code_i) x_i and xs = sum x_i over the group.
// Launch modes and epilogues as in gemv_stream.h (kPlain with up to 4
// matrices sharing x, kSwiGLU, kResid).
#pragma once

#include <climits>

#include "gemv_mfl.h"
#include "gemv_stream.h"
#include "gemv_x1b.h"
#include "gemv_mf32.h"

namespace draco {

template <int QT> struct X1Fmt;
template <> struct X1Fmt<kQ4_K> { static constexpr int UPB = 4, G = 2, GL = 32; };
template <> struct X1Fmt<kQ6_K> { static constexpr int UPB = 4, G = 4, GL = 16; };

template <int QT> struct X1Raw;
template <> struct X1Raw<kQ4_K> { uint4 head, qs0, qs1; };
template <> struct X1Raw<kQ6_K> { uint4 qla, qlb, qh; uint32_t sc0, sc1, d; };

typedef int x1_v4i __attribute__((ext_vector_type(4)));
typedef int x1_v2i __attribute__((ext_vector_type(2)));

struct X1Buf {
  __amdgpu_buffer_rsrc_t rsrc;
  int soff;  // wave-uniform byte offset of the row
  __device__ __forceinline__ uint4 b128(int off) const {
    const x1_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, soff, 0);
    return uint4{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
  }
  __device__ __forceinline__ void b64(int off, uint32_t& lo, uint32_t& hi) const {
    const x1_v2i v = __builtin_amdgcn_raw_buffer_load_b64(rsrc, off, soff, 0);
    lo = (uint32_t)v.x;
    hi = (uint32_t)v.y;
  }
  __device__ __forceinline__ uint32_t b16(int off) const {
    return (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc, off, soff, 0);
  }
};

// Unit u (64 weights) of a row; offsets relative to the row start.
template <int QT, bool DL>
__device__ __forceinline__ X1Raw<QT> x1_load(const X1Buf& b, int u) {
  X1Raw<QT> r;
  const int blk = (u >> 2) * Fmt<QT>::BYTES, j = u & 3;
  if constexpr (QT == kQ4_K) {
    r.head = b.b128(blk);
    r.qs0 = b.b128(blk + 16 + 32 * j);
    r.qs1 = b.b128(blk + 32 + 32 * j);
  } else {
    constexpr int QL = DL ? 0 : 2, QH = DL ? 128 : 130, SC = DL ? 192 : 194, D = DL ? 208 : 0;
    const int n = j >> 1, h = j & 1;
    r.qla = b.b128(blk + QL + 64 * n + 16 * h);
    r.qlb = b.b128(blk + QL + 64 * n + 32 + 16 * h);
    r.qh = b.b128(blk + QH + 32 * n + 16 * h);
    b.b64(blk + SC + 8 * n, r.sc0, r.sc1);
    r.d = b.b16(blk + D);
  }
  return r;
}

// Element offset (within the row) of group g of unit u.
template <int QT>
__device__ __forceinline__ int x1_group_pos(int u, int g) {
  const int j = u & 3;
  if constexpr (QT == kQ4_K) return 256 * (u >> 2) + 64 * j + 32 * g;
  return 256 * (u >> 2) + 128 * (j >> 1) + 32 * g + 16 * (j & 1);
}

// The lane's activations for unit u: G groups of GL bf16 = 8 x 16 bytes.
struct X1Act {
  uint32_t w[32];
  float xs[4];
};

template <int QT, bool FULL>
__device__ __forceinline__ void x1_load_x(const uint16_t* __restrict__ x, int u, bool live, X1Act& a) {
  constexpr int G = X1Fmt<QT>::G, GL = X1Fmt<QT>::GL, CPG = GL / 8;  // 16-byte chunks per group
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4* p = reinterpret_cast<const uint4*>(x + x1_group_pos<QT>(u, g));
#pragma unroll
    for (int c = 0; c < CPG; ++c) {
      uint4 v = p[c];
      if constexpr (!FULL) {
        if (!live) v = uint4{0u, 0u, 0u, 0u};
      }
      a.w[(g * CPG + c) * 4 + 0] = v.x;
      a.w[(g * CPG + c) * 4 + 1] = v.y;
      a.w[(g * CPG + c) * 4 + 2] = v.z;
      a.w[(g * CPG + c) * 4 + 3] = v.w;
    }
  }
}

template <int QT>
__device__ __forceinline__ void x1_group_sums(X1Act& a) {
  constexpr int G = X1Fmt<QT>::G, GL = X1Fmt<QT>::GL;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < GL / 2; ++j) t = dot2bf(a.w[g * (GL / 2) + j], kOnePair, t);
    a.xs[g] = t;
  }
}

// LDS image of the activations (XL kernels): for each step s (64 units of 64
// weights) 512 16-byte chunks in lane-permuted order -- chunk j of the
// activations of unit l at slot s * 512 + j * 64 + l, so the eight
// ds_read_b128 of a lane's unit are each 1 KB contiguous across the wave --
// followed by the per-group sums, float [step][g][64].
template <int QT>
__device__ __forceinline__ int x1_slot_of_chunk(int c) {  // natural chunk (8 bf16) within a step
  const int p = c * 8;
  if constexpr (QT == kQ4_K) return ((p & 63) >> 3) * 64 + (p >> 6);
  const int q = p & 255;
  const int u = 4 * (p >> 8) + 2 * (q >> 7) + ((q >> 4) & 1);
  const int j = 2 * ((q >> 5) & 3) + ((q >> 3) & 1);
  return j * 64 + u;
}

__host__ __device__ inline size_t x1_lds_bytes(int qtype, int k) {
  const int steps = ((k >> 6) + 63) >> 6;
  const int g = qtype == kQ4_K ? 2 : 4;
  return (size_t)steps * 512 * 16 + (size_t)steps * g * 64 * 4;
}

// the persistent kernel's LDS: the image, its sums and a 4 KB pad
__host__ __device__ inline size_t x1p_lds_bytes(int qtype, int k) { return x1_lds_bytes(qtype, k) + 256 * 16; }

// Group sums of the staged image (after the barrier that ends the stores);
// ends in a barrier.
template <int QT>
__device__ __forceinline__ void x1_stage_sums(uint4* lds, int k) {
  constexpr int G = X1Fmt<QT>::G, CPG = X1Fmt<QT>::GL / 8;
  const int units = k >> 6, steps = (units + 63) >> 6;
  float* sums = reinterpret_cast<float*>(lds + steps * 512);
  for (int i = threadIdx.x; i < units * G; i += blockDim.x) {
    const int u = i / G, g = i - u * G;
    const int st = u >> 6, l = u & 63;
    float t = 0.f;
#pragma unroll
    for (int cc = 0; cc < CPG; ++cc) {
      const uint4 v = lds[st * 512 + (g * CPG + cc) * 64 + l];
      t = dot2bf(v.x, kOnePair, t);
      t = dot2bf(v.y, kOnePair, t);
      t = dot2bf(v.z, kOnePair, t);
      t = dot2bf(v.w, kOnePair, t);
    }
    sums[(st * G + g) * 64 + l] = t;
  }
  __syncthreads();
}

// Every thread of the workgroup calls this; it ends in a barrier.
template <int QT>
__device__ __forceinline__ void x1_stage(uint4* lds, const uint16_t* __restrict__ x, int k) {
  const int chunks = k >> 3;
  const uint4* xs = reinterpret_cast<const uint4*>(x);
  for (int c = threadIdx.x; c < chunks; c += blockDim.x)
    lds[(c >> 9) * 512 + x1_slot_of_chunk<QT>(c & 511)] = xs[c];
  __syncthreads();
  x1_stage_sums<QT>(lds, k);
}

// The same from XC chunks per thread already in registers (chunk
// threadIdx.x + 256 j in xr[j]; workgroups of 256 threads, K <= 2048 XC).
// Chunks past K go to a 4 KB pad after the image (x1p_lds_bytes) instead of
// being skipped: with an unconditional store the loads stay where they were
// issued instead of being sunk into a branch behind the weight loads.
template <int XC>
__device__ __forceinline__ void x1_fetch_x(const void* __restrict__ x, int k, uint4 (&xr)[XC]) {
  const uint4* xs = static_cast<const uint4*>(x);
  const int chunks = k >> 3;
#pragma unroll
  for (int j = 0; j < XC; ++j) xr[j] = xs[min((int)threadIdx.x + 256 * j, chunks - 1)];
}

// The same two chunks from a float32 row h with the RMSNorm applied:
// y = h / sqrt(mean(h^2) + eps) * w, rounded to bf16 (draco/runtime/cpu/ops.py:15-19).
// red: 4 floats of LDS outside the activation image; every thread of the
// workgroup calls this (the sum of squares is a workgroup reduction).
// Workgroup 0 also stores the normalized row to x_norm (if not NULL).
__device__ __forceinline__ void x1_fetch_x_rmsnorm(const float* __restrict__ h, const float* __restrict__ w,
                                                   float eps, uint16_t* x_norm, int k, float* red, uint4 (&xr)[2]) {
  const int chunks = k >> 3;
  const float4* h4 = reinterpret_cast<const float4*>(h);
  const float4* w4 = reinterpret_cast<const float4*>(w);
  float4 v[4], g[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = min((int)threadIdx.x + 256 * j, chunks - 1);
    v[2 * j] = h4[2 * c];
    v[2 * j + 1] = h4[2 * c + 1];
    g[2 * j] = w4[2 * c];
    g[2 * j + 1] = w4[2 * c + 1];
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if ((int)threadIdx.x + 256 * j < chunks) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const float4 a = v[2 * j + q];
        ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
      }
    }
  }
  // x * (1 / r) in place of the reference's x / r: within one float32 ulp,
  // below the bfloat16 rounding that follows, and one division per thread
  // instead of sixteen
  const float inv = 1.f / sqrtf(block_sum_256(ss, red) / (float)k + eps);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    uint32_t pk[4];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float4 a = v[2 * j + q], b = g[2 * j + q];
      pk[2 * q] = f32_to_bf16_rne(a.x * inv * b.x) | ((uint32_t)f32_to_bf16_rne(a.y * inv * b.y) << 16);
      pk[2 * q + 1] = f32_to_bf16_rne(a.z * inv * b.z) | ((uint32_t)f32_to_bf16_rne(a.w * inv * b.w) << 16);
    }
    xr[j] = uint4{pk[0], pk[1], pk[2], pk[3]};
    const int c = (int)threadIdx.x + 256 * j;
    if (x_norm && blockIdx.x == 0 && c < chunks) reinterpret_cast<uint4*>(x_norm)[c] = xr[j];
  }
}

// The slots are computed for every chunk (clamped) and chosen by a select:
// a slot computed only for chunks inside the row put each store behind a
// branch, and the compiler then sank each chunk's load next to its store and
// waited on it there -- eight serialized loads in the 14336-wide down
// projection (Q6_K 4096 x 14336: 14.8 us, 14.1 with the loads issued together;
// Q4_K 10.8 -> 10.5 us).
//
// The slots and group sums of the units past the row end in the last step are
// zeroed, so every lane reads its step's activations without a mask (its
// weights there are the last unit's again, which meet zeros).
template <int QT, int XC>
__device__ __forceinline__ void x1_stage_regs(uint4* lds, const uint4 (&xr)[XC], int k) {
  constexpr int G = X1Fmt<QT>::G;
  const int chunks = k >> 3;
  const int pad = (int)(x1_lds_bytes(QT, k) / 16);
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int c = (int)threadIdx.x + 256 * j;
    const int cc = min(c, chunks - 1);
    const int slot = (cc >> 9) * 512 + x1_slot_of_chunk<QT>(cc & 511);
    lds[c < chunks ? slot : pad + (int)threadIdx.x] = xr[j];
  }
  const int units = k >> 6, steps = (units + 63) >> 6;
  const int l0 = units - 64 * (steps - 1);  // first dead lane of the last step
  float* sums = reinterpret_cast<float*>(lds + steps * 512);
  for (int i = threadIdx.x; i < (64 - l0) * 8; i += blockDim.x) {
    const int l = l0 + (i >> 3), j = i & 7;
    lds[(steps - 1) * 512 + j * 64 + l] = uint4{0u, 0u, 0u, 0u};
    if (j < G) sums[((steps - 1) * G + j) * 64 + l] = 0.f;
  }
  __syncthreads();
  x1_stage_sums<QT>(lds, k);
}

// The lane's activations of step s from the LDS image (zero when !live).
template <int QT>
__device__ __forceinline__ void x1_read_lds(const uint4* __restrict__ lds, int k, int s, int lane, bool live,
                                            X1Act& a) {
  constexpr int G = X1Fmt<QT>::G;
  const int steps = ((k >> 6) + 63) >> 6;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint4 v = lds[s * 512 + j * 64 + lane];
    if (!live) v = uint4{0u, 0u, 0u, 0u};
    a.w[4 * j + 0] = v.x;
    a.w[4 * j + 1] = v.y;
    a.w[4 * j + 2] = v.z;
    a.w[4 * j + 3] = v.w;
  }
  const float* sums = reinterpret_cast<const float*>(lds + steps * 512);
#pragma unroll
  for (int g = 0; g < G; ++g) a.xs[g] = live ? sums[(s * G + g) * 64 + lane] : 0.f;
}

// Per-lane constants of the unit position j = u & 3 (the same for every step
// of a lane, since a step is 64 units): Q4_K sub-block half and byte shift,
// Q6_K half-row h.
struct X1Lane {
  uint32_t hi_mask;  // Q4_K: all ones when the unit's sub-blocks are 4..7
  uint32_t sh;       // Q4_K: 16 * (j & 1), byte offset of sub-block 2j in the scale word; Q6_K: 8 * (j & 1)
};

template <int QT>
__device__ __forceinline__ X1Lane x1_lane(int lane) {
  const int j = lane & 3;
  X1Lane c;
  c.hi_mask = j >= 2 ? 0xFFFFFFFFu : 0u;
  c.sh = QT == kQ4_K ? 16u * (j & 1) : 8u * (j & 1);
  return c;
}

// sum_i w_i x_i over the unit.
template <int QT>
__device__ __forceinline__ float x1_unit_dot(const X1Raw<QT>& r, const X1Lane& c, const X1Act& a) {
  if constexpr (QT == kQ4_K) {
    const float d = f16_bits_to_f32(r.head.x), dmin = f16_bits_to_f32(r.head.x >> 16);
    // 6-bit scales / mins of sub-blocks 2j, 2j + 1 (the reference's _scale_min
    // in SWAR form: byte i of scw / mw belongs to sub-block i, or 4 + i when
    // the unit is in the upper half), selected without branches
    const uint32_t s0 = r.head.y, s1 = r.head.z, s2 = r.head.w;
    const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, m_lo = s1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    const uint32_t scw = ((sc_hi & c.hi_mask) | (sc_lo & ~c.hi_mask)) >> c.sh;
    const uint32_t mw = ((m_hi & c.hi_mask) | (m_lo & ~c.hi_mask)) >> c.sh;
    const uint32_t q[8] = {r.qs0.x, r.qs0.y, r.qs0.z, r.qs0.w, r.qs1.x, r.qs1.y, r.qs1.z, r.qs1.w};
    float out = 0.f;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t cw = g == 0 ? nib_lo(q[i]) : nib_hi(q[i]);
        dot = dot2bf(code_pair_lo(cw), a.w[16 * g + 2 * i], dot);
        dot = dot2bf(code_pair_hi(cw), a.w[16 * g + 2 * i + 1], dot);
      }
      const float av = d * ubyte_f(scw, g);
      // a * (dot - 128 xs) - dmin * m * xs
      out = fmaf(av, fmaf(-kCodeBias, a.xs[g], dot), out);
      out = fmaf(-(dmin * ubyte_f(mw, g)), a.xs[g], out);
    }
    return out;
  } else {
    const float d = f16_bits_to_f32(r.d);
    const uint32_t ql[2][4] = {{r.qla.x, r.qla.y, r.qla.z, r.qla.w}, {r.qlb.x, r.qlb.y, r.qlb.z, r.qlb.w}};
    const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    // scale of row t: sc[8n + h + 2t] = byte 2t of the 8 scale bytes shifted by h
    const uint32_t sa = r.sc0 >> c.sh, sb = r.sc1 >> c.sh;
    float out = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t cw = q6_codes(t, ql[0][i], ql[1][i], qh[i]);
        dot = dot2bf(code_pair_lo(cw), a.w[8 * t + 2 * i], dot);
        dot = dot2bf(code_pair_hi(cw), a.w[8 * t + 2 * i + 1], dot);
      }
      const float sc = sbyte_f(t < 2 ? sa : sb, 2 * (t & 1));
      out = fmaf(d * sc, fmaf(-(kCodeBias + 32.f), a.xs[t], dot), out);
    }
    return out;
  }
}

template <int QT, bool DL, int MODE, int R, bool FULL, int OCC, bool XL>
__global__ __launch_bounds__(256, OCC) void gemv_x1_kernel(StreamJob job) {
  constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  constexpr int RR = R * NR;
  extern __shared__ uint4 x1_smem[];
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * R;
  if constexpr (XL) x1_stage<QT>(x1_smem, static_cast<const uint16_t*>(job.x), job.k);
  if (row0 >= job.rows) return;
  const int units = job.k >> 6;
  const int steps = (units + 63) >> 6;
  const uint16_t* x = static_cast<const uint16_t*>(job.x);

  // buffer resource per matrix, row offsets in the scalar offset
  X1Buf rb[RR];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int grow = min(row0 + r, job.rows - 1);
    int mat = 0, lrow = grow;
    if constexpr (MODE == kPlain) row_of(job, grow, mat, lrow);
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      const int m = NR == 2 ? q : mat;
      rb[r * NR + q].rsrc = make_rsrc(job.w[m], (uint32_t)((int64_t)job.n[m] * job.row_bytes));
      rb[r * NR + q].soff = (int)((int64_t)lrow * job.row_bytes);
    }
  }

  const X1Lane lc = x1_lane<QT>(lane);
  float acc[RR];
#pragma unroll
  for (int i = 0; i < RR; ++i) acc[i] = 0.f;

  for (int s = 0; s < steps; ++s) {
    const int u = lane + 64 * s;
    const bool live = FULL || u < units;
    const int ul = live ? u : units - 1;  // lanes past the row end re-read the last unit, x = 0
    X1Raw<QT> raw[RR];
    X1Act xa;
    if constexpr (XL) {
#pragma unroll
      for (int i = 0; i < RR; ++i) raw[i] = x1_load<QT, DL>(rb[i], ul);
      x1_read_lds<QT>(x1_smem, job.k, s, lane, live, xa);
    } else {
      x1_load_x<QT, FULL>(x, ul, live, xa);
#pragma unroll
      for (int i = 0; i < RR; ++i) raw[i] = x1_load<QT, DL>(rb[i], ul);
      x1_group_sums<QT>(xa);
    }
#pragma unroll
    for (int i = 0; i < RR; ++i) acc[i] += x1_unit_dot<QT>(raw[i], lc, xa);
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int grow = row0 + r;
    int mat = 0, lrow = grow;
    if constexpr (MODE == kPlain) row_of(job, grow < job.rows ? grow : job.rows - 1, mat, lrow);
    float v[NR];
#pragma unroll
    for (int q = 0; q < NR; ++q) v[q] = wave_sum_dpp(acc[r * NR + q]);
    if (lane != r || grow >= job.rows) continue;
    const size_t o = (size_t)lrow;
    if constexpr (MODE == kResid) {
      const float out = job.resid[o] + v[0];
      job.resid[o] = out;
      if (job.resid_bf16) job.resid_bf16[o] = f32_to_bf16_rne(out);
    } else {
      float out = v[0];
      if constexpr (MODE == kSwiGLU) out = silu(v[0]) * v[1];
      if (MODE == kPlain && job.bias) out += job.bias[lrow];
      if (job.y[mat]) job.y[mat][o] = out;
      if (job.yb[mat]) job.yb[mat][o] = f32_to_bf16_rne(out);
    }
  }
}

// Rows of a persistent wave: w, w + W, w + 2W, ... of the launch's row
// space.  kPlain concatenates up to four matrices (row r belongs to matrix
// (r >= c1) + (r >= c2) + (r >= c3)); kSwiGLU pairs gate and up.  Buffer
// resources are built once; rows past the wave's last get an empty resource,
// so their loads are issued (keeping every wait count exact) but return
// zeros without touching memory.
template <int MODE>
struct X1Rows {
  static constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  static constexpr int NM = MODE == kPlain ? kMaxMats : NR;
  int w, W, nrow;
  int c1 = INT_MAX, c2 = INT_MAX, c3 = INT_MAX;
  __amdgpu_buffer_rsrc_t rs[NM];
  __amdgpu_buffer_rsrc_t empty;

  __device__ __forceinline__ X1Rows(const StreamJob& job) {
    W = gridDim.x * 4;
    w = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    nrow = job.rows > w ? (job.rows - w + W - 1) / W : 0;
    if constexpr (MODE == kPlain) {
      if (job.n_mats > 1) c1 = job.n[0];
      if (job.n_mats > 2) c2 = c1 + job.n[1];
      if (job.n_mats > 3) c3 = c2 + job.n[2];
    }
#pragma unroll
    for (int m = 0; m < NM; ++m)
      rs[m] = make_rsrc(job.w[m], m < job.n_mats || NR == 2 ? (uint32_t)((int64_t)job.n[m] * job.row_bytes) : 0u);
    empty = make_rsrc(job.w[0], 0u);
  }
  __device__ __forceinline__ void locate(int r, int& mat, int& lrow) const {
    mat = 0;
    lrow = r;
    if constexpr (MODE == kPlain) {
      mat = (r >= c1) + (r >= c2) + (r >= c3);
      lrow = r - (mat == 0 ? 0 : mat == 1 ? c1 : mat == 2 ? c2 : c3);
    }
  }
  // wave-uniform: matrix q (kSwiGLU) / the owning matrix (kPlain) of row i
  __device__ __forceinline__ X1Buf buf(const StreamJob& job, int i, int q) const {
    X1Buf b;
    if (i >= nrow) {
      b.rsrc = empty;
      b.soff = 0;
      return b;
    }
    int mat, lrow;
    locate(w + i * W, mat, lrow);
    if constexpr (MODE == kPlain) {
      b.rsrc = mat == 0 ? rs[0] : mat == 1 ? rs[1] : mat == 2 ? rs[2] : rs[3];
    } else {
      b.rsrc = rs[q];
    }
    b.soff = lrow * job.row_bytes;
    return b;
  }
  // lanes 0 .. cnt - 1 store the results of rows i0 + lane (held in res)
  __device__ __forceinline__ void flush(const StreamJob& job, int i0, int cnt, float res) const {
    const int lane = threadIdx.x & 63;
    if (lane >= cnt) return;
    int mat, lrow;
    locate(w + (i0 + lane) * W, mat, lrow);
    if constexpr (MODE == kResid) {
      const float out = job.resid[lrow] + res;
      job.resid[lrow] = out;
      if (job.resid_bf16) job.resid_bf16[lrow] = f32_to_bf16_rne(out);
    } else {
      float out = res;
      if (MODE == kPlain && job.bias) out += job.bias[lrow];
      float* y = job.y[0];
      uint16_t* yb = job.yb[0];
      if constexpr (MODE == kPlain) {
        y = mat == 0 ? job.y[0] : mat == 1 ? job.y[1] : mat == 2 ? job.y[2] : job.y[3];
        yb = mat == 0 ? job.yb[0] : mat == 1 ? job.yb[1] : mat == 2 ? job.yb[2] : job.yb[3];
      }
      if (y) y[lrow] = out;
      if (yb) yb[lrow] = f32_to_bf16_rne(out);
    }
  }
};

// Persistent form for rows of one step (K <= 4096): a fixed grid of waves,
// wave w computes rows w, w + W, w + 2W, ... (W = all waves) with the packed
// bytes of the next PF rows in flight while it multiplies the current one.
// Issue order keeps every vector-memory wait exact: the activations are
// requested first, then the first PF rows; each iteration requests row i + PF
// before it multiplies row i; results are kept in lane i % 64 of one register
// and stored after every 64 rows, so no store sits between the loads.  The
// activations (the bf16 LDS image) are read into registers once.
template <int QT, bool DL, int MODE, int PF, bool NORM = false>
__global__ __launch_bounds__(256) void gemv_x1p_kernel(StreamJob job) {
  constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  constexpr int NB = PF + 1;
  extern __shared__ uint4 x1_smem[];
  const int lane = threadIdx.x & 63;
  const X1Rows<MODE> rows(job);
  const int nrow = rows.nrow;
  const int k = job.k;
  const int units = k >> 6;
  const bool live = lane < units;
  const int ul = live ? lane : units - 1;

  // 1. activations (two 16-byte chunks per thread), then the first rows
  uint4 xr[2];
  if constexpr (!NORM) x1_fetch_x<2>(job.x, k, xr);
  X1Raw<QT> buf[NB][NR];
#pragma unroll
  for (int p = 0; p < PF; ++p)
#pragma unroll
    for (int q = 0; q < NR; ++q) buf[p][q] = x1_load<QT, DL>(rows.buf(job, p, q), ul);
  if constexpr (NORM) {
    // the row's RMSNorm (a workgroup reduction) after the first weight loads are out
    float* red = reinterpret_cast<float*>(x1_smem + x1p_lds_bytes(QT, k) / 16);
    x1_fetch_x_rmsnorm(static_cast<const float*>(job.x), job.norm_w, job.norm_eps, job.x_norm, k, red, xr);
  }

  // 2. the LDS image and group sums; the lane's activations into registers
  x1_stage_regs<QT, 2>(x1_smem, xr, k);
  if (nrow == 0) return;
  const X1Lane lc = x1_lane<QT>(lane);
  X1Act xa;
  x1_read_lds<QT>(x1_smem, k, 0, lane, live, xa);

  // 3. rows
  float res = 0.f;
  for (int i0 = 0; i0 < nrow; i0 += NB) {
#pragma unroll
    for (int p = 0; p < NB; ++p) {
      const int i = i0 + p;
#pragma unroll
      for (int q = 0; q < NR; ++q) buf[(p + PF) % NB][q] = x1_load<QT, DL>(rows.buf(job, i + PF, q), ul);
      __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the math
      if (i < nrow) {
        float v[NR];
#pragma unroll
        for (int q = 0; q < NR; ++q) v[q] = wave_sum_dpp(x1_unit_dot<QT>(buf[p][q], lc, xa));
        float out = v[0];
        if constexpr (MODE == kSwiGLU) out = silu(v[0]) * v[1];
        res = (lane == (i & 63)) ? out : res;
        if ((i & 63) == 63) rows.flush(job, i - 63, 64, res);
      }
    }
  }
  if (nrow & 63) rows.flush(job, nrow & ~63, nrow & 63, res);
}

template <int QT, bool DL, int MODE, int PF, bool NORM = false>
static int launch_x1p(const StreamJob& job, int blocks_per_cu, hipStream_t s) {
  if (job.k > 4096 || job.k % 256 != 0) return set_error(DRACO_EINVAL_SHAPE, "persistent GEMV takes K <= 4096");
  const size_t lds = x1p_lds_bytes(QT, job.k) + (NORM ? 16 : 0);
  const int need = (job.rows + 3) / 4;
  const int blocks = std::max(1, std::min(need, device_cus() * blocks_per_cu));
  hipLaunchKernelGGL((gemv_x1p_kernel<QT, DL, MODE, PF, NORM>), dim3(blocks), dim3(256), lds, s, job);
  return check_launch("gemv_x1p");
}

// Persistent form for rows of S steps (4096 < K <= 4096 S; the down
// projection, K = 14336, has S = 4): the same row walk as above over items
// (row, step), PF items ahead in flight (one: two was measured slower).  A step's activations come from the
// LDS image at every item (64 bf16 and the group sums per lane), the unit
// dots of a row accumulate per lane and meet in one wave reduction when the
// row's last step is done.
template <int QT, bool DL, int MODE, int S, int PF>
__global__ __launch_bounds__(256) void gemv_x1s_kernel(StreamJob job) {
  static_assert(MODE != kSwiGLU, "one matrix per row");
  constexpr int NB = PF + 1;  // item ring: the current item and PF in flight
  // rows per unrolled iteration: enough that every item's ring slot and step
  // are compile-time constants (the unit offsets of each step are then per-lane
  // constants of the launch)
  constexpr int RU = S % NB == 0 ? 1 : NB;
  constexpr int U = RU * S;
  extern __shared__ uint4 x1_smem[];
  const int lane = threadIdx.x & 63;
  const X1Rows<MODE> rows(job);
  const int nrow = rows.nrow;
  const int k = job.k;
  const int units = k >> 6;
  // the lane's unit of each step (lanes past the row end re-read the last
  // unit; their activations and sums are zero in the image)
  int ul[S];
#pragma unroll
  for (int s = 0; s < S; ++s) ul[s] = min(lane + 64 * s, units - 1);

  // 1. activations (2 S 16-byte chunks per thread), then the first item
  uint4 xr[2 * S];
  x1_fetch_x<2 * S>(job.x, k, xr);
  X1Raw<QT> buf[NB];
#pragma unroll
  for (int p = 0; p < PF; ++p) buf[p] = x1_load<QT, DL>(rows.buf(job, p / S, 0), ul[p % S]);

  // 2. the LDS image and group sums
  x1_stage_regs<QT, 2 * S>(x1_smem, xr, k);
  if (nrow == 0) return;
  const X1Lane lc = x1_lane<QT>(lane);

  // 3. items (row i, step s), U per iteration
  float res = 0.f, acc = 0.f;
  for (int i0 = 0; i0 < nrow; i0 += RU) {
#pragma unroll
    for (int p = 0; p < U; ++p) {
      const int i = i0 + p / S;
      const int s = p % S;
      const int pn = p + PF;
      buf[pn % NB] = x1_load<QT, DL>(rows.buf(job, i0 + pn / S, 0), ul[pn % S]);
      __builtin_amdgcn_sched_barrier(0);  // keep the load ahead of the math
      if (i < nrow) {
        X1Act xa;
        x1_read_lds<QT>(x1_smem, k, s, lane, true, xa);
        acc += x1_unit_dot<QT>(buf[p % NB], lc, xa);
        if (s == S - 1) {
          const float v = wave_sum_dpp(acc);
          acc = 0.f;
          res = (lane == (i & 63)) ? v : res;
          if ((i & 63) == 63) rows.flush(job, i - 63, 64, res);
        }
      }
    }
  }
  if (nrow & 63) rows.flush(job, nrow & ~63, nrow & 63, res);
}

template <int QT, bool DL, int MODE, int S, int PF = 1>
static int launch_x1s(const StreamJob& job, int blocks_per_cu, hipStream_t s) {
  const int steps = ((job.k >> 6) + 63) >> 6;
  if (steps != S || job.k % 256 != 0) return set_error(DRACO_EINVAL_SHAPE, "GEMV row of %d steps, kernel takes %d", steps, S);
  const size_t lds = x1p_lds_bytes(QT, job.k);
  if (lds > 64 * 1024) return set_error(DRACO_EINVAL_SHAPE, "activation image needs %zu bytes of LDS", lds);
  const int need = (job.rows + 3) / 4;
  const int blocks = std::max(1, std::min(need, device_cus() * blocks_per_cu));
  hipLaunchKernelGGL((gemv_x1s_kernel<QT, DL, MODE, S, PF>), dim3(blocks), dim3(256), lds, s, job);
  return check_launch("gemv_x1s");
}

template <int QT, bool DL, int MODE, int R, int OCC = 1, bool ALLOW_FULL = true, bool XL = false>
static int launch_x1(const StreamJob& job, hipStream_t s) {
  const int waves = (job.rows + R - 1) / R;
  const int blocks = (waves + 3) / 4;
  const size_t lds = XL ? x1_lds_bytes(QT, job.k) : 0;
  if (lds > 64 * 1024) return set_error(DRACO_EINVAL_SHAPE, "activation image needs %zu bytes of LDS", lds);
  if (ALLOW_FULL && (job.k >> 6) % 64 == 0)
    hipLaunchKernelGGL((gemv_x1_kernel<QT, DL, MODE, R, true, OCC, XL>), dim3(blocks), dim3(256), lds, s, job);
  else
    hipLaunchKernelGGL((gemv_x1_kernel<QT, DL, MODE, R, false, OCC, XL>), dim3(blocks), dim3(256), lds, s, job);
  return check_launch("gemv_x1");
}

}  // namespace draco

namespace draco {

// Decode GEMV dispatch: single-token bfloat16 launches of the K-quants go to
// the 64-weight-unit kernels above -- the persistent form when a row is one
// step (K <= 4096), the one-shot form for longer rows (both with the LDS
// activation image); everything else (Q8_0 / Q4_0, float32
// activations, 2..16 activation rows) to the streaming kernel.  The one-shot
// form is compiled with predicated loads (ALLOW_FULL = false): letting the
// compiler interleave each row's loads with the previous row's math was
// measured faster than hoisting every load of the step.
// Whether the persistent single-token kernel runs this launch (and so can
// take the fused RMSNorm prologue).
inline bool x1p_ok(int qtype, const StreamJob& job, bool xbf16) {
  if (!(job.m == 1 && xbf16 && (qtype == kQ4_K || qtype == kQ6_K) && job.k <= 4096)) return false;
  for (int i = 0; i < job.n_mats; ++i)
    if ((int64_t)job.n[i] * job.row_bytes >= ((int64_t)1 << 31)) return false;
  return true;
}

// The fused-RMSNorm launch (job.x float32, job.norm_w set); x1p_ok must hold.
template <int MODE>
static int gemv_dispatch_norm(int qtype, bool d_last, const StreamJob& job, hipStream_t s) {
  // two workgroups per CU (measured against 1-5 per CU on the q/k/v, gate/up
  // and lm_head launches of the Llama-3-8B step: q/k/v 7.33 us vs 7.78 at
  // three, gate/up 14.7 vs 15.6 at four, lm_head 77.4 vs 78.4 at four)
  constexpr int bpc = 2;
  if (qtype == kQ4_K) return launch_x1p<kQ4_K, false, MODE, 1, true>(job, bpc, s);
  return d_last ? launch_x1p<kQ6_K, true, MODE, 1, true>(job, bpc, s)
                : launch_x1p<kQ6_K, false, MODE, 1, true>(job, bpc, s);
}

template <int MODE>
static int gemv_dispatch_mode(int qtype, bool d_last, const StreamJob& job, bool xbf16, hipStream_t s) {
  bool x1 = job.m == 1 && xbf16 && (qtype == kQ4_K || qtype == kQ6_K);
  for (int i = 0; i < job.n_mats; ++i)
    if ((int64_t)job.n[i] * job.row_bytes >= ((int64_t)1 << 31)) x1 = false;  // 32-bit buffer offsets
  if (x1 && job.k <= 4096) {
    // one row in flight ahead of the math.  Single-matrix launches: four
    // workgroups per CU for long matrices, three below 8192 rows (measured:
    // 14336 x 4096 Q4_K 8.6 us at four vs 9.0 at two, 12288 rows 7.9 at four
    // vs 8.1 at three).  Launches that move two rows per item (kSwiGLU) or end
    // in the residual update: two per CU (gate/up 2 x 14336 x 4096 14.7 us vs
    // 15.6 at four, o 4096 x 4096 5.0 vs 5.1 at three)
    const int bpc = (MODE == kSwiGLU || MODE == kResid) ? 2 : job.rows >= 8192 ? 4 : 3;
    if (qtype == kQ4_K) return launch_x1p<kQ4_K, false, MODE, 1>(job, bpc, s);
    return d_last ? launch_x1p<kQ6_K, true, MODE, 1>(job, bpc, s) : launch_x1p<kQ6_K, false, MODE, 1>(job, bpc, s);
  }
  // one token, Q8_0 / Q4_0, rows of at most 4096: the block-format
  // single-token kernel (activations in registers, gemv_x1b.h)
  if constexpr (MODE != kSwiGLU) {
    if (x1b_ok(qtype, job)) return x1b_dispatch<MODE>(qtype, job, xbf16, s);
  }
  // float32 activations, 2..8 rows (or one row too long for the kernel
  // above), Q4_0 / Q8_0: the float32 matrix-core kernel (activations used as
  // they are, one 4 x 4 x 1 MFMA per 64 weights; Q4_0 4096 x 14336 at one
  // row 15.1 us against 17.0 on the streaming kernel)
  if constexpr (MODE != kSwiGLU) {
    if (mf32_ok(qtype, job, xbf16)) return mf32_dispatch<MODE>(qtype, job, s);
  }
  // activation rows too long for the LDS image: the streaming kernel over K
  // windows -- bf16 rows below 8, float32 rows up to 4, and 5..8 float32
  // rows when two windows cover K (Q4_0 14336 x 4096, 8 rows: 94 -> 51 us;
  // 4096 x 14336, 4 rows: 106 -> 54 us; 8 rows over seven windows was slower
  // than the matrix cores below, 101 against 84 us)
  if constexpr (MODE != kSwiGLU) {
    const int kw = stream_window_k(qtype, job, xbf16);
    const bool rows_ok = xbf16 ? job.m < 8 : (job.m <= 4 || (job.m <= 8 && job.k <= 2 * kw));
    // not the four-group formats: Q2_K / Q3_K / Q6_K at 4 bf16 rows of 14336
    // were slower windowed (32.1 -> 46.8, 54.6 -> 56.1, 44.9 -> 50.1 us; the
    // other seven types 1-14 % faster)
    const bool type_ok = qtype != kQ2_K && qtype != kQ3_K && qtype != kQ6_K;
    if (rows_ok && type_ok && kw >= 2048 && (MODE == kResid || (job.n_mats == 1 && job.y[0])))
      return stream_windowed<MODE>(qtype, d_last, job, xbf16, kw, s);
  }
  // 8..16 activation rows: the matrix-core kernel (measured faster than the
  // streaming kernel from 8 rows on; at 4 rows they tie or the latter wins)
  if (job.m >= 8 && mfma_gemv_ok(qtype, job, xbf16)) return gemv_mfma_dispatch<MODE>(qtype, d_last, job, xbf16, s);
  if constexpr (MODE != kSwiGLU) {
    // rows of 2..4 steps (K <= 16384, the down projection): the persistent
    // multi-step form
    const int steps = ((job.k >> 6) + 63) >> 6;
    if (x1 && steps >= 2 && steps <= 4 && job.k % 256 == 0 && x1p_lds_bytes(qtype, job.k) <= 64 * 1024) {
      constexpr int bpc = 2;  // Q6_K 4096 x 14336: 14.6 us at two per CU, 14.7 at three, 15.3 at four
#define DRACO_X1S(S_)                                                                      \
  if (steps == S_) {                                                                       \
    if (qtype == kQ4_K) return launch_x1s<kQ4_K, false, MODE, S_>(job, bpc, s);             \
    return d_last ? launch_x1s<kQ6_K, true, MODE, S_>(job, bpc, s)                         \
                  : launch_x1s<kQ6_K, false, MODE, S_>(job, bpc, s);                       \
  }
      DRACO_X1S(2)
      DRACO_X1S(3)
      DRACO_X1S(4)
#undef DRACO_X1S
    }
    if (x1 && x1_lds_bytes(qtype, job.k) <= 64 * 1024) {
      if (qtype == kQ4_K) return launch_x1<kQ4_K, false, MODE, 2, 1, false, true>(job, s);
      return d_last ? launch_x1<kQ6_K, true, MODE, 2, 1, false, true>(job, s)
                    : launch_x1<kQ6_K, false, MODE, 2, 1, false, true>(job, s);
    }
  }
  return stream_dispatch<MODE>(qtype, d_last, job, xbf16, s);
}

}  // namespace draco
