// Register-level GEMV core shared by the decode GEMV and the MoE expert kernels.
//
// A wave64 owns R consecutive weight rows [n0, n0 + R) and walks their K axis
// in 32-weight units (lane l takes units l, l + 64, ...).  For each unit it
// loads the packed bytes of the R rows once, unpacks the codes in registers
// and accumulates, per group g of the unit,
//     acc[r][m] += a_g * sum_i(code_i * x_m[pos_i]) + b_g * sum_i(x_m[pos_i])
// so the block scale and min are applied once per group, not once per weight.
// The activations of a unit serve all R rows.  Accumulation is float32.
//
// Two variants:
//  * gemv_accumulate_lds: the activations are staged in LDS by the workgroup
//    first, and the weight units are double-buffered in registers: the loads
//    of unit u + 64 are issued before the math of unit u.  Because the vector
//    memory counter retires loads in issue order, the prefetch only overlaps
//    the math if the math reads nothing else from global memory -- hence x in
//    LDS (whose reads are counted separately).  With bfloat16 activations the
//    codes are turned into bf16 pairs (128 + code, exact: one v_perm_b32 per
//    pair against the constant byte 0x43) and multiplied with
//    v_dot2_f32_bf16; the bias 128 * sum(x) is folded into b_g.
//  * gemv_accumulate: activations read from global memory, no prefetch; used
//    where x does not fit in LDS (many activation rows, long K) and by MoE.
#pragma once

#include "gguf_common.h"

namespace draco {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}

// Sum over the 64 lanes, the same value in every lane: DPP within rows of 16
// lanes (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror: every lane then holds its row's sum s_r), then row_bcast:15 into
// rows 1 and 3 (s1 + s0, s3 + s2) and row_bcast:31 into rows 2 and 3, so lane
// 63 holds (s3 + s2) + (s1 + s0), read out as a wave-uniform value.  No LDS
// round trip; the bits equal a butterfly over lanes 16 and 32 (float addition
// is commutative, so every lane of the butterfly holds this same sum).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  v += dpp_f<0x142, 0xA>(v);
  v += dpp_f<0x143, 0xC>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over a 256-thread workgroup (4 waves), result in every thread; red:
// 4 floats of LDS.  Every thread must call it (two barriers).
__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum_dpp(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float silu(float g) { return g / (1.f + __expf(-g)); }

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

// bf16 pair (128 + byte0, 128 + byte1) / (128 + byte2, 128 + byte3) of a dword of
// small unsigned codes (< 128): bf16 0x43XX is exactly 128 + XX for XX < 128.
__device__ __forceinline__ uint32_t code_pair_lo(uint32_t v) { return __builtin_amdgcn_perm(0x43434343u, v, 0x04010400u); }
__device__ __forceinline__ uint32_t code_pair_hi(uint32_t v) { return __builtin_amdgcn_perm(0x43434343u, v, 0x04030402u); }
constexpr float kCodeBias = 128.f;
constexpr uint32_t kOnePair = 0x3F803F80u;  // bf16 (1.0, 1.0)

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
  if constexpr (QT == kQ8_0 || QT == kQ8_K) {
    a[0] = f16_bits_to_f32(r.d);
    b[0] = 0.f;
  } else if constexpr (QT == kQ4_0 || QT == kQ5_0) {
    a[0] = f16_bits_to_f32(r.d);
    b[0] = (QT == kQ4_0 ? -8.f : -16.f) * a[0];
  } else if constexpr (QT == kQ4_1 || QT == kQ5_1) {
    a[0] = f16_bits_to_f32(r.dm);
    b[0] = f16_bits_to_f32(r.dm >> 16);
  } else if constexpr (Fmt<QT>::FAM == kFamK4) {
    // all eight 6-bit scales / mins as bytes (SWAR form of the reference's
    // _scale_min), then this unit's two sub-blocks j0, j0 + 1 by byte select
    const float d = f16_bits_to_f32(r.head.x), dmin = f16_bits_to_f32(r.head.x >> 16);
    const uint32_t s0 = r.head.y, s1 = r.head.z, s2 = r.head.w;
    const int j0 = 2 * ((u & 7) >> 1);
    const bool hi = j0 >= 4;
    const uint32_t scw = hi ? ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u)) : (s0 & 0x3F3F3F3Fu);
    const uint32_t mw = hi ? (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u)) : (s1 & 0x3F3F3F3Fu);
    const int sh = 8 * (j0 & 3);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      a[g] = d * (float)((scw >> (sh + 8 * g)) & 0xFFu);
      b[g] = -(dmin * (float)((mw >> (sh + 8 * g)) & 0xFFu));
    }
  } else if constexpr (QT == kQ2_K) {
    // scale byte of group t: sc[8*half + 2*t + sub], low nibble scale, high nibble min
    const float d = f16_bits_to_f32(r.dm), dmin = f16_bits_to_f32(r.dm >> 16);
    const int sub = ((u & 7) >> 1) & 1;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t byte = (r.sc[t >> 1] >> (8 * (2 * (t & 1) + sub))) & 0xFFu;
      a[t] = d * (float)(byte & 0x0Fu);
      b[t] = -(dmin * (float)(byte >> 4));
    }
  } else if constexpr (QT == kQ3_K) {
    // 6-bit scale 8*half + 2*t + sub: low nibble from byte (2t + sub) % 8
    // (nibble `half`), top two bits from byte 8 + (2t + sub) % 4 (bits
    // 2*(2*half + t/2)); built as the two scale words of this half
    const float d = f16_bits_to_f32(r.d);
    const int half = (u & 7) >> 2, sub = ((u & 7) >> 1) & 1;
    const int nsh = 4 * half;
    const uint32_t wa = ((r.s12[0] >> nsh) & 0x0F0F0F0Fu) | (((r.s12[2] >> nsh) & 0x03030303u) << 4);
    const uint32_t wb = ((r.s12[1] >> nsh) & 0x0F0F0F0Fu) | (((r.s12[2] >> (nsh + 2)) & 0x03030303u) << 4);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t sc = ((t < 2 ? wa : wb) >> (8 * (2 * (t & 1) + sub))) & 0xFFu;
      a[t] = d * (float)((int)sc - 32);
      b[t] = -4.f * a[t];
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

// Four 1-bit fields (bits 0..3 of x) spread to bit 0 of each byte.
__device__ __forceinline__ uint32_t spread4(uint32_t x) { return ((x & 0xFu) * 0x00204081u) & 0x01010101u; }

// Dword j (codes 4j .. 4j+3, one per byte) of group g, unsigned codes only.
// `u` is the unit index (Q5_K and Q3_K select their high-bit plane by it).
template <int QT>
__device__ __forceinline__ uint32_t unit_code_dword(const Raw<QT>& r, int g, int j, int u) {
  if constexpr (QT == kQ4_0 || QT == kQ4_1) {
    return j < 4 ? nib_lo(r.q[j]) : nib_hi(r.q[j - 4]);
  } else if constexpr (QT == kQ5_0 || QT == kQ5_1) {
    const uint32_t n = j < 4 ? nib_lo(r.q[j]) : nib_hi(r.q[j - 4]);
    return n | (spread4(r.qh >> (4 * j)) << 4);
  } else if constexpr (QT == kQ4_K) {
    const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
    return g == 0 ? nib_lo(q[j]) : nib_hi(q[j]);
  } else if constexpr (QT == kQ5_K) {
    // fifth bit of sub-block 2*((u & 7) >> 1) + g is bit (that index) of qh[l]
    const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
    const uint32_t h[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    const int bit = 2 * ((u & 7) >> 1) + g;
    return (g == 0 ? nib_lo(q[j]) : nib_hi(q[j])) | (((h[j] >> bit) & 0x01010101u) << 4);
  } else if constexpr (QT == kQ2_K) {
    return (r.qs[j] >> (2 * g)) & 0x03030303u;
  } else if constexpr (QT == kQ3_K) {
    const int half = (u & 7) >> 2;
    return ((r.qs[j] >> (2 * g)) & 0x03030303u) | (((r.hm[j] >> (4 * half + g)) & 0x01010101u) << 2);
  } else {
    return q6_codes(g, r.qla[j], r.qlb[j], r.qh[j]);
  }
}

// Code of element i (0..GL-1) of group g as float.
template <int QT>
__device__ __forceinline__ float unit_code(const Raw<QT>& r, int g, int i, int u) {
  if constexpr (QT == kQ8_0 || QT == kQ8_K) {
    return sbyte_f(r.q[i >> 2], i & 3);
  } else {
    return ubyte_f(unit_code_dword<QT>(r, g, i >> 2, u), i & 3);
  }
}

// Formats on the bf16 dot2 path: unsigned codes carried as bf16 128 + code
// (one byte permute per pair), the 128 taken back out through the group's
// activation sum.  That cancellation costs log2(128 / max code) bits, so the
// 2- and 3-bit formats (Q2_K, Q3_K) take the float32 FMA path instead.
template <int QT> struct UnsignedCodes {
  static constexpr bool value = Fmt<QT>::OFF && QT != kQ2_K && QT != kQ3_K;
};

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
          if constexpr (F::OFF) {
#pragma unroll
            for (int i = 0; i < GL; ++i) xsum += xv[i];
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < GL; ++i) dot = fmaf(unit_code<QT>(raw[r], g, i, u), xv[i], dot);
            acc[r][mi] = fmaf(a[r][g], dot, acc[r][mi]);
            if constexpr (F::OFF) acc[r][mi] = fmaf(b[r][g], xsum, acc[r][mi]);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-staged activations + double-buffered weight units
// ---------------------------------------------------------------------------

// Copies activation rows 0..m-1 (rows m..MT-1 zero) into LDS as MT rows of k
// elements; all threads of the workgroup must call it (it ends in a barrier).
template <int MT, bool XBF16, class XRow>
__device__ __forceinline__ void stage_x_lds(uint4* lds, int m, int k, XRow xrow) {
  constexpr int XB = XBF16 ? 2 : 4;
  const int chunks = k * XB / 16;
  for (int i = threadIdx.x; i < MT * chunks; i += blockDim.x) {
    const int mi = i / chunks, c = i - mi * chunks;
    uint4 v = {0u, 0u, 0u, 0u};
    if (mi < m) v = reinterpret_cast<const uint4*>(xrow(mi))[c];
    lds[i] = v;
  }
  __syncthreads();
}

// Permuted LDS layout of staged activations (used when K is a whole number of
// 2048-element steps): within each step, the j-th 16-byte chunk that lane l
// reads for its unit (unit index l inside the step) is stored at slot
// j * 64 + l, so each LDS read instruction of a wave covers 1 KB contiguous
// (no bank conflicts).  CE = elements per 16-byte chunk.
template <bool XBF16> struct XChunk { static constexpr int CE = XBF16 ? 8 : 4; };

// Natural element offset (within a step) of chunk j of lane l.
template <int QT, bool XBF16>
__device__ __forceinline__ int perm_natural_pos(int l, int j) {
  constexpr int CE = XChunk<XBF16>::CE, GL = Fmt<QT>::GL;
  const int e = j * CE;
  return group_pos<QT>(l, e / GL) + (e % GL);
}

// Slot (j * 64 + l) of the permuted layout that holds natural chunk c of a
// step (elements CE * c .. CE * c + CE - 1): the inverse of perm_natural_pos.
template <int QT, bool XBF16>
__device__ __forceinline__ int perm_slot_of_chunk(int c) {
  constexpr int CE = XChunk<XBF16>::CE;
  const int p = c * CE;  // natural element offset within the 2048-element step
  int l, e;              // unit (= lane) and element index within the unit's G * GL activations
  if constexpr (Fmt<QT>::FAM == kFamK4) {
    const int q = p & 255;
    l = 8 * (p >> 8) + 2 * (q >> 6) + ((q >> 4) & 1);
    e = 16 * ((q >> 5) & 1) + (q & 15);
  } else if constexpr (Fmt<QT>::FAM == kFamK6) {
    const int q = p & 255;
    l = 8 * (p >> 8) + 4 * (q >> 7) + ((q >> 3) & 3);
    e = 8 * ((q >> 5) & 3) + (q & 7);
  } else {
    l = p >> 5;
    e = p & 31;
  }
  return (e / CE) * 64 + l;
}

// Stages activation rows 0..m-1 (rows m..MT-1 zero) into LDS in the
// permuted layout.  The global reads are contiguous (thread t reads chunk t,
// so a wave's load instruction covers 1 KB of consecutive bytes); only the
// LDS writes are scattered.  All threads of the workgroup must call it (it
// ends in a barrier).
template <int QT, int MT, bool XBF16, class XRow>
__device__ __forceinline__ void stage_x_lds_perm(uint4* lds, int m, int k, XRow xrow) {
  constexpr int CE = XChunk<XBF16>::CE;
  constexpr int CPS = 2048 / CE;  // chunks per step
  const int chunks = k / CE;      // per activation row
  for (int i = threadIdx.x; i < MT * chunks; i += blockDim.x) {
    const int mi = i / chunks, c = i - mi * chunks;
    const int step = c / CPS, cs = c - step * CPS;
    uint4 v = {0u, 0u, 0u, 0u};
    if (mi < m) v = reinterpret_cast<const uint4*>(xrow(mi))[c];
    lds[(size_t)mi * chunks + (size_t)step * CPS + perm_slot_of_chunk<QT, XBF16>(cs)] = v;
  }
  __syncthreads();
}

// Group sums from the permuted layout, [mi][unit][g]; ends in a barrier.
template <int QT, int MT, bool XBF16>
__device__ __forceinline__ void stage_group_sums_perm(const uint4* __restrict__ xs, float* __restrict__ xsum, int m,
                                                      int k) {
  constexpr int G = Fmt<QT>::G, GL = Fmt<QT>::GL, CE = XChunk<XBF16>::CE;
  constexpr int CPG = GL / CE;  // chunks per group
  const int units = k >> 5;
  for (int i = threadIdx.x; i < MT * units * G; i += blockDim.x) {
    const int mi = i / (units * G), rem = i - mi * units * G;
    const int u = rem / G, g = rem - u * G;
    float t = 0.f;
    if (mi < m) {
      const int step = u >> 6, l = u & 63;
      const uint4* base = xs + ((size_t)mi * k + (size_t)step * 2048) / CE;
#pragma unroll
      for (int jj = 0; jj < CPG; ++jj) {
        const uint4 v = base[(g * CPG + jj) * 64 + l];
        if constexpr (XBF16) {
          t += bf16_lo(v.x) + bf16_hi(v.x) + bf16_lo(v.y) + bf16_hi(v.y) + bf16_lo(v.z) + bf16_hi(v.z) +
               bf16_lo(v.w) + bf16_hi(v.w);
        } else {
          t += __uint_as_float(v.x) + __uint_as_float(v.y) + __uint_as_float(v.z) + __uint_as_float(v.w);
        }
      }
    }
    xsum[i] = t;
  }
  __syncthreads();
}

template <int QT, bool DL, int R>
__device__ __forceinline__ void load_rows(Raw<QT> (&dst)[R], const uint8_t* __restrict__ w, int64_t row_bytes,
                                          int n0, int n, int u) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = n0 + r < n ? n0 + r : n - 1;
    dst[r] = load_unit<QT, DL>(w, (int64_t)row * row_bytes, u);
  }
}

// One 32-weight unit of R rows against MT activation rows.  xs: activation
// rows (LDS or global), row stride k elements.  XPRE: xsum holds the
// per-group activation sums of every unit ([mi][unit][g], row stride
// units * G floats); otherwise they are summed here.
template <int QT, int MT, bool XBF16, int R, bool XPRE = false, bool PERM = false>
__device__ __forceinline__ void unit_math_lds(const Raw<QT> (&raw)[R], int u, int m, int k,
                                              const uint4* __restrict__ xs, float (&acc)[R][MT],
                                              const float* __restrict__ xsum = nullptr) {
  using F = Fmt<QT>;
  constexpr int G = F::G, GL = F::GL;
  const int units = k >> 5;
  // PERM: chunk c (16 bytes) of this unit's activations is at uint4 slot
  // (row base + step base) / CE + c * 64 + (u & 63)
  auto xchunk = [&](int mi, int c) -> const uint4* {
    constexpr int CE = XChunk<XBF16>::CE;
    return xs + ((size_t)mi * k + (size_t)(u >> 6) * 2048) / CE + c * 64 + (u & 63);
  };
  float a[R][G], b[R][G];
#pragma unroll
  for (int r = 0; r < R; ++r) unit_coeffs<QT>(raw[r], u, a[r], b[r]);

  if constexpr (XBF16 && UnsignedCodes<QT>::value) {
    // bf16 code pairs of every row, shared by all activation rows
    uint32_t cp[R][G][GL / 2];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < GL / 4; ++j) {
          const uint32_t c = unit_code_dword<QT>(raw[r], g, j, u);
          cp[r][g][2 * j] = code_pair_lo(c);
          cp[r][g][2 * j + 1] = code_pair_hi(c);
        }
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      if (mi < m) {
        const uint32_t* xrow = reinterpret_cast<const uint32_t*>(xs) + (size_t)mi * (k >> 1);
        float xsg[G];
        if constexpr (XPRE) {
          const float* p = xsum + ((size_t)mi * units + u) * G;
          if constexpr (G == 4) {
            const float4 v = *reinterpret_cast<const float4*>(p);
            xsg[0] = v.x; xsg[1] = v.y; xsg[2] = v.z; xsg[3] = v.w;
          } else if constexpr (G == 2) {
            const float2 v = *reinterpret_cast<const float2*>(p);
            xsg[0] = v.x; xsg[1] = v.y;
          } else {
            xsg[0] = p[0];
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          uint32_t xw[GL / 2];
#pragma unroll
          for (int j = 0; j < GL / 8; ++j) {
            const uint4 v = PERM ? *xchunk(mi, g * (GL / 8) + j)
                                 : reinterpret_cast<const uint4*>(xrow + (group_pos<QT>(u, g) >> 1))[j];
            xw[4 * j] = v.x; xw[4 * j + 1] = v.y; xw[4 * j + 2] = v.z; xw[4 * j + 3] = v.w;
          }
          if constexpr (!XPRE) {
            float t = 0.f;
#pragma unroll
            for (int j = 0; j < GL / 2; ++j) t = dot2bf(xw[j], kOnePair, t);
            xsg[g] = t;
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float dot = 0.f;
#pragma unroll
            for (int j = 0; j < GL / 2; ++j) dot = dot2bf(cp[r][g][j], xw[j], dot);
            acc[r][mi] = fmaf(a[r][g], dot, acc[r][mi]);
            acc[r][mi] = fmaf(b[r][g] - kCodeBias * a[r][g], xsg[g], acc[r][mi]);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      if (mi < m) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float xv[GL];
          if constexpr (PERM) {
            constexpr int CE = XChunk<XBF16>::CE;
#pragma unroll
            for (int j = 0; j < GL / CE; ++j) {
              const uint4 v = *xchunk(mi, g * (GL / CE) + j);
              if constexpr (XBF16) {
                xv[8 * j + 0] = bf16_lo(v.x); xv[8 * j + 1] = bf16_hi(v.x);
                xv[8 * j + 2] = bf16_lo(v.y); xv[8 * j + 3] = bf16_hi(v.y);
                xv[8 * j + 4] = bf16_lo(v.z); xv[8 * j + 5] = bf16_hi(v.z);
                xv[8 * j + 6] = bf16_lo(v.w); xv[8 * j + 7] = bf16_hi(v.w);
              } else {
                xv[4 * j + 0] = __uint_as_float(v.x); xv[4 * j + 1] = __uint_as_float(v.y);
                xv[4 * j + 2] = __uint_as_float(v.z); xv[4 * j + 3] = __uint_as_float(v.w);
              }
            }
          } else if constexpr (XBF16) {
            load_x<GL, true>(reinterpret_cast<const uint16_t*>(xs) + (size_t)mi * k, group_pos<QT>(u, g), xv);
          } else {
            load_x<GL, false>(reinterpret_cast<const float*>(xs) + (size_t)mi * k, group_pos<QT>(u, g), xv);
          }
          float xsum_g = 0.f;
          if constexpr (F::OFF) {
            if constexpr (XPRE) {
              xsum_g = xsum[((size_t)mi * units + u) * G + g];
            } else {
#pragma unroll
              for (int i = 0; i < GL; ++i) xsum_g += xv[i];
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < GL; ++i) dot = fmaf(unit_code<QT>(raw[r], g, i, u), xv[i], dot);
            acc[r][mi] = fmaf(a[r][g], dot, acc[r][mi]);
            if constexpr (F::OFF) acc[r][mi] = fmaf(b[r][g], xsum_g, acc[r][mi]);
          }
        }
      }
    }
  }
}

// Per-group activation sums of every unit, [mi][unit][g] (mi < MT; zero for
// mi >= m), from activations already staged in LDS; ends in a barrier.
template <int QT, int MT, bool XBF16>
__device__ __forceinline__ void stage_group_sums(const uint4* __restrict__ xs, float* __restrict__ xsum, int m,
                                                 int k) {
  constexpr int G = Fmt<QT>::G, GL = Fmt<QT>::GL;
  const int units = k >> 5;
  for (int i = threadIdx.x; i < MT * units * G; i += blockDim.x) {
    const int mi = i / (units * G), rem = i - mi * units * G;
    const int u = rem / G, g = rem - u * G;
    float t = 0.f;
    if (mi < m) {
      float xv[GL];
      if constexpr (XBF16) {
        load_x<GL, true>(reinterpret_cast<const uint16_t*>(xs) + (size_t)mi * k, group_pos<QT>(u, g), xv);
      } else {
        load_x<GL, false>(reinterpret_cast<const float*>(xs) + (size_t)mi * k, group_pos<QT>(u, g), xv);
      }
#pragma unroll
      for (int j = 0; j < GL; ++j) t += xv[j];
    }
    xsum[i] = t;
  }
  __syncthreads();
}

// Same contract as gemv_accumulate, activations already staged in LDS by stage_x_lds.
template <int QT, bool DL, int MT, bool XBF16, int R>
__device__ __forceinline__ void gemv_accumulate_lds(const uint8_t* __restrict__ w, int64_t row_bytes, int n0,
                                                    int n, int k, int m, const uint4* __restrict__ xs,
                                                    float (&acc)[R][MT]) {
  const int lane = threadIdx.x & 63;
  const int units = k >> 5;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[r][mi] = 0.f;
  Raw<QT> buf0[R], buf1[R];
  int u = lane;
  if (u < units) load_rows<QT, DL, R>(buf0, w, row_bytes, n0, n, u);
  while (u < units) {
    if (u + 64 < units) load_rows<QT, DL, R>(buf1, w, row_bytes, n0, n, u + 64);
    unit_math_lds<QT, MT, XBF16, R>(buf0, u, m, k, xs, acc);
    u += 64;
    if (u >= units) break;
    if (u + 64 < units) load_rows<QT, DL, R>(buf0, w, row_bytes, n0, n, u + 64);
    unit_math_lds<QT, MT, XBF16, R>(buf1, u, m, k, xs, acc);
    u += 64;
  }
}

}  // namespace draco
