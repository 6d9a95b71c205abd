// Small-batch decode GEMV (2..16 activation rows) on the matrix cores.
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  m < M <= 16
//
// With M tokens every decoded weight serves M products, so the products go to
// v_mfma_f32_16x16x32_bf16: A = the activations (16 token rows x 32 k, rows
// past M are zero), B = the codes of 16 weight rows (exact in bf16 as
// 128 + code, one v_perm_b32 per pair), one MFMA per 32-element scale group
// (a Q4_K sub-block, a Q4_0 block), whose C operand is -(128 + off) S (S =
// sum_k x of the group, from one more MFMA against B = -(128 + off), shared by
// the wave's weight rows), so it yields sum x (code - off) with the bias
// cancelled.  w = a (code - off) + b per group; the scales are applied on the
// VALU, the Q4_K mins (b = -dmin m_g) through one more MFMA chain per row.
// float32 activations are split into three bf16 planes and take three MFMAs
// per group, against unbiased codes.
//
// Grid: a workgroup owns TPW tiles of 16 weight rows; four waves per tile
// split K (wave ks takes 256-element chunks ks, ks + 4, ...), reading their
// codes straight into registers (lane l decodes row l % 16, k-slice l / 16 of
// the MFMA layout) with the next chunk's loads in flight, and their partial
// 16 x 16 tiles are summed through LDS at the end.  Modes as the other
// decode GEMVs: kPlain (up to 4 matrices, every row count a multiple of 16),
// kSwiGLU (gate and up tiles side by side), kResid.
#pragma once

#include <climits>

#include "gemv_stream.h"

namespace draco {

typedef __bf16 mf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mf_f32x4 __attribute__((ext_vector_type(4)));

// Codes of one lane for one 256-element chunk: 8 groups x 8 codes (2 dwords
// of one byte per code), plus what the group coefficients need.
template <int QT> struct MfChunk;
template <> struct MfChunk<kQ4_K> { uint4 head; uint32_t qs[4][2]; };    // qs bytes 32p + 8q .. +8, p = 0..3
template <> struct MfChunk<kQ4_0> { uint32_t d[8]; uint32_t qs[8][2]; };  // per block: f16 d, 8 qs bytes

// Element offset (within the 256-element chunk) of group g's k-slice q.
template <int QT>
__device__ __forceinline__ int mf_pos(int g, int q) {
  if constexpr (QT == kQ4_K) return 64 * (g >> 1) + 32 * (g & 1) + 8 * q;
  return 32 * g + 8 * q;
}

// The lane's codes of one chunk; `rowoff` is the byte offset of the lane's
// weight row within the matrix buffer (a per-lane vector offset).
template <int QT>
__device__ __forceinline__ MfChunk<QT> mf_load(__amdgpu_buffer_rsrc_t rsrc, int rowoff, int chunk, int q) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  typedef int v2i __attribute__((ext_vector_type(2)));
  MfChunk<QT> c;
  if constexpr (QT == kQ4_K) {
    const int base = rowoff + chunk * 144;
    const v4i h = __builtin_amdgcn_raw_buffer_load_b128(rsrc, base, 0, 0);
    c.head = uint4{(uint32_t)h.x, (uint32_t)h.y, (uint32_t)h.z, (uint32_t)h.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const v2i t = __builtin_amdgcn_raw_buffer_load_b64(rsrc, base + 16 + 32 * p + 8 * q, 0, 0);
      c.qs[p][0] = (uint32_t)t.x;
      c.qs[p][1] = (uint32_t)t.y;
    }
  } else {
    // eight 18-byte blocks; lane slice q reads qs bytes 8 (q & 1) .. + 8 (low
    // nibbles for q < 2, high nibbles for q >= 2) -- unaligned 8-byte loads
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int base = rowoff + (chunk * 8 + g) * 18;
      c.d[g] = (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc, base, 0, 0);
      const v2i t = __builtin_amdgcn_raw_buffer_load_b64(rsrc, base + 2 + 8 * (q & 1), 0, 0);
      c.qs[g][0] = (uint32_t)t.x;
      c.qs[g][1] = (uint32_t)t.y;
    }
  }
  return c;
}

// B operand of group g: 8 codes as bf16 (128 + code), element order of the k-slice.
template <int QT>
__device__ __forceinline__ mf_bf16x8 mf_codes(const MfChunk<QT>& c, int g, int q) {
  uint32_t w0, w1;
  if constexpr (QT == kQ4_K) {
    w0 = (g & 1) ? nib_hi(c.qs[g >> 1][0]) : nib_lo(c.qs[g >> 1][0]);
    w1 = (g & 1) ? nib_hi(c.qs[g >> 1][1]) : nib_lo(c.qs[g >> 1][1]);
  } else {
    const bool hi = q >= 2;
    w0 = hi ? nib_hi(c.qs[g][0]) : nib_lo(c.qs[g][0]);
    w1 = hi ? nib_hi(c.qs[g][1]) : nib_lo(c.qs[g][1]);
  }
  const uint32_t v[4] = {code_pair_lo(w0), code_pair_hi(w0), code_pair_lo(w1), code_pair_hi(w1)};
  return __builtin_bit_cast(mf_bf16x8, v);
}

// Byte I of w as float (v_cvt_f32_ubyteI).
template <int I>
__device__ __forceinline__ float cvt_ubyte(uint32_t w) {
  float f;
  if constexpr (I == 0)
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(w));
  else if constexpr (I == 1)
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(w));
  else if constexpr (I == 2)
    asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(w));
  else
    asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(w));
  return f;
}

// B operand without the 128 bias: the codes themselves as bf16 (exact small
// integers; byte -> float -> upper half of the float bits), used with float32
// activations, whose three-plane products otherwise lose too many bits in the
// cancellation of the bias.
template <int QT>
__device__ __forceinline__ mf_bf16x8 mf_codes_exact(const MfChunk<QT>& c, int g, int q) {
  uint32_t w0, w1;
  if constexpr (QT == kQ4_K) {
    w0 = (g & 1) ? nib_hi(c.qs[g >> 1][0]) : nib_lo(c.qs[g >> 1][0]);
    w1 = (g & 1) ? nib_hi(c.qs[g >> 1][1]) : nib_lo(c.qs[g >> 1][1]);
  } else {
    const bool hi = q >= 2;
    w0 = hi ? nib_hi(c.qs[g][0]) : nib_lo(c.qs[g][0]);
    w1 = hi ? nib_hi(c.qs[g][1]) : nib_lo(c.qs[g][1]);
  }
  // each code to float (exact; one v_cvt_f32_ubyteN per code of the masked
  // word -- left to itself the compiler extracts every byte first), pairs to
  // bf16 (exact: integers < 256) with one v_cvt_pk_bf16_f32 per pair
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  uint32_t v[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t w = i == 0 ? w0 : w1;
    const f32x2 lo = {cvt_ubyte<0>(w), cvt_ubyte<1>(w)}, hi = {cvt_ubyte<2>(w), cvt_ubyte<3>(w)};
    v[2 * i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2v));
    v[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2v));
  }
  return __builtin_bit_cast(mf_bf16x8, v);
}

// Group coefficients: w = a * (code - off) + b; off folds Q4_0's code offset
// into the bias subtraction below (one cancellation instead of two).
template <int QT> struct MfOff { static constexpr float value = QT == kQ4_0 ? 8.f : 0.f; };

template <int QT>
__device__ __forceinline__ void mf_coeffs(const MfChunk<QT>& c, float (&a)[8], float (&cb)[8]) {
  if constexpr (QT == kQ4_K) {
    const float d = f16_bits_to_f32(c.head.x), dmin = f16_bits_to_f32(c.head.x >> 16);
    const uint32_t s0 = c.head.y, s1 = c.head.z, s2 = c.head.w;
    const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, m_lo = s1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const float sc = ubyte_f(g < 4 ? sc_lo : sc_hi, g & 3);
      const float mn = ubyte_f(g < 4 ? m_lo : m_hi, g & 3);
      a[g] = d * sc;
      cb[g] = -(dmin * mn);
    }
  } else {
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      a[g] = f16_bits_to_f32(c.d[g]);
      cb[g] = 0.f;
    }
  }
}

// A operand: 8 activations of token row m at element p of the chunk.  Rows
// past M read row M - 1 instead of zeros: row m of the product depends only
// on row m of A, and rows >= M are never stored.  float32 activations are split exactly enough into three bf16
// planes x = hi + mid + lo (each the round-to-nearest bf16 of what the
// previous ones leave; |x - hi - mid - lo| <= 2^-27 |x|): a two-plane split
// (2^-18) is not enough for the 1e-3 elementwise bound on outputs near zero.
template <bool XBF16>
__device__ __forceinline__ void mf_load_x(const void* __restrict__ xrow, int p, mf_bf16x8 (&pl)[XBF16 ? 1 : 3]) {
  if constexpr (XBF16) {
    const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xrow) + p);
    pl[0] = __builtin_bit_cast(mf_bf16x8, v);
  } else {
    float f[8];
    {
      const float4* s = reinterpret_cast<const float4*>(static_cast<const float*>(xrow) + p);
      const float4 u = s[0], w = s[1];
      f[0] = u.x; f[1] = u.y; f[2] = u.z; f[3] = u.w; f[4] = w.x; f[5] = w.y; f[6] = w.z; f[7] = w.w;
    }
    uint32_t b[3][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t part[3][2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        float rem = f[2 * i + e];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          part[j][e] = f32_to_bf16_rne(rem);
          rem -= __uint_as_float(part[j][e] << 16);
        }
      }
#pragma unroll
      for (int j = 0; j < 3; ++j) b[j][i] = part[j][0] | (part[j][1] << 16);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) pl[j] = __builtin_bit_cast(mf_bf16x8, b[j]);
  }
}

// Group sums of one chunk's bf16 activations (x as the A operand of the 16 x 16
// x 32 MFMA: lane (q, nl) holds token row nl, k-slice q of each group) in the A
// layout of v_mfma_f32_16x16x4f32: sx[b] = sum of group 4b + q of token row nl.
// Each lane adds its slice, the four slices meet across lanes l ^ 16, l ^ 32.
__device__ __forceinline__ void mf_group_sums(const mf_bf16x8 (&x)[8][1], int q, float (&sx)[2]) {
  float p[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const uint4 u = __builtin_bit_cast(uint4, x[g][0]);
    const uint32_t h[4] = {u.x, u.y, u.z, u.w};
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) t += __uint_as_float(h[i] << 16) + __uint_as_float(h[i] & 0xFFFF0000u);
    t += __shfl_xor(t, 16);
    p[g] = t + __shfl_xor(t, 32);
  }
  sx[0] = q == 0 ? p[0] : q == 1 ? p[1] : q == 2 ? p[2] : p[3];
  sx[1] = q == 0 ? p[4] : q == 1 ? p[5] : q == 2 ? p[6] : p[7];
}

// The same for float32 activations held as three bf16 planes (each element's
// three planes added in float32 first).
__device__ __forceinline__ void mf_group_sums3(const mf_bf16x8 (&x)[8][3], int q, float (&sx)[2]) {
  float p[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    uint32_t h[3][4];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const uint4 u = __builtin_bit_cast(uint4, x[g][j]);
      h[j][0] = u.x; h[j][1] = u.y; h[j][2] = u.z; h[j][3] = u.w;
    }
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = __uint_as_float(h[0][i] << 16) + __uint_as_float(h[1][i] << 16) + __uint_as_float(h[2][i] << 16);
      const float hi = __uint_as_float(h[0][i] & 0xFFFF0000u) + __uint_as_float(h[1][i] & 0xFFFF0000u) +
                       __uint_as_float(h[2][i] & 0xFFFF0000u);
      t += lo + hi;
    }
    t += __shfl_xor(t, 16);
    p[g] = t + __shfl_xor(t, 32);
  }
  sx[0] = q == 0 ? p[0] : q == 1 ? p[1] : q == 2 ? p[2] : p[3];
  sx[1] = q == 0 ? p[4] : q == 1 ? p[5] : q == 2 ? p[6] : p[7];
}

// acc += the products of one 256-element chunk: activations x (per group, NP
// bf16 planes) against NR weight rows' codes w; sx (SX): the chunk's group
// sums from mf_group_sums.
//
// bf16 activations: the group sums come from an MFMA against B = -(128 + off)
// in every element, so they arrive already times -(128 + off), and enter the
// codes' MFMA as its C operand: dg = -(128 + off) S + sum x (128 + code) =
// sum x (code - off), the code bias cancelled inside the matrix core before
// anything is scaled.  Q4_K: the group scales are applied per group
// (t += sc_g dg_g, sc_g the 6-bit integer) and d once per chunk; the min
// term dmin sum_g m_g S_g is one more MFMA chain per row (B = m_g, exact in
// bf16), scaled by dmin once per chunk.  Q4_0: acc += d_g dg_g.
// float32 activations (three bf16 planes, codes without the bias): the group
// sums against all-ones and the scales on the VALU per group.
template <int QT, bool XBF16, int NR, bool SX>
__device__ __forceinline__ void mf_chunk_q4_impl(const mf_bf16x8 (&x)[8][XBF16 ? 1 : 3], const MfChunk<QT> (&w)[NR],
                                                 int q, mf_f32x4 (&acc)[NR], const float (&sx)[2]) {
  const mf_f32x4 z = {0.f, 0.f, 0.f, 0.f};
  if constexpr (XBF16) {
    // bf16 pairs (-128, -128) for Q4_K, (-136, -136) for Q4_0 (codes offset by 8)
    constexpr uint32_t kNeg = QT == kQ4_K ? 0xC300C300u : 0xC308C308u;
    const uint32_t negs[4] = {kNeg, kNeg, kNeg, kNeg};
    const mf_bf16x8 bneg = __builtin_bit_cast(mf_bf16x8, negs);
    if constexpr (QT == kQ4_K) {
      float sc[NR][8], mn[NR][2];
      uint32_t mw[NR][2];
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const uint32_t s0 = w[r].head.y, s1 = w[r].head.z, s2 = w[r].head.w;
        const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, m_lo = s1 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
        const uint32_t m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
#pragma unroll
        for (int g = 0; g < 8; ++g) sc[r][g] = ubyte_f(g < 4 ? sc_lo : sc_hi, g & 3);
        if constexpr (SX) {
          // B of the min MFMAs: m of groups q and 4 + q (row nl)
          mn[r][0] = (float)((m_lo >> (8 * q)) & 0xFFu);
          mn[r][1] = (float)((m_hi >> (8 * q)) & 0xFFu);
        } else {
          mw[r][0] = m_lo;
          mw[r][1] = m_hi;
        }
      }
      mf_f32x4 t[NR], t2[NR];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const mf_f32x4 sgn = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[g][0], bneg, z, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const mf_f32x4 dg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[g][0], mf_codes<QT>(w[r], g, q), sgn, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 4; ++v) t[r][v] = g == 0 ? sc[r][g] * dg[v] : fmaf(sc[r][g], dg[v], t[r][v]);
          if constexpr (!SX) {
            // sum_g m_g (-128 S_g), from the group sums the codes' MFMA used
            const float m = ubyte_f(mw[r][g >> 2], g & 3);
#pragma unroll
            for (int v = 0; v < 4; ++v) t2[r][v] = g == 0 ? m * sgn[v] : fmaf(m, sgn[v], t2[r][v]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const float d = f16_bits_to_f32(w[r].head.x), dmin = f16_bits_to_f32(w[r].head.x >> 16);
        float dm = dmin * (1.f / 128.f);  // t2 = -128 sum_g m_g S_g
        if constexpr (SX) {
          // sum_g m_g S_g in one pass of the float32 matrix cores: A = the group sums
          // (token row nl, group 4b + q), B = m (group 4b + q, weight row nl)
          t2[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(sx[0], mn[r][0], z, 0, 0, 0);
          t2[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(sx[1], mn[r][1], t2[r], 0, 0, 0);
          dm = -dmin;
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[r][v] = fmaf(dm, t2[r][v], fmaf(d, t[r][v], acc[r][v]));
      }
    } else {
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const mf_f32x4 sgn = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[g][0], bneg, z, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const mf_f32x4 dg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[g][0], mf_codes<QT>(w[r], g, q), sgn, 0, 0, 0);
          const float d = f16_bits_to_f32(w[r].d[g]);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[r][v] = fmaf(d, dg[v], acc[r][v]);
        }
      }
    }
  } else {
    constexpr int NP = 3;
    const uint32_t ones[4] = {kOnePair, kOnePair, kOnePair, kOnePair};
    const mf_bf16x8 bones = __builtin_bit_cast(mf_bf16x8, ones);
    float a[NR][8], cb[NR][8];
#pragma unroll
    for (int r = 0; r < NR; ++r) mf_coeffs<QT>(w[r], a[r], cb[r]);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      mf_f32x4 sg = z;
#pragma unroll
      for (int j = NP - 1; j >= 0; --j) sg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[g][j], bones, sg, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const mf_bf16x8 bc = mf_codes_exact<QT>(w[r], g, q);
        mf_f32x4 dg = z;
#pragma unroll
        for (int j = NP - 1; j >= 0; --j) dg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[g][j], bc, dg, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          // sum x * (code - off) = D - off S before it is scaled
          const float xcode = fmaf(-MfOff<QT>::value, sg[v], dg[v]);
          if constexpr (QT == kQ4_K) acc[r][v] = fmaf(cb[r][g], sg[v], acc[r][v]);
          acc[r][v] = fmaf(a[r][g], xcode, acc[r][v]);
        }
      }
    }
  }
}

template <int QT, bool XBF16, int NR>
__device__ __forceinline__ void mf_chunk_q4(const mf_bf16x8 (&x)[8][XBF16 ? 1 : 3], const MfChunk<QT> (&w)[NR],
                                            int q, mf_f32x4 (&acc)[NR]) {
  const float none[2] = {0.f, 0.f};
  mf_chunk_q4_impl<QT, XBF16, NR, false>(x, w, q, acc, none);
}
// The same with the chunk's group sums from mf_group_sums (Q4_K, bf16).
template <int NR>
__device__ __forceinline__ void mf_chunk_q4k_sx(const mf_bf16x8 (&x)[8][1], const MfChunk<kQ4_K> (&w)[NR], int q,
                                                mf_f32x4 (&acc)[NR], const float (&sx)[2]) {
  mf_chunk_q4_impl<kQ4_K, true, NR, true>(x, w, q, acc, sx);
}

// Q4_K against float32 activations as three bf16 planes, with the chunk's
// group sums from mf_group_sums3: per group three MFMAs against the exact
// codes (D = sum x q), t += sc_g D_g, d once per chunk; the min term
// sum_g m_g S_g from two v_mfma_f32_16x16x4f32 (A = the sums, B = m), times
// dmin once per chunk.
template <int NR>
__device__ __forceinline__ void mf_chunk_q4k_sx3(const mf_bf16x8 (&x)[8][3], const MfChunk<kQ4_K> (&w)[NR], int q,
                                                 mf_f32x4 (&acc)[NR], const float (&sx)[2]) {
  const mf_f32x4 z = {0.f, 0.f, 0.f, 0.f};
  float sc[NR][8], mn[NR][2];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const uint32_t s0 = w[r].head.y, s1 = w[r].head.z, s2 = w[r].head.w;
    const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, m_lo = s1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
#pragma unroll
    for (int g = 0; g < 8; ++g) sc[r][g] = ubyte_f(g < 4 ? sc_lo : sc_hi, g & 3);
    mn[r][0] = (float)((m_lo >> (8 * q)) & 0xFFu);
    mn[r][1] = (float)((m_hi >> (8 * q)) & 0xFFu);
  }
  mf_f32x4 t[NR];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const mf_bf16x8 bc = mf_codes_exact<kQ4_K>(w[r], g, q);
      mf_f32x4 dg = z;
#pragma unroll
      for (int j = 2; j >= 0; --j) dg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[g][j], bc, dg, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v) t[r][v] = g == 0 ? sc[r][g] * dg[v] : fmaf(sc[r][g], dg[v], t[r][v]);
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const float d = f16_bits_to_f32(w[r].head.x), dmin = f16_bits_to_f32(w[r].head.x >> 16);
    mf_f32x4 t2 = __builtin_amdgcn_mfma_f32_16x16x4f32(sx[0], mn[r][0], z, 0, 0, 0);
    t2 = __builtin_amdgcn_mfma_f32_16x16x4f32(sx[1], mn[r][1], t2, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[r][v] = fmaf(-dmin, t2[v], fmaf(d, t[r][v], acc[r][v]));
  }
}

// The three bf16 planes of a float32 value (hi, mid, lo: each the
// round-to-nearest bf16 of what the previous ones leave; the split
// mf_load_x does on the fly).
__device__ __forceinline__ void mf_split3(float v, uint16_t& hi, uint16_t& mid, uint16_t& lo) {
  const uint32_t a = f32_to_bf16_rne(v);
  const float r1 = v - __uint_as_float(a << 16);
  const uint32_t b = f32_to_bf16_rne(r1);
  hi = (uint16_t)a;
  mid = (uint16_t)b;
  lo = (uint16_t)f32_to_bf16_rne(r1 - __uint_as_float(b << 16));
}

// acc (the lane's 4 values of the 16 x 16 tile) += the products over the
// 256-element chunks ks, ks + KS, ... < chunks of NR weight rows (buffer
// resources rs, the lane's row at byte offset rowoff) with the lane's
// activation row xrow (KS waves split K).  Software pipeline: the activations
// and codes of chunk c + KS are loaded while chunk c is multiplied.
//
// XPL: the activations are already three bf16 planes (hi, mid, lo of a float32
// row, as mf_split3 writes them) at xrow, xrow + pstride, xrow + 2 pstride
// (uint16 elements); no split on the fly.
template <int QT, bool XBF16, int NR, bool XPL = false, int KS = 4>
__device__ __forceinline__ void mf_accumulate(const __amdgpu_buffer_rsrc_t (&rs)[NR], int rowoff,
                                              const void* __restrict__ xrow, int q, int ks, int chunks,
                                              mf_f32x4 (&acc)[NR], size_t pstride = 0) {
  static_assert(!(XPL && XBF16), "pre-split planes carry float32 activations");
  // two buffer sets used alternately (no copies)
  constexpr int NP = XBF16 ? 1 : 3;
  MfChunk<QT> wb[2][NR];
  mf_bf16x8 xb[2][8][NP];
  auto load_chunk = [&](int slot, int cc) {
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int p = cc * 256 + mf_pos<QT>(g, q);
      if constexpr (XPL) {
        const uint16_t* xp = static_cast<const uint16_t*>(xrow) + p;
#pragma unroll
        for (int j = 0; j < 3; ++j)
          xb[slot][g][j] = __builtin_bit_cast(mf_bf16x8, *reinterpret_cast<const uint4*>(xp + j * pstride));
      } else {
        mf_load_x<XBF16>(xrow, p, xb[slot][g]);
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) wb[slot][r] = mf_load<QT>(rs[r], rowoff, cc, q);
  };
  auto compute_chunk = [&](int slot) { mf_chunk_q4<QT, XBF16, NR>(xb[slot], wb[slot], q, acc); };
  if (ks < chunks) load_chunk(0, ks);
  for (int c = ks; c < chunks; c += 2 * KS) {
    if (c + KS < chunks) load_chunk(1, c + KS);
    compute_chunk(0);
    if (c + KS >= chunks) break;
    if (c + 2 * KS < chunks) load_chunk(0, c + 2 * KS);
    compute_chunk(1);
  }

}

// Q6_K: sixteen 16-weight groups per 256-weight chunk, each with its own int8
// scale, so one v_mfma_f32_16x16x16_bf16 per group (lane l: row / column
// l % 16, k slice 4 (l / 16)).  A lane's codes of group g = 8n + 2t + h
// (half n, shift t, sixteen-element half h) are bytes 16h + 4q .. + 4 of
// ql[64n + 32 (t & 1)] (nibble t >> 1) and of qh[32n] (bits 2t, 2t + 1):
// eight ql dwords and four qh dwords per lane and chunk, 2-byte aligned
// (unaligned loads).  With B = 128 + q exact in bf16 and w = d sc_g (q - 32),
// sum_k x w = d sc_g (D - 160 S) per group.
typedef short mf_s16x4 __attribute__((ext_vector_type(4)));
struct MfQ6 {
  uint32_t ql[8];  // [4n + 2 (t & 1) + h]
  uint32_t qh[4];  // [2n + h]
  uint4 sc;        // the 16 int8 group scales
  uint32_t d;
};

template <bool DL>
__device__ __forceinline__ MfQ6 mf_load_q6(__amdgpu_buffer_rsrc_t rsrc, int rowoff, int chunk, int q) {
  constexpr int QL = DL ? 0 : 2, QH = DL ? 128 : 130, SC = DL ? 192 : 194, D = DL ? 208 : 0;
  typedef int v4i __attribute__((ext_vector_type(4)));
  const int base = rowoff + chunk * 210;
  MfQ6 c;
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        c.ql[4 * n + 2 * tb + h] =
            (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsrc, base + QL + 64 * n + 32 * tb + 16 * h + 4 * q, 0, 0);
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      c.qh[2 * n + h] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsrc, base + QH + 32 * n + 16 * h + 4 * q, 0, 0);
  const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, base + SC, 0, 0);
  c.sc = uint4{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
  c.d = (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc, base + D, 0, 0);
  return c;
}

// B operand of group g: 4 codes as bf16 128 + q.
__device__ __forceinline__ mf_s16x4 mf_codes_q6(const MfQ6& c, int g) {
  const int n = g >> 3, t = (g >> 1) & 3, h = g & 1;
  const uint32_t lo = (c.ql[4 * n + 2 * (t & 1) + h] >> (4 * (t >> 1))) & 0x0F0F0F0Fu;
  const uint32_t hi = ((c.qh[2 * n + h] >> (2 * t)) & 0x03030303u) << 4;
  const uint32_t q = lo | hi;
  const uint32_t v[2] = {__builtin_amdgcn_perm(0x43434343u, q, 0x04010400u),
                         __builtin_amdgcn_perm(0x43434343u, q, 0x04030402u)};
  return __builtin_bit_cast(mf_s16x4, v);
}

// The group sums times -160 (an MFMA against B = -160, exact in bf16) are the
// C operand of the codes' MFMA, so dg = sum x (q - 32) leaves the matrix core
// with the bias cancelled; t += sc_g dg_g per group, times d once per chunk.
template <int NR>
__device__ __forceinline__ void mf_chunk_q6(const uint2 (&x)[16], const MfQ6 (&w)[NR], mf_f32x4 (&acc)[NR]) {
  const uint32_t neg2[2] = {0xC320C320u, 0xC320C320u};  // bf16 (-160, -160)
  const mf_s16x4 bneg = __builtin_bit_cast(mf_s16x4, neg2);
  float sc[NR][16];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const uint32_t sw[4] = {w[r].sc.x, w[r].sc.y, w[r].sc.z, w[r].sc.w};
#pragma unroll
    for (int g = 0; g < 16; ++g) sc[r][g] = sbyte_f(sw[g >> 2], g & 3);
  }
  const mf_f32x4 z = {0.f, 0.f, 0.f, 0.f};
  mf_f32x4 t[NR];
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    const mf_s16x4 av = __builtin_bit_cast(mf_s16x4, x[g]);
    const mf_f32x4 sgn = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bneg, z, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const mf_f32x4 dg = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, mf_codes_q6(w[r], g), sgn, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v) t[r][v] = g == 0 ? sc[r][g] * dg[v] : fmaf(sc[r][g], dg[v], t[r][v]);
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const float d = f16_bits_to_f32(w[r].d);
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[r][v] = fmaf(d, t[r][v], acc[r][v]);
  }
}

template <bool DL, int NR, int KS = 4>
__device__ __forceinline__ void mf_accumulate_q6k(const __amdgpu_buffer_rsrc_t (&rs)[NR], int rowoff,
                                                  const void* __restrict__ xrow, int q, int ks, int chunks,
                                                  mf_f32x4 (&acc)[NR]) {
  const uint16_t* x = static_cast<const uint16_t*>(xrow);
  MfQ6 wb[2][NR];
  uint2 xb[2][16];
  auto load_chunk = [&](int slot, int cc) {
#pragma unroll
    for (int g = 0; g < 16; ++g) xb[slot][g] = *reinterpret_cast<const uint2*>(x + cc * 256 + 16 * g + 4 * q);
#pragma unroll
    for (int r = 0; r < NR; ++r) wb[slot][r] = mf_load_q6<DL>(rs[r], rowoff, cc, q);
  };
  auto compute_chunk = [&](int slot) { mf_chunk_q6<NR>(xb[slot], wb[slot], acc); };
  if (ks < chunks) load_chunk(0, ks);
  for (int c = ks; c < chunks; c += 2 * KS) {
    if (c + KS < chunks) load_chunk(1, c + KS);
    compute_chunk(0);
    if (c + KS >= chunks) break;
    if (c + 2 * KS < chunks) load_chunk(0, c + 2 * KS);
    compute_chunk(1);
  }
}

// KS waves split K per tile (4, or 8 where there are too few tiles to give
// every CU more than four waves: 4096 x 14336, 256 tiles).
template <int QT, bool DL, bool XBF16, int MODE, int TPW, int KS = 4>
__global__ __launch_bounds__(TPW * KS * 64) void gemv_mfma_kernel(StreamJob job) {
  constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  __shared__ mf_f32x4 part[TPW][KS][NR][64];
  const int lane = threadIdx.x & 63;
  // wave-uniform indices in scalar registers (the buffer resources built from
  // them must be uniform, or every load becomes a waterfall loop)
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = wid / KS, ks = wid % KS;
  const int row0 = (blockIdx.x * TPW + t) * 16;
  const int q = lane >> 4, nl = lane & 15;
  const int k = job.k, M = job.m;
  const int chunks = k >> 8;

  // the tile's matrix (a tile never straddles two: every row count is a
  // multiple of 16) and the lane's row in it (clamped; rows past the end are
  // computed, not stored)
  const int trow = min(row0, job.rows - 1);
  int mat = 0, lrow0 = trow;
  if constexpr (MODE == kPlain) row_of(job, trow, mat, lrow0);
  __amdgpu_buffer_rsrc_t rs[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int mm = NR == 2 ? r : mat;
    rs[r] = make_rsrc(job.w[mm], (uint32_t)((int64_t)job.n[mm] * job.row_bytes));
  }
  // this workgroup's chunks: all, or split blockIdx.y's range
  constexpr int kChunkBytes = Fmt<QT>::BYTES * (256 / Fmt<QT>::QK);
  int c0 = 0, nch = chunks;
  if (job.part) {
    c0 = (int)blockIdx.y * job.split_chunks;
    nch = min(job.split_chunks, chunks - c0);
  }
  const int rowoff =
      (int)((int64_t)min(lrow0 + nl, job.n[NR == 2 ? 0 : mat] - 1) * job.row_bytes) + c0 * kChunkBytes;

  mf_f32x4 acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  const void* xrow =
      static_cast<const uint8_t*>(job.x) + ((size_t)min(nl, M - 1) * k + (size_t)c0 * 256) * (XBF16 ? 2 : 4);
  if constexpr (QT == kQ6_K)
    mf_accumulate_q6k<DL, NR, KS>(rs, rowoff, xrow, q, ks, nch, acc);
  else
    mf_accumulate<QT, XBF16, NR, false, KS>(rs, rowoff, xrow, q, ks, nch, acc);

  // sum the KS partial tiles
#pragma unroll
  for (int r = 0; r < NR; ++r) part[t][ks][r][lane] = acc[r];
  __syncthreads();
  if (ks != 0) return;
  mf_f32x4 tot[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    tot[r] = part[t][0][r][lane];
#pragma unroll
    for (int j = 1; j < KS; ++j) {
      const mf_f32x4 p = part[t][j][r][lane];
#pragma unroll
      for (int v = 0; v < 4; ++v) tot[r][v] += p[v];
    }
  }
  const int orow = row0 + nl;
  if (orow >= job.rows) return;
  int omat = 0, olrow = orow;
  if constexpr (MODE == kPlain) row_of(job, orow, omat, olrow);
  const int n = job.n[omat];
  if constexpr (MODE != kSwiGLU) {
    if (job.part) {  // one matrix: the split's raw sums
      float* const pp = job.part + (size_t)blockIdx.y * M * n;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (4 * q + v < M) pp[(size_t)(4 * q + v) * n + olrow] = tot[0][v];
      return;
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int m = 4 * q + v;  // D layout: lane l holds rows 4 (l / 16) + v, column l % 16
    if (m >= M) continue;
    const size_t o = (size_t)m * n + olrow;
    if constexpr (MODE == kResid) {
      const float out = job.resid[o] + tot[0][v];
      job.resid[o] = out;
      if (job.resid_bf16) job.resid_bf16[o] = f32_to_bf16_rne(out);
    } else {
      float out = tot[0][v];
      if constexpr (MODE == kSwiGLU) out = silu(tot[0][v]) * tot[1][v];
      if (MODE == kPlain && job.bias) out += job.bias[olrow];
      if (job.y[omat]) job.y[omat][o] = out;
      if (job.yb[omat]) job.yb[omat][o] = f32_to_bf16_rne(out);
    }
  }
}

// Persistent form for bf16 activations and K <= 4096 (at most 16 chunks): a
// fixed grid of workgroups walks the 16-row weight tiles (tile t, t + grid,
// ...).  Wave ks of a workgroup always takes chunks ks, ks + 4, ks + 8,
// ks + 12, so its activation fragments are loaded into registers once for
// the whole launch; per tile it streams only the weights, with the next
// tile's weights requested before the current tile's math (an empty buffer
// resource past the last tile or chunk keeps every wait count exact).  The
// four partial tiles meet in LDS (double-buffered, one barrier per tile) and
// wave 0 stores the result while the others go on.
template <int QT> struct MfpTypes;
template <> struct MfpTypes<kQ4_K> { typedef MfChunk<kQ4_K> W; typedef mf_bf16x8 X[8][1]; };
template <> struct MfpTypes<kQ4_0> { typedef MfChunk<kQ4_0> W; typedef mf_bf16x8 X[8][1]; };
template <> struct MfpTypes<kQ6_K> { typedef MfQ6 W; typedef uint2 X[16]; };

// The wave's activation fragments (chunks ks, ks + W, ... of token row xrow).
template <int QT, int W>
__device__ __forceinline__ void mfp_load_x(const uint16_t* __restrict__ xrow, int chunks, int ks, int q,
                                           typename MfpTypes<QT>::X (&xr)[16 / W]) {
#pragma unroll
  for (int j = 0; j < 16 / W; ++j) {
    const int cc = min(ks + W * j, chunks - 1);
    if constexpr (QT == kQ6_K) {
#pragma unroll
      for (int g = 0; g < 16; ++g) xr[j][g] = *reinterpret_cast<const uint2*>(xrow + cc * 256 + 16 * g + 4 * q);
    } else {
#pragma unroll
      for (int g = 0; g < 8; ++g) mf_load_x<true>(xrow, cc * 256 + mf_pos<QT>(g, q), xr[j][g]);
    }
  }
}

// A weight row as seen by one lane: its matrix's buffer resource and the row's
// byte offset.
struct MfRow {
  __amdgpu_buffer_rsrc_t rs;
  int rowoff;
};

// Streams this workgroup's ntiles weight tiles against resident activations.
// tile_rsrc(i, r) gives matrix r's resource and the lane's row offset for
// tile i (an MfRow; called for i < ntiles only); emit(i, tot) runs on wave 0 with tile
// i's summed 16 x 16 result.  Ends in a barrier (the partial buffers are free).
template <int QT, bool DL, int NR, int W, class TileRsrc, class Emit>
__device__ __forceinline__ void mfp_stream(const typename MfpTypes<QT>::X (&xr)[16 / W], int chunks, int ntiles,
                                           __amdgpu_buffer_rsrc_t empty, TileRsrc tile_rsrc, Emit emit,
                                           mf_f32x4 (&part)[2][W][NR][64]) {
  constexpr int CPW = 16 / W;
  typedef typename MfpTypes<QT>::W WChunk;
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4;
  auto load_tile = [&](int i, WChunk (&dst)[CPW][NR]) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      MfRow row{empty, 0};
      if (i < ntiles) row = tile_rsrc(i, r);
      const __amdgpu_buffer_rsrc_t rs = row.rs;
      const int rowoff = row.rowoff;
#pragma unroll
      for (int j = 0; j < CPW; ++j) {
        const int cc = ks + W * j;
        const __amdgpu_buffer_rsrc_t rj = cc < chunks ? rs : empty;
        if constexpr (QT == kQ6_K)
          dst[j][r] = mf_load_q6<DL>(rj, rowoff, min(cc, chunks - 1), q);
        else
          dst[j][r] = mf_load<QT>(rj, rowoff, min(cc, chunks - 1), q);
      }
    }
  };
  float sx[CPW][2];  // Q4_K: the resident chunks' group sums
  if constexpr (QT == kQ4_K)
#pragma unroll
    for (int j = 0; j < CPW; ++j) mf_group_sums(xr[j], q, sx[j]);
  WChunk wb[2][CPW][NR];
  load_tile(0, wb[0]);
  for (int i0 = 0; i0 < ntiles; i0 += 2) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int i = i0 + p;
      load_tile(i + 1, wb[p ^ 1]);
      __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the math
      if (i < ntiles) {
        mf_f32x4 acc[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < CPW; ++j) {
          if (ks + W * j < chunks) {
            if constexpr (QT == kQ6_K)
              mf_chunk_q6<NR>(xr[j], wb[p][j], acc);
            else if constexpr (QT == kQ4_K)
              mf_chunk_q4k_sx<NR>(xr[j], wb[p][j], q, acc, sx[j]);
            else
              mf_chunk_q4<QT, true, NR>(xr[j], wb[p][j], q, acc);
          }
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) part[p][ks][r][lane] = acc[r];
      }
      __syncthreads();
      if (i < ntiles && ks == 0) {
        mf_f32x4 tot[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          tot[r] = part[p][0][r][lane];
#pragma unroll
          for (int j = 1; j < W; ++j) {
            const mf_f32x4 pp = part[p][j][r][lane];
#pragma unroll
            for (int v = 0; v < 4; ++v) tot[r][v] += pp[v];
          }
        }
        emit(i, tot);
      }
    }
  }
  __syncthreads();
}

template <int QT, bool DL, int MODE, int W>
__global__ __launch_bounds__(W * 64) void gemv_mfp_kernel(StreamJob job) {
  constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  __shared__ mf_f32x4 part[2][W][NR][64];
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, nl = lane & 15;
  const int k = job.k, M = job.m;
  const int chunks = k >> 8;
  const int ntiles = job.rows >> 4;
  const int my_tiles = ntiles > (int)blockIdx.x ? (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;

  // the wave's activations, resident for the launch (rows past M repeat row M - 1)
  typename MfpTypes<QT>::X xr[16 / W];
  mfp_load_x<QT, W>(static_cast<const uint16_t*>(job.x) + (size_t)min(nl, M - 1) * k, chunks, ks, q, xr);

  // matrices of the launch (kPlain: row tiles of up to four matrices back to back)
  int c1 = INT_MAX, c2 = INT_MAX, c3 = INT_MAX;
  if constexpr (MODE == kPlain) {
    if (job.n_mats > 1) c1 = job.n[0];
    if (job.n_mats > 2) c2 = c1 + job.n[1];
    if (job.n_mats > 3) c3 = c2 + job.n[2];
  }
  // the launch's pointers and sizes as scalars (the lambdas below copy them;
  // a copy of the whole argument would be indexed at run time, from scratch)
  const uint8_t *w0 = job.w[0], *w1 = job.w[1], *w2 = job.w[2], *w3 = job.w[3];
  const int n0 = job.n[0], n1 = job.n[1], n2 = job.n[2], n3 = job.n[3];
  float *y0 = job.y[0], *y1 = job.y[1], *y2 = job.y[2], *y3 = job.y[3];
  uint16_t *b0 = job.yb[0], *b1 = job.yb[1], *b2 = job.yb[2], *b3 = job.yb[3];
  float* const resid = job.resid;
  uint16_t* const resid_bf16 = job.resid_bf16;
  const float* const bias = job.bias;
  const int row_bytes = job.row_bytes;
  // (chains of selects on a running value: a select keyed by an index would be
  // turned into a table lookup in scratch)
  auto pick = [](int mat, auto v0, auto v1, auto v2, auto v3) {
    auto v = v0;
    v = mat >= 1 ? v1 : v;
    v = mat >= 2 ? v2 : v;
    v = mat >= 3 ? v3 : v;
    return v;
  };
  auto locate = [=](int row, int& mat, int& lrow) {
    mat = 0;
    lrow = row;
    if constexpr (MODE == kPlain) {
      mat = (row >= c1) + (row >= c2) + (row >= c3);
      int base = row >= c1 ? c1 : 0;
      base = row >= c2 ? c2 : base;
      base = row >= c3 ? c3 : base;
      lrow = row - base;
    }
  };
  auto tile_rsrc = [=](int i, int r) {
    int mat, lrow;
    locate(16 * ((int)blockIdx.x + i * (int)gridDim.x), mat, lrow);
    const int mm = NR == 2 ? r : mat;
    const uint8_t* wp = pick(mm, w0, w1, w2, w3);
    const int nn = pick(mm, n0, n1, n2, n3);
    return MfRow{make_rsrc(wp, (uint32_t)((int64_t)nn * row_bytes)), (lrow + nl) * row_bytes};
  };
  auto emit = [=](int i, const mf_f32x4 (&tot)[NR]) {
    int omat, olrow;
    locate(16 * ((int)blockIdx.x + i * (int)gridDim.x) + nl, omat, olrow);
    const int n = pick(omat, n0, n1, n2, n3);
    float* const yp = pick(omat, y0, y1, y2, y3);
    uint16_t* const ybp = pick(omat, b0, b1, b2, b3);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * q + v;  // D layout: lane l holds rows 4 (l / 16) + v, column l % 16
      if (m >= M) continue;
      const size_t o = (size_t)m * n + olrow;
      if constexpr (MODE == kResid) {
        const float out = resid[o] + tot[0][v];
        resid[o] = out;
        if (resid_bf16) resid_bf16[o] = f32_to_bf16_rne(out);
      } else {
        float out = tot[0][v];
        if constexpr (MODE == kSwiGLU) out = silu(tot[0][v]) * tot[1][v];
        if (MODE == kPlain && bias) out += bias[olrow];
        if (yp) yp[o] = out;
        if (ybp) ybp[o] = f32_to_bf16_rne(out);
      }
    }
  };
  mfp_stream<QT, DL, NR, W>(xr, chunks, my_tiles, make_rsrc(w0, 0u), tile_rsrc, emit, part);
}

template <int QT, bool DL, int MODE, int W>
static int launch_gemv_mfp(const StreamJob& job, int blocks_per_cu, hipStream_t s) {
  if (job.k > 4096 || job.k % 256 != 0 || job.rows % 16 != 0)
    return set_error(DRACO_EINVAL_SHAPE, "persistent matrix-core GEMV takes K <= 4096 and whole 16-row tiles");
  const int tiles = job.rows / 16;
  const int blocks = std::max(1, std::min(tiles, device_cus() * blocks_per_cu));
  hipLaunchKernelGGL((gemv_mfp_kernel<QT, DL, MODE, W>), dim3(blocks), dim3(W * 64), 0, s, job);
  return check_launch("gemv_mfp");
}

// Whether the matrix-core GEMV takes this launch: K-quant Q4_K or Q4_0,
// 2..16 activation rows, K a multiple of 256, every matrix a whole number of
// 16-row tiles, 32-bit buffer offsets.
inline bool mfma_gemv_ok(int qtype, const StreamJob& job, bool xbf16) {
  if (!(qtype == kQ4_K || qtype == kQ4_0 || (qtype == kQ6_K && xbf16)) || job.m < 2 || job.m > 16 ||
      job.k % 256 != 0)
    return false;
  for (int i = 0; i < job.n_mats; ++i) {
    if (job.n[i] % 16 != 0) return false;
    if ((int64_t)job.n[i] * job.row_bytes >= ((int64_t)1 << 31)) return false;
  }
  return true;
}

// The split launch's second half: out = sum over s in order of part[s] (per
// element), then the mode's epilogue (kResid: resid += out and its bf16 copy;
// kPlain: y = out + bias).
template <int MODE>
__global__ __launch_bounds__(256) void gemv_split_sum_kernel(const float* __restrict__ part, int splits, int M, int n,
                                                             float* __restrict__ y, uint16_t* __restrict__ yb,
                                                             const float* __restrict__ bias) {
  const size_t total = (size_t)M * n;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  float acc = part[i];
  for (int s = 1; s < splits; ++s) acc += part[(size_t)s * total + i];
  if constexpr (MODE == kResid) {
    const float out = y[i] + acc;
    y[i] = out;
    if (yb) yb[i] = f32_to_bf16_rne(out);
  } else {
    const float out = acc + (bias ? bias[i % (size_t)n] : 0.f);
    if (y) y[i] = out;
    if (yb) yb[i] = f32_to_bf16_rne(out);
  }
}

// One split of a split-K launch with bf16 activations (Q4_K / Q6_K): grid
// (tiles, splits), eight waves, wave ks multiplying chunk 8 s + ks of its
// tile.  The split's activation slab (16 token rows x 8 chunks, 64 KB) is
// read by the whole workgroup as consecutive 16-byte pieces into LDS (rows
// padded by 16 bytes) and the lanes take their fragments from there: read
// straight from global memory, each fragment load touches 16 rows 28 KB
// apart and the slab's cache lines are fetched several times over.  The
// wave's weights are requested before the slab is staged.  Stores the raw
// 16 x 16 sums to part[s]; gemv_split_sum_kernel finishes.  RT row tiles
// per workgroup share the slab (measured on MI355X, 4096 x 14336 at 16 rows
// with the sum launch: Q6_K 31.8 / 39.1 / 35.7 us at RT = 1 / 2 / 4, Q4_K
// 23.6 / 27.7 / 24.2; launched with RT = 1).
template <int QT, bool DL, int RT = 1>
__global__ __launch_bounds__(512) void gemv_split_lx_kernel(StreamJob job) {
  constexpr int XS = 8 * 256 + 8;  // LDS row stride (bf16 elements)
  __shared__ __attribute__((aligned(16))) uint16_t xs[16 * XS];
  __shared__ mf_f32x4 part[8][RT][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int ks = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, nl = lane & 15;
  const int k = job.k, M = job.m, chunks = k >> 8;
  const int s = blockIdx.y, c0 = 8 * s, nch = min(8, chunks - c0);
  const int row0 = (int)blockIdx.x * 16 * RT;
  const int n = job.n[0];
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(job.w[0], (uint32_t)((int64_t)n * job.row_bytes));
  // the wave's chunk of each of its RT row tiles (an empty resource past the
  // split's last chunk)
  const int cc = c0 + ks;
  const __amdgpu_buffer_rsrc_t rw = ks < nch ? rs : make_rsrc(nullptr, 0u);
  typedef typename MfpTypes<QT>::W WChunk;
  WChunk wc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int rowoff = (int)((int64_t)min(row0 + 16 * t + nl, n - 1) * job.row_bytes);
    if constexpr (QT == kQ6_K)
      wc[t] = mf_load_q6<DL>(rw, rowoff, min(cc, chunks - 1), q);
    else
      wc[t] = mf_load<QT>(rw, rowoff, min(cc, chunks - 1), q);
  }
  // the slab: 16 rows x nch * 32 pieces of 16 bytes (rows past M repeat row M - 1)
  const uint16_t* x = static_cast<const uint16_t*>(job.x);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int pc = tid + 512 * j;
    const int row = pc >> 8, col = pc & 255;  // 256 pieces per row of 8 chunks
    if (col < nch * 32) {
      const uint4 v = *reinterpret_cast<const uint4*>(x + (size_t)min(row, M - 1) * k + c0 * 256 + col * 8);
      *reinterpret_cast<uint4*>(&xs[row * XS + col * 8]) = v;
    }
  }
  __syncthreads();
  mf_f32x4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  if (ks < nch) {
    const uint16_t* xr = &xs[nl * XS + ks * 256];
    if constexpr (QT == kQ6_K) {
      uint2 xf[16];
#pragma unroll
      for (int g = 0; g < 16; ++g) xf[g] = *reinterpret_cast<const uint2*>(xr + 16 * g + 4 * q);
      mf_chunk_q6<RT>(xf, wc, acc);
    } else {
      mf_bf16x8 xf[8][1];
#pragma unroll
      for (int g = 0; g < 8; ++g) xf[g][0] = *reinterpret_cast<const mf_bf16x8*>(xr + mf_pos<QT>(g, q));
      mf_chunk_q4<QT, true, RT>(xf, wc, q, acc);
    }
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) part[ks][t][lane] = acc[t];
  __syncthreads();
  if (ks >= RT) return;  // wave t < RT sums row tile t
  const int t = ks;
  mf_f32x4 tot = part[0][t][lane];
#pragma unroll
  for (int j = 1; j < 8; ++j) {
    const mf_f32x4 pp = part[j][t][lane];
#pragma unroll
    for (int v = 0; v < 4; ++v) tot[v] += pp[v];
  }
  const int orow = row0 + 16 * t + nl;
  if (orow >= n) return;
  float* const pp = job.part + (size_t)s * M * n;
#pragma unroll
  for (int v = 0; v < 4; ++v)
    if (4 * q + v < M) pp[(size_t)(4 * q + v) * n + orow] = tot[v];
}

// Splits of a one-matrix matrix-core launch with K > 4096 (one tile per
// workgroup, eight waves over K) that has fewer tiles than the GPU has CUs
// four times over: eight chunks per split (one per wave), as many splits as
// keep the grid within 16 workgroups per CU; 1 = no split.
inline int gemv_split_count(const StreamJob& job) {
  const int chunks = job.k >> 8;
  if (job.n_mats != 1 || job.k <= 4096) return 1;
  const int64_t tiles = (job.rows + 15) / 16;
  if (tiles >= (int64_t)device_cus() * 4) return 1;
  const int s = (chunks + 7) / 8;
  return tiles * s <= (int64_t)device_cus() * 16 ? s : 1;
}

// Workspace bytes of a split launch (0: not split).
inline size_t gemv_split_bytes(const StreamJob& job) {
  const int s = gemv_split_count(job);
  return s > 1 ? (size_t)s * job.m * job.n[0] * sizeof(float) : 0;
}

template <int QT, bool DL, bool XBF16, int MODE>
static int launch_gemv_mfma(const StreamJob& job, hipStream_t s) {
  const int tiles = (job.rows + 15) / 16;
  // two tiles per workgroup for very tall matrices (bf16 only: with float32
  // activations the 512-thread form would spill registers)
  if constexpr (XBF16) {
    if (tiles >= 2048) {
      hipLaunchKernelGGL((gemv_mfma_kernel<QT, DL, XBF16, MODE, 2>), dim3((tiles + 1) / 2), dim3(512), 0, s, job);
      return check_launch("gemv_mfma");
    }
  }
  // split K (job.part set by the caller from gemv_split_bytes): the grid's y
  // dimension walks the splits, then the ordered sum
  const int splits = job.part ? (job.k / 256 + job.split_chunks - 1) / job.split_chunks : 1;
  // bf16: eight waves split K (two per SIMD; 4096 x 14336 Q6_K at 16 rows 44.9
  // -> 42.4 us, at 8 rows 37.6 -> 34.6; Q4_K 25.8 -> 24.8); float32 activations
  // need all 512 registers of a lane (one wave per SIMD), so four
  if constexpr (XBF16 && (QT == kQ4_K || QT == kQ6_K)) {
    if (job.part && job.split_chunks == 8)
      hipLaunchKernelGGL((gemv_split_lx_kernel<QT, DL>), dim3(tiles, splits), dim3(512), 0, s, job);
    else
      hipLaunchKernelGGL((gemv_mfma_kernel<QT, DL, XBF16, MODE, 1, 8>), dim3(tiles, splits), dim3(512), 0, s, job);
  } else if constexpr (XBF16)
    hipLaunchKernelGGL((gemv_mfma_kernel<QT, DL, XBF16, MODE, 1, 8>), dim3(tiles, splits), dim3(512), 0, s, job);
  else
    hipLaunchKernelGGL((gemv_mfma_kernel<QT, DL, XBF16, MODE, 1>), dim3(tiles, splits), dim3(256), 0, s, job);
  if (int rc = check_launch("gemv_mfma")) return rc;
  if constexpr (MODE != kSwiGLU) {
    if (job.part) {
      const size_t total = (size_t)job.m * job.n[0];
      float* const y = MODE == kResid ? job.resid : job.y[0];
      uint16_t* const yb = MODE == kResid ? job.resid_bf16 : job.yb[0];
      hipLaunchKernelGGL(gemv_split_sum_kernel<MODE>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                         job.part, splits, job.m, job.n[0], y, yb, job.bias);
      return check_launch("gemv_split_sum");
    }
  }
  return 0;
}

}  // namespace draco
