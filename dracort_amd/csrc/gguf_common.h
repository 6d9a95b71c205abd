// GGUF block geometry and per-lane block decoders for gfx950.
//
// Block layouts follow the reference's table (draco/format/gguf.py:75-87):
//   Q4_0  32 elems,  18 B : f16 d | u8 qs[16]  (elem i = low nibble of qs[i], elem 16+i = high nibble)
//   Q4_1  32 elems,  20 B : f16 d | f16 m | u8 qs[16]
//   Q5_0  32 elems,  22 B : f16 d | u32 qh | u8 qs[16]   (bit e of qh = fifth bit of elem e)
//   Q5_1  32 elems,  24 B : f16 d | f16 m | u32 qh | u8 qs[16]
//   Q8_0  32 elems,  34 B : f16 d | int8 qs[32]
//   Q8_K 256 elems, 258 B : f16 d | int8 qs[256]
//   Q2_K 256 elems,  84 B : f16 d | f16 dmin | u8 qs[64] | u8 scales[16]
//   Q3_K 256 elems, 110 B : f16 d | u8 scales[12] | u8 qs[64] | u8 hmask[32]
//   Q4_K 256 elems, 144 B : f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
//   Q5_K 256 elems, 176 B : f16 d | f16 dmin | u8 scales[12] | u8 qh[32] | u8 qs[128]
//   Q6_K 256 elems, 210 B : f16 d | u8 ql[128] | u8 qh[64] | i8 scales[16]
// and, with the layout flag (upstream ggml field order, DL = true):
//   Q2_K : u8 scales[16] | u8 qs[64] | f16 d | f16 dmin
//   Q3_K : u8 hmask[32] | u8 qs[64] | u8 scales[12] | f16 d
//   Q6_K : u8 ql[128] | u8 qh[64] | i8 scales[16] | f16 d
//
// Every kernel here walks a weight row in "units" of 32 weights.  A unit is
// the natural slice one lane decodes from one load group; the formats fall in
// three families by where a unit's weights sit in the row:
//   kFam32 (Q8_0 Q4_0 Q4_1 Q5_0 Q5_1 Q8_K): 32 consecutive weights, one group
//   kFamK4 (Q4_K Q5_K): 16 bytes of qs = 2 groups of 16 (low / high nibbles),
//                       8 units per super-block
//   kFamK6 (Q6_K Q2_K Q3_K): 8 consecutive l of one half = 4 groups of 8,
//                       8 units per super-block
// A unit holds G groups of GL codes; group g has one scale a[g] and one
// offset coefficient b[g] so that  w = a[g] * code + b[g]  (algebraically; the
// bit-exact dequant kernel applies the reference's own rounding sequence).
//
// Loads: Q4_K / Q5_K units are 16-byte aligned (144 = 9 * 16, 176 = 11 * 16)
// and use dwordx4 loads; Q4_1 (20 B), Q5_1 (24 B) and Q2_K (84 B) blocks are
// 4-byte aligned.  Q8_0 (34 B), Q4_0 (18 B), Q5_0 (22 B), Q8_K (258 B), Q3_K
// (110 B) and Q6_K (210 B) fields sit at even but not always 4-aligned
// offsets; they are read with dword loads from the 4-aligned address at or
// below the field, and re-aligned with v_alignbyte.  Each dword loaded
// contains at least one byte of the field it serves, so no load touches a
// dword that lies wholly outside the weight buffer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace draco {

enum : int {
  kQ4_0 = 2,
  kQ4_1 = 3,
  kQ5_0 = 6,
  kQ5_1 = 7,
  kQ8_0 = 8,
  kQ2_K = 10,
  kQ3_K = 11,
  kQ4_K = 12,
  kQ5_K = 13,
  kQ6_K = 14,
  kQ8_K = 15,
};

enum : int { kFam32 = 0, kFamK4 = 1, kFamK6 = 2 };

// QK elements / BYTES bytes per block, UPB units per block, G groups of GL
// codes per unit, FAM position family, OFF: w = a*code + b has an offset term
// (false: b = 0, signed int8 codes).
template <int QT> struct Fmt;
template <> struct Fmt<kQ8_0> { static constexpr int QK = 32,  BYTES = 34,  UPB = 1, G = 1, GL = 32, FAM = kFam32; static constexpr bool OFF = false; };
template <> struct Fmt<kQ4_0> { static constexpr int QK = 32,  BYTES = 18,  UPB = 1, G = 1, GL = 32, FAM = kFam32; static constexpr bool OFF = true; };
template <> struct Fmt<kQ4_1> { static constexpr int QK = 32,  BYTES = 20,  UPB = 1, G = 1, GL = 32, FAM = kFam32; static constexpr bool OFF = true; };
template <> struct Fmt<kQ5_0> { static constexpr int QK = 32,  BYTES = 22,  UPB = 1, G = 1, GL = 32, FAM = kFam32; static constexpr bool OFF = true; };
template <> struct Fmt<kQ5_1> { static constexpr int QK = 32,  BYTES = 24,  UPB = 1, G = 1, GL = 32, FAM = kFam32; static constexpr bool OFF = true; };
template <> struct Fmt<kQ8_K> { static constexpr int QK = 256, BYTES = 258, UPB = 8, G = 1, GL = 32, FAM = kFam32; static constexpr bool OFF = false; };
template <> struct Fmt<kQ4_K> { static constexpr int QK = 256, BYTES = 144, UPB = 8, G = 2, GL = 16, FAM = kFamK4; static constexpr bool OFF = true; };
template <> struct Fmt<kQ5_K> { static constexpr int QK = 256, BYTES = 176, UPB = 8, G = 2, GL = 16, FAM = kFamK4; static constexpr bool OFF = true; };
template <> struct Fmt<kQ2_K> { static constexpr int QK = 256, BYTES = 84,  UPB = 8, G = 4, GL = 8,  FAM = kFamK6; static constexpr bool OFF = true; };
template <> struct Fmt<kQ3_K> { static constexpr int QK = 256, BYTES = 110, UPB = 8, G = 4, GL = 8,  FAM = kFamK6; static constexpr bool OFF = true; };
template <> struct Fmt<kQ6_K> { static constexpr int QK = 256, BYTES = 210, UPB = 8, G = 4, GL = 8,  FAM = kFamK6; static constexpr bool OFF = true; };

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

// ---------------------------------------------------------------------------
// Byte loaders.  load_unit reads a unit through one of these:
//   GlobalLoader  flat pointer + 64-bit offset (any row layout)
//   BufferLoader  buffer resource (base, byte size) + a wave-uniform offset in
//                 an SGPR (soffset) + a per-lane offset (voffset): no vector
//                 address arithmetic, and reads past num_records return 0
//                 instead of faulting.  Offsets are 32-bit (tensors < 2 GiB).
// ---------------------------------------------------------------------------
struct GlobalLoader {
  const uint8_t* base;
  __device__ __forceinline__ uint32_t u32(int64_t off) const {
    return *reinterpret_cast<const uint32_t*>(base + off);
  }
  __device__ __forceinline__ uint4 u128(int64_t off) const { return *reinterpret_cast<const uint4*>(base + off); }
};

// gfx9-family buffer descriptor word 3 (raw buffer, 32-bit data format)
constexpr int kBufferRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kBufferRsrcWord3);
}

struct BufferLoader {
  __amdgpu_buffer_rsrc_t rsrc;
  int soff;  // wave-uniform byte offset (multiple of 4)
  __device__ __forceinline__ uint32_t u32(int64_t off) const {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)off, soff, 0);
  }
  __device__ __forceinline__ uint4 u128(int64_t off) const {
    typedef int v4i __attribute__((ext_vector_type(4)));
    const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off, soff, 0);
    return uint4{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
  }
};

// ---------------------------------------------------------------------------
// Raw unit payloads (what a lane keeps in registers for one unit)
// ---------------------------------------------------------------------------
template <int QT> struct Raw;

// Q8_0: d + 32 signed codes (8 dwords)
template <> struct Raw<kQ8_0> { uint32_t d; uint32_t q[8]; };
// Q4_0: d + 16 bytes of nibbles
template <> struct Raw<kQ4_0> { uint32_t d; uint32_t q[4]; };
// Q4_K: 16-byte block head (d, dmin, scales) + 16 bytes of qs
template <> struct Raw<kQ4_K> { uint4 head; uint4 qs; };
// Q6_K: 8 bytes of ql (low half), 8 of ql (+32), 8 of qh, 8 of scales, d
template <> struct Raw<kQ6_K> { uint32_t qla[2], qlb[2], qh[2], sc[2]; uint32_t d; };
// Q4_1: d | m<<16, 16 bytes of nibbles
template <> struct Raw<kQ4_1> { uint32_t dm; uint32_t q[4]; };
// Q5_0: d, the 32 fifth bits, 16 bytes of nibbles
template <> struct Raw<kQ5_0> { uint32_t d; uint32_t qh; uint32_t q[4]; };
// Q5_1: d | m<<16, the 32 fifth bits, 16 bytes of nibbles
template <> struct Raw<kQ5_1> { uint32_t dm; uint32_t qh; uint32_t q[4]; };
// Q8_K: d + 32 signed codes (8 dwords)
template <> struct Raw<kQ8_K> { uint32_t d; uint32_t q[8]; };
// Q5_K: 16-byte block head (d, dmin, scales), 16 bytes of qh, 16 bytes of qs
template <> struct Raw<kQ5_K> { uint4 head; uint4 qs; uint4 qh; };
// Q2_K: d | dmin<<16, 8 bytes of qs, the 8 scale bytes of the unit's half
template <> struct Raw<kQ2_K> { uint32_t dm; uint32_t qs[2]; uint32_t sc[2]; };
// Q3_K: 8 bytes of qs, 8 of hmask, the 12 scale bytes, d
template <> struct Raw<kQ3_K> { uint32_t qs[2], hm[2], s12[3]; uint32_t d; };

// Byte offset of the block that holds unit `u` of a row starting at `row_off`.
template <int QT>
__device__ __forceinline__ int64_t unit_block_off(int64_t row_off, int u) {
  return row_off + (int64_t)(u / Fmt<QT>::UPB) * Fmt<QT>::BYTES;
}

// 8 bytes at an even offset `o` (see ld8_even) through a loader.
template <class L>
__device__ __forceinline__ void ld8_even_l(const L& ld, int64_t o, uint32_t& w0, uint32_t& w1) {
  const int64_t p = o & ~int64_t(3);
  const uint32_t a = ld.u32(p), b = ld.u32(p + 4);
  const uint32_t c = ld.u32((o + 7) & ~int64_t(3));
  const uint32_t sh = (uint32_t)o & 3u;
  w0 = __builtin_amdgcn_alignbyte(b, a, sh);
  w1 = __builtin_amdgcn_alignbyte(c, b, sh);
}

template <class L>
__device__ __forceinline__ uint32_t ld16_even_l(const L& ld, int64_t o) {
  const uint32_t w = ld.u32(o & ~int64_t(3));
  return (o & 2) ? (w >> 16) : (w & 0xFFFFu);
}

// 12 bytes at an even offset `o`.
template <class L>
__device__ __forceinline__ void ld12_even_l(const L& ld, int64_t o, uint32_t (&w)[3]) {
  const int64_t p = o & ~int64_t(3);
  const uint32_t a = ld.u32(p), b = ld.u32(p + 4), c = ld.u32(p + 8);
  const uint32_t e = ld.u32((o + 11) & ~int64_t(3));
  const uint32_t sh = (uint32_t)o & 3u;
  w[0] = __builtin_amdgcn_alignbyte(b, a, sh);
  w[1] = __builtin_amdgcn_alignbyte(c, b, sh);
  w[2] = __builtin_amdgcn_alignbyte(e, c, sh);
}

// 32 bytes at an even offset `o` (8 dwords).
template <class L>
__device__ __forceinline__ void ld32_even_l(const L& ld, int64_t o, uint32_t (&q)[8]) {
  const int64_t p = o & ~int64_t(3);
  uint32_t v[9];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = ld.u32(p + 4 * i);
  v[8] = ld.u32((o + 31) & ~int64_t(3));
  const uint32_t sh = (uint32_t)o & 3u;
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], sh);
}

// Unit `u` of the row at byte `row_off`.  Offsets are relative to the
// loader's base, which must be 4-byte aligned.
template <int QT, bool DL, class L>
__device__ __forceinline__ Raw<QT> load_unit_l(const L& ld, int64_t row_off, int u) {
  Raw<QT> r;
  if constexpr (QT == kQ8_0 || QT == kQ4_0) {
    constexpr int NB = QT == kQ8_0 ? 34 : 18, NW = QT == kQ8_0 ? 9 : 5, NQ = QT == kQ8_0 ? 8 : 4;
    const int64_t o = row_off + (int64_t)u * NB;
    const int64_t p = o & ~int64_t(3);
    uint32_t v[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) v[i] = ld.u32(p + 4 * i);
    const bool odd = (o & 2) != 0;
    r.d = odd ? (v[0] >> 16) : (v[0] & 0xFFFFu);
#pragma unroll
    for (int i = 0; i < NQ; ++i) r.q[i] = odd ? v[i + 1] : __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);
  } else if constexpr (QT == kQ4_1 || QT == kQ5_1) {
    // 20 / 24-byte blocks: always 4-byte aligned
    const int64_t o = row_off + (int64_t)u * Fmt<QT>::BYTES;
    if constexpr (QT == kQ4_1) {
      r.dm = ld.u32(o);
#pragma unroll
      for (int i = 0; i < 4; ++i) r.q[i] = ld.u32(o + 4 + 4 * i);
    } else {
      r.dm = ld.u32(o);
      r.qh = ld.u32(o + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) r.q[i] = ld.u32(o + 8 + 4 * i);
    }
  } else if constexpr (QT == kQ5_0) {
    // 22-byte block at an even offset: six dwords, re-aligned to the block
    const int64_t o = row_off + (int64_t)u * 22;
    const int64_t p = o & ~int64_t(3);
    uint32_t v[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) v[i] = ld.u32(p + 4 * i);
    const uint32_t sh = (uint32_t)o & 3u;
    uint32_t a[6];  // block bytes 4i .. 4i+3 (a[5]: bytes 20, 21 in the low half)
#pragma unroll
    for (int i = 0; i < 5; ++i) a[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], sh);
    a[5] = v[5] >> (8 * sh);
    r.d = a[0] & 0xFFFFu;
    r.qh = __builtin_amdgcn_alignbyte(a[1], a[0], 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.q[i] = __builtin_amdgcn_alignbyte(a[i + 2], a[i + 1], 2);
  } else if constexpr (QT == kQ8_K) {
    const int64_t b = unit_block_off<QT>(row_off, u);
    r.d = ld16_even_l(ld, b);
    ld32_even_l(ld, b + 2 + 32 * (u & 7), r.q);
  } else if constexpr (QT == kQ4_K || QT == kQ5_K) {
    const int64_t b = unit_block_off<QT>(row_off, u);
    r.head = ld.u128(b);
    if constexpr (QT == kQ4_K) {
      r.qs = ld.u128(b + 16 + 16 * (u & 7));
    } else {
      r.qh = ld.u128(b + 16 + 16 * (u & 1));
      r.qs = ld.u128(b + 48 + 16 * (u & 7));
    }
  } else if constexpr (QT == kQ2_K) {
    // 84-byte blocks: 4-byte aligned; unit s = (half, sub, l0) reads the 8 qs
    // bytes 32*half + 16*sub + l0 .. +8 and the 8 scale bytes of its half
    const int64_t b = unit_block_off<QT>(row_off, u);
    const int s = u & 7, half = s >> 2;
    constexpr int QS = DL ? 16 : 4, SC = DL ? 0 : 68, D = DL ? 80 : 0;
    const int64_t q = b + QS + 32 * half + 8 * (s & 3);
    r.qs[0] = ld.u32(q);
    r.qs[1] = ld.u32(q + 4);
    r.sc[0] = ld.u32(b + SC + 8 * half);
    r.sc[1] = ld.u32(b + SC + 8 * half + 4);
    r.dm = ld.u32(b + D);
  } else if constexpr (QT == kQ3_K) {
    const int64_t b = unit_block_off<QT>(row_off, u);
    const int s = u & 7, half = s >> 2;
    constexpr int QS = DL ? 32 : 14, HM = DL ? 0 : 78, SC = DL ? 96 : 2, D = DL ? 108 : 0;
    ld8_even_l(ld, b + QS + 32 * half + 8 * (s & 3), r.qs[0], r.qs[1]);
    ld8_even_l(ld, b + HM + 8 * (s & 3), r.hm[0], r.hm[1]);
    ld12_even_l(ld, b + SC, r.s12);
    r.d = ld16_even_l(ld, b + D);
  } else {
    const int64_t b = unit_block_off<QT>(row_off, u);
    const int s = u & 7, half = s >> 2, l0 = 8 * (s & 3);
    constexpr int QL = DL ? 0 : 2, QH = DL ? 128 : 130, SC = DL ? 192 : 194, D = DL ? 208 : 0;
    ld8_even_l(ld, b + QL + 64 * half + l0, r.qla[0], r.qla[1]);
    ld8_even_l(ld, b + QL + 64 * half + 32 + l0, r.qlb[0], r.qlb[1]);
    ld8_even_l(ld, b + QH + 32 * half + l0, r.qh[0], r.qh[1]);
    ld8_even_l(ld, b + SC + 8 * half, r.sc[0], r.sc[1]);
    r.d = ld16_even_l(ld, b + D);
  }
  return r;
}

template <int QT, bool DL = false>
__device__ __forceinline__ Raw<QT> load_unit(const uint8_t* __restrict__ w, int64_t row_off, int u) {
  return load_unit_l<QT, DL>(GlobalLoader{w}, row_off, u);
}

// ---------------------------------------------------------------------------
// Element positions: K offset (within the row) of element i of group g of unit u
// ---------------------------------------------------------------------------
template <int QT>
__device__ __forceinline__ int group_pos(int u, int g) {
  if constexpr (Fmt<QT>::FAM == kFam32) {
    return 32 * u;  // one group of 32 contiguous elements
  } else if constexpr (Fmt<QT>::FAM == kFamK4) {
    const int c = u & 7;
    return 256 * (u >> 3) + 64 * (c >> 1) + 16 * (c & 1) + 32 * g;
  } else {
    const int s = u & 7;
    return 256 * (u >> 3) + 128 * (s >> 2) + 32 * g + 8 * (s & 3);
  }
}

// ---------------------------------------------------------------------------
// Code extraction: 4 codes per dword, one code per byte (unsigned 0..63, or
// signed int8 for Q8_0), in element order of the group.
// ---------------------------------------------------------------------------

// Q4_K / Q4_0: dword j of qs -> low nibbles (group 0 / first 16) and high nibbles.
__device__ __forceinline__ uint32_t nib_lo(uint32_t v) { return v & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t nib_hi(uint32_t v) { return (v >> 4) & 0x0F0F0F0Fu; }

// Q6_K: group t codes for 4 consecutive l from (ql_a, ql_b, qh) dwords.
__device__ __forceinline__ uint32_t q6_codes(int t, uint32_t a, uint32_t b, uint32_t h) {
  switch (t) {
    case 0: return (a & 0x0F0F0F0Fu) | ((h & 0x03030303u) << 4);
    case 1: return (b & 0x0F0F0F0Fu) | ((h & 0x0C0C0C0Cu) << 2);
    case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
    default: return ((b >> 4) & 0x0F0F0F0Fu) | ((h & 0xC0C0C0C0u) >> 2);
  }
}

// Byte i of v as float; the compiler selects v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ float ubyte_f(uint32_t v, int i) { return (float)((v >> (8 * i)) & 0xFFu); }

__device__ __forceinline__ float sbyte_f(uint32_t v, int i) {
  return (float)(int32_t)(int8_t)((v >> (8 * i)) & 0xFFu);
}

// Q4_K 6-bit scale / min of sub-block j (0..7) from the 12 scale bytes held in
// head.y (bytes 0-3), head.z (bytes 4-7), head.w (bytes 8-11);
// same unpacking as the reference _scale_min (draco/format/gguf.py:436-442).
__device__ __forceinline__ void q4k_scale_min(const uint4& head, int j, uint32_t& sc, uint32_t& m) {
  const uint32_t s0 = head.y, s1 = head.z, s2 = head.w;
  if (j < 4) {
    sc = (s0 >> (8 * j)) & 63u;
    m = (s1 >> (8 * j)) & 63u;
  } else {
    const int k = j - 4;
    sc = ((s2 >> (8 * k)) & 0x0Fu) | (((s0 >> (8 * k + 6)) & 3u) << 4);
    m = ((s2 >> (8 * k + 4)) & 0x0Fu) | (((s1 >> (8 * k + 6)) & 3u) << 4);
  }
}

}  // namespace draco
