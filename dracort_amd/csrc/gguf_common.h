// GGUF block geometry and per-lane block decoders for gfx950.
//
// Block layouts follow the reference's table (draco/format/gguf.py:75-87):
//   Q8_0  32 elems,  34 B : f16 d | int8 qs[32]
//   Q4_0  32 elems,  18 B : f16 d | u8 qs[16]  (elem i = low nibble of qs[i], elem 16+i = high nibble)
//   Q4_K 256 elems, 144 B : f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
//   Q6_K 256 elems, 210 B : f16 d | u8 ql[128] | u8 qh[64] | i8 scales[16]   (reference order)
//                           u8 ql[128] | u8 qh[64] | i8 scales[16] | f16 d   (upstream ggml order)
//
// Every kernel here walks a weight row in "units" of 32 weights.  A unit is
// the natural slice one lane decodes from one load group:
//   Q8_0 / Q4_0 : one block                      (1 unit per block)
//   Q4_K        : 16 bytes of qs = 32 nibbles    (8 units per super-block)
//   Q6_K        : 8 consecutive l of one half    (8 units per super-block)
// A unit holds G groups of 32/G codes; group g has one scale a[g] and one
// offset coefficient b[g] so that  w = a[g] * code + b[g]  (algebraically; the
// bit-exact dequant kernel applies the reference's own rounding sequence).
//
// Loads: Q4_K units are 16-byte aligned (144 = 9 * 16) and use dwordx4 loads.
// Q8_0 (34 B), Q4_0 (18 B) and Q6_K (210 B) fields sit at even but not always
// 4-aligned offsets; they are read with dword loads from the 4-aligned address
// at or below the field, and re-aligned with v_alignbyte.  Each dword loaded
// contains at least one byte of the field it serves, so no load touches a
// dword that lies wholly outside the weight buffer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace draco {

enum : int {
  kQ4_0 = 2,
  kQ8_0 = 8,
  kQ4_K = 12,
  kQ6_K = 14,
};

template <int QT> struct Fmt;
template <> struct Fmt<kQ8_0> { static constexpr int QK = 32,  BYTES = 34,  UPB = 1, G = 1, GL = 32; };
template <> struct Fmt<kQ4_0> { static constexpr int QK = 32,  BYTES = 18,  UPB = 1, G = 1, GL = 32; };
template <> struct Fmt<kQ4_K> { static constexpr int QK = 256, BYTES = 144, UPB = 8, G = 2, GL = 16; };
template <> struct Fmt<kQ6_K> { static constexpr int QK = 256, BYTES = 210, UPB = 8, G = 4, GL = 8; };

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
  } else if constexpr (QT == kQ4_K) {
    const int64_t b = unit_block_off<QT>(row_off, u);
    r.head = ld.u128(b);
    r.qs = ld.u128(b + 16 + 16 * (u & 7));
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
  if constexpr (QT == kQ8_0 || QT == kQ4_0) {
    return 32 * u;  // one group of 32 contiguous elements
  } else if constexpr (QT == kQ4_K) {
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
