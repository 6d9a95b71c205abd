// Bit-exact GGUF block dequantization to float32 for gfx950.
//
// Replaces the reference's _dequantize (draco/format/gguf.py:272-497) for
// Q8_0 (:300-303), Q8_K (:305-308), Q4_0 (:310-316), Q4_1 (:318-324),
// Q5_0 / Q5_1 (:326-353), Q2_K (:355-374), Q3_K (:376-423), Q4_K / Q5_K
// (:425-468) and Q6_K (:470-495).  The float32 rounding sequence is the
// reference's:
//   Q8_0  fl(q * d)                 Q4_0  fl((q - 8) * d)
//   Q4_K  fl(fl(fl(d*sc) * q) - fl(dmin*m))
//   Q6_K  fl(fl(d*sc) * (q - 32))
// so this translation unit is compiled with -ffp-contract=off and each kernel
// body also disables contraction: an FMA would skip one of the roundings.
// Q4_1 / Q5_1 / Q2_K / Q5_K compute a*code + b with an explicit fmaf, where a
// and b are exact float32 products of the block's float16 and integer scales:
// the reference rounds that same exact value once (Q4_1 / Q5_1 add m to an
// exact product in float32; Q2_K / Q5_K form it in float64 and round it to
// float32 on the way to the kernel), and so does the FMA.  Q5_0 / Q8_K / Q3_K
// are exact products (code - c) * scale, as in the reference.
//
// One thread decodes one 32-weight unit (see gguf_common.h) and writes it with
// 16-byte stores; the kernel is bound by the float32 write stream (~7x the
// packed read for Q4_K).
#include "gemv_core.h"
#include "draco_internal.h"

namespace draco {

// 16-byte store of four outputs; NaN in place of all four when `bad`.
__device__ __forceinline__ void st4(float* p, float a, float b, float c, float d, bool bad) {
  const float nan = __builtin_nanf("");
  *reinterpret_cast<float4*>(p) = bad ? make_float4(nan, nan, nan, nan) : make_float4(a, b, c, d);
}

// Output row `row` holds weight row ids[row] (ids != NULL: the embedding
// gather; an id outside [0, n_src_rows) gives a NaN row and reads row 0) or
// weight row `row`.
template <int QT, bool DL>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                      int64_t n_units, int units_per_row, int64_t row_bytes,
                                                      int64_t k, const int32_t* __restrict__ ids,
                                                      int64_t n_src_rows) {
#pragma clang fp contract(off)
  const int64_t gu = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gu >= n_units) return;
  const int64_t row = gu / units_per_row;
  const int u = (int)(gu - row * units_per_row);
  int64_t src = row;
  bool bad = false;
  if (ids) {
    src = ids[row];
    bad = src < 0 || src >= n_src_rows;
    src = bad ? 0 : src;
  }
  const Raw<QT> r = load_unit<QT, DL>(w, src * row_bytes, u);
  float* o = out + row * k;

  if constexpr (QT == kQ8_0) {
    const float d = f16_bits_to_f32(r.d);
    float* p = o + group_pos<QT>(u, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      st4(p + 4 * j, sbyte_f(r.q[j], 0) * d, sbyte_f(r.q[j], 1) * d, sbyte_f(r.q[j], 2) * d,
          sbyte_f(r.q[j], 3) * d, bad);
  } else if constexpr (QT == kQ4_0) {
    const float d = f16_bits_to_f32(r.d);
    float* p = o + group_pos<QT>(u, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = nib_lo(r.q[j]), hi = nib_hi(r.q[j]);
      float v[4], h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = (float)((int)((lo >> (8 * i)) & 0xFFu) - 8) * d;
        h[i] = (float)((int)((hi >> (8 * i)) & 0xFFu) - 8) * d;
      }
      st4(p + 4 * j, v[0], v[1], v[2], v[3], bad);
      st4(p + 16 + 4 * j, h[0], h[1], h[2], h[3], bad);
    }
  } else if constexpr (QT == kQ4_K) {
    const float d = f16_bits_to_f32(r.head.x), dmin = f16_bits_to_f32(r.head.x >> 16);
    const int j0 = 2 * ((u & 7) >> 1);
    const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      uint32_t sc, mn;
      q4k_scale_min(r.head, j0 + g, sc, mn);
      const float d1 = d * (float)sc;
      const float m1 = dmin * (float)mn;
      float* p = o + group_pos<QT>(u, g);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = g == 0 ? nib_lo(q[j]) : nib_hi(q[j]);
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float prod = d1 * ubyte_f(c, i);
          v[i] = prod - m1;
        }
        st4(p + 4 * j, v[0], v[1], v[2], v[3], bad);
      }
    }
  } else if constexpr (QT != kQ6_K) {
    // Q4_1 Q5_1 Q2_K Q5_K: w = fma(a, code, b), one rounding.  Q8_K Q5_0 Q3_K
    // (no separate offset): w = a * (code - c), exact, which also keeps the
    // reference's sign of zero (-0 for a zero code times a negative scale;
    // an FMA whose two terms cancel gives +0).
    constexpr int G = Fmt<QT>::G, GL = Fmt<QT>::GL;
    constexpr bool SYM = QT == kQ8_K || QT == kQ5_0 || QT == kQ3_K;
    constexpr float C = QT == kQ5_0 ? 16.f : (QT == kQ3_K ? 4.f : 0.f);
    float a[G], b[G];
    unit_coeffs<QT>(r, u, a, b);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float* p = o + group_pos<QT>(u, g);
#pragma unroll
      for (int j = 0; j < GL / 4; ++j) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float c = unit_code<QT>(r, g, 4 * j + i, u);
          v[i] = SYM ? (c - C) * a[g] : fmaf(a[g], c, b[g]);
        }
        st4(p + 4 * j, v[0], v[1], v[2], v[3], bad);
      }
    }
  } else {  // Q6_K
    const float d = f16_bits_to_f32(r.d);
    const int l16 = ((u & 7) & 3) >> 1;  // l0 / 16
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = l16 + 2 * t;
      const uint32_t scw = j < 4 ? r.sc[0] : r.sc[1];
      const float dl = d * sbyte_f(scw, j & 3);
      float* p = o + group_pos<QT>(u, t);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t c = q6_codes(t, r.qla[h], r.qlb[h], r.qh[h]);
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = dl * (float)((int)((c >> (8 * i)) & 0xFFu) - 32);
        st4(p + 4 * h, v[0], v[1], v[2], v[3], bad);
      }
    }
  }
}

template <int QT, bool DL>
static int launch_dequant(const uint8_t* w, float* out, int64_t n_rows, int64_t k, const int32_t* ids,
                          int64_t n_src_rows, hipStream_t s) {
  const int units_per_row = (int)(k / 32);
  const int64_t row_bytes = (k / Fmt<QT>::QK) * Fmt<QT>::BYTES;
  const int64_t n_units = n_rows * units_per_row;
  const int64_t blocks = (n_units + 255) / 256;
  hipLaunchKernelGGL((dequant_kernel<QT, DL>), dim3((unsigned)blocks), dim3(256), 0, s, w, out, n_units,
                     units_per_row, row_bytes, k, ids, n_src_rows);
  return check_launch("dequant");
}

int dequant_dispatch(int qtype, bool d_last, const void* w, float* out, int64_t n_rows, int64_t k, hipStream_t s) {
  return dequant_rows_dispatch(qtype, d_last, w, nullptr, n_rows, out, n_rows, k, s);
}

int dequant_rows_dispatch(int qtype, bool d_last, const void* w, const int32_t* ids, int64_t n_src_rows, float* out,
                          int64_t n_rows, int64_t k, hipStream_t s) {
  const uint8_t* p = static_cast<const uint8_t*>(w);
  switch (qtype) {
    case kQ8_0: return launch_dequant<kQ8_0, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ4_0: return launch_dequant<kQ4_0, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ4_1: return launch_dequant<kQ4_1, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ5_0: return launch_dequant<kQ5_0, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ5_1: return launch_dequant<kQ5_1, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ8_K: return launch_dequant<kQ8_K, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ4_K: return launch_dequant<kQ4_K, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ5_K: return launch_dequant<kQ5_K, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ2_K:
      return d_last ? launch_dequant<kQ2_K, true>(p, out, n_rows, k, ids, n_src_rows, s)
                    : launch_dequant<kQ2_K, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ3_K:
      return d_last ? launch_dequant<kQ3_K, true>(p, out, n_rows, k, ids, n_src_rows, s)
                    : launch_dequant<kQ3_K, false>(p, out, n_rows, k, ids, n_src_rows, s);
    case kQ6_K:
      return d_last ? launch_dequant<kQ6_K, true>(p, out, n_rows, k, ids, n_src_rows, s)
                    : launch_dequant<kQ6_K, false>(p, out, n_rows, k, ids, n_src_rows, s);
    default: return set_error(DRACO_EINVAL_QTYPE, "unsupported ggml type %d", qtype);
  }
}

}  // namespace draco
