// Prefill GEMM for Q4_K weights on the f16 matrix cores (gfx950).
//
//   y[m, n] = sum_k x[m, k] W[n, k],  W[n, k] = d sc_j q_k - dmin m_j
//
// for a Q4_K super-block (d, dmin f16; sub-block j of 32 weights with 6-bit
// scale sc_j and min m_j; 4-bit codes q).  Two facts make the matrix cores
// do almost all of the work exactly:
//   * sc_j q_k <= 63 * 15 = 945 is an integer below 2048, exact in f16, so
//     one f16 MFMA chain over a whole super-block (eight v_mfma_f32_16x16x32_f16)
//     gives D1 = sum_k x_k sc_j q_k with exact products, scaled once by d;
//   * the min term is sum_j m_j S_j with S_j the activation sum of sub-block
//     j: one bf16 MFMA per plane with A = S (three bf16 planes, exact to
//     2^-24) and B = m_j (exact), eight of its 32 K positions used, gives
//     D2, scaled once by dmin.
// So y += d D1 - dmin D2 per super-block, two FMAs per output where the
// per-sub-block form needs sixteen.
//
// The activations reach the kernel as f16 plus the sub-block sums, both
// written by gemm_prep_kernel: one workgroup per token row finds the row's
// largest |x| and scales the row by the power of two 2^-t that puts it in
// [2^14, 2^15) (undone on the output through 2^t).  Up or down, so f16 never
// overflows and a row of small values never falls into f16's subnormals: every
// element within 2^-31 of the row's largest is exact in f16 (a bf16 value has 8
// significant bits, f16 keeps them down to 2^-17), and the ones below that
// contribute less than 2^-31 of the row's largest term to any output.
//
// Tiling: a 256-thread workgroup owns BM (64) tokens x 128 weight rows; its
// four waves each own (BM / 2) x 64 outputs as 16 x 16 MFMA tiles.  Per K
// step of 64 (two sub-blocks) the workgroup stages the f16 activation tile and
// the f16 sc q tile in LDS (each thread converts the 16 code bytes of half a
// weight row: one v_perm and one packed f16 FMA per two codes); at a
// super-block's first step it also stages the activation sums and the mins,
// d and dmin.  LDS is double-buffered (step s + 1 is staged while step s
// multiplies, one barrier per step) and the global loads run two steps ahead
// in two register sets.  Measured on MI355X: the f16 16x16x32 MFMA peaks at
// ~1.9 PFLOP/s with two waves per SIMD (1.25 with one), and LDS reads at
// ~340 GB/s per CU, which a 32 x 64 wave tile (48 KB of fragment reads per
// 64-deep step per workgroup) nearly saturates: this kernel is LDS- and
// issue-bound at 15-18 % of the bf16 peak.
#pragma once

#include "draco_internal.h"
#include "gemv_core.h"

namespace draco {

typedef _Float16 gq_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 gq_f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 gq_bf16x8 __attribute__((ext_vector_type(8)));
typedef float gq_f32x4 __attribute__((ext_vector_type(4)));
typedef int gq_v4i __attribute__((ext_vector_type(4)));
typedef int gq_v2i __attribute__((ext_vector_type(2)));

// Workspace of the Q4_K GEMM: f16 activations [M, K], sub-block sums as three
// bf16 planes [3][M][K / 32], per-row power-of-two output scales [M].
struct GemmQ4kWs {
  uint16_t* xh;
  uint16_t* sp;
  float* rsc;
};

inline size_t gemm_q4k_ws_layout(int64_t m, int64_t k, char* base, GemmQ4kWs* ws) {
  auto al = [](size_t v) { return (v + 255) & ~size_t(255); };
  const size_t xh = al((size_t)m * k * 2), sp = al((size_t)3 * m * (k / 32) * 2), rs = al((size_t)m * 4);
  if (ws) {
    ws->xh = reinterpret_cast<uint16_t*>(base);
    ws->sp = reinterpret_cast<uint16_t*>(base + xh);
    ws->rsc = reinterpret_cast<float*>(base + xh + sp);
  }
  return xh + sp + rs;
}

__device__ __forceinline__ uint32_t gq_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// One workgroup per token row: scale, f16 copy, sub-block sums.
__global__ __launch_bounds__(256) void gemm_prep_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                        GemmQ4kWs ws) {
  __shared__ float wmax[4];
  const int m = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)m * K);
  const int chunks = K >> 3, groups = K >> 5;

  float mx = 0.f;
  for (int c = tid; c < chunks; c += 256) {
    const uint4 v = xr[c];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mx = fmaxf(mx, fabsf(__uint_as_float(w[i] << 16)));
      mx = fmaxf(mx, fabsf(__uint_as_float(w[i] & 0xFFFF0000u)));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) wmax[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  // |x| 2^-t in [2^14, 2^15) for every finite nonzero row (f16 tops out at
  // 65504, its normals start at 2^-14); zero and NaN / inf rows pass unscaled.
  // The scaling is an exponent shift (v_ldexp) per element: 2^-t itself can
  // exceed float32's range for rows of subnormal bf16 values
  int t = 0;
  if (mx > 0.f && __builtin_isfinite(mx)) t = ilogbf(mx) - 14;

  // one 16-byte chunk (8 elements) per thread, so the loads and stores of a
  // wave are contiguous; a 32-element group is four neighbouring lanes, whose
  // partial sums meet in two exchanges ((s0 + s1) + (s2 + s3))
  const size_t plane = (size_t)M * groups;
  uint4* const dst = reinterpret_cast<uint4*>(ws.xh + (size_t)m * K);
  for (int c = tid; c < chunks; c += 256) {  // chunks is a multiple of 4: whole groups per pass
    const uint4 v = xr[c];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f0 = ldexpf(__uint_as_float(w[i] << 16), -t), f1 = ldexpf(__uint_as_float(w[i] & 0xFFFF0000u), -t);
      sum += f0;
      sum += f1;
      h[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f0, f1));
    }
    dst[c] = uint4{h[0], h[1], h[2], h[3]};
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if ((c & 3) == 0) {
      const uint32_t hi = gq_bf16_rne(sum);
      const float r1 = sum - __uint_as_float(hi << 16);
      const uint32_t mid = gq_bf16_rne(r1);
      const uint32_t lo = gq_bf16_rne(r1 - __uint_as_float(mid << 16));
      const size_t o = (size_t)m * groups + (c >> 2);
      ws.sp[o] = (uint16_t)hi;
      ws.sp[plane + o] = (uint16_t)mid;
      ws.sp[2 * plane + o] = (uint16_t)lo;
    }
  }
  if (tid == 0) ws.rsc[m] = ldexpf(1.f, t);
}

template <int BM>
__global__ __launch_bounds__(256) void gemm_q4k_kernel(const uint8_t* __restrict__ w, GemmQ4kWs ws,
                                                       const float* __restrict__ bias, float* __restrict__ y, int M,
                                                       int N, int K, int tiles_m) {
  constexpr int BN = 128, BK = 64, LDA = BK + 8;  // f16 per LDS row (144 B: conflict-free b128 fragment reads)
  constexpr int WTM = BM / 2, TI = WTM / 16, TJ = 4;
  constexpr int APT = BM * 8 / 256;  // 16-byte activation pieces per thread per step
  constexpr int SPT = (3 * BM + 255) / 256;
  // two LDS buffers per operand: step s + 1 is staged while step s multiplies
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDA];
  __shared__ uint4 Ss[2][3][BM];  // [super-block parity][plane][row]: 8 sub-block sums (bf16)
  __shared__ uint4 Ms[2][BN];     // [parity][weight row]: 8 mins (bf16)
  __shared__ float2 Ds[2][BN];    // [parity][weight row]: d, dmin

  // XCD-aware order: workgroups are dealt to the 8 XCDs round robin; renumber
  // so each XCD gets a contiguous run of tiles (the token tiles of one weight
  // tile share that XCD's L2)
  const int nb = gridDim.x;
  int bid = blockIdx.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  const int tm = bid % tiles_m, tn = bid / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int sbs = K >> 8, groups = K >> 5, steps = K / BK;
  const uint32_t row_bytes = (uint32_t)sbs * 144u;

  // weight-tile role: row br of the tile, half bh of its 32 code bytes per step
  const int br = tid >> 1, bh = tid & 1;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w, (uint32_t)N * row_bytes);
  const int wrow = (int)((uint32_t)min(n0 + br, N - 1) * row_bytes);

  // global data of one step, in two register sets (steps of either parity)
  struct Set {
    uint4 a[APT];
    uint4 b, h;
    uint4 s[SPT];
  } set[2];
  auto load = [&](Set& st, int ks) {
    const int k0 = ks * BK, sb = ks >> 2, p = ks & 3;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int idx = tid + 256 * i;
      const int row = idx >> 3, c8 = idx & 7;
      st.a[i] = m0 + row < M ? *reinterpret_cast<const uint4*>(ws.xh + (size_t)(m0 + row) * K + k0 + 8 * c8)
                             : uint4{0u, 0u, 0u, 0u};
    }
    const gq_v4i q = __builtin_amdgcn_raw_buffer_load_b128(wrs, wrow + sb * 144 + 16 + 32 * p + 16 * bh, 0, 0);
    st.b = uint4{(uint32_t)q.x, (uint32_t)q.y, (uint32_t)q.z, (uint32_t)q.w};
    if (p == 0) {
      const gq_v4i hd = __builtin_amdgcn_raw_buffer_load_b128(wrs, wrow + sb * 144, 0, 0);
      st.h = uint4{(uint32_t)hd.x, (uint32_t)hd.y, (uint32_t)hd.z, (uint32_t)hd.w};
#pragma unroll
      for (int i = 0; i < SPT; ++i) {
        const int idx = tid + 256 * i;
        const int pl = idx / BM, row = idx - pl * BM;
        st.s[i] = (idx < 3 * BM && m0 + row < M)
                      ? *reinterpret_cast<const uint4*>(ws.sp + (size_t)pl * M * groups + (size_t)(m0 + row) * groups +
                                                        8 * sb)
                      : uint4{0u, 0u, 0u, 0u};
      }
    }
  };

  uint32_t sc_lo = 0, sc_hi = 0;  // the staged row's eight 6-bit scales of the current super-block
  // LDS image of step ks (buffer ks & 1) from a register set
  auto stage = [&](const Set& st, int ks) {
    const int buf = ks & 1, sb = ks >> 2, p = ks & 3;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int idx = tid + 256 * i;
      *reinterpret_cast<uint4*>(&As[buf][(idx >> 3) * LDA + 8 * (idx & 7)]) = st.a[i];
    }
    if (p == 0) {
      const uint32_t s0 = st.h.y, s1 = st.h.z, s2 = st.h.w;
      sc_lo = s0 & 0x3F3F3F3Fu;
      sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
      if (bh == 0) {
        const uint32_t m_lo = s1 & 0x3F3F3F3Fu;
        const uint32_t m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
        uint32_t mb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t mw = j < 2 ? m_lo : m_hi;
          const int sh = 16 * (j & 1);
          mb[j] = gq_bf16_rne((float)((mw >> sh) & 0xFFu)) | (gq_bf16_rne((float)((mw >> (sh + 8)) & 0xFFu)) << 16);
        }
        Ms[sb & 1][br] = uint4{mb[0], mb[1], mb[2], mb[3]};
        Ds[sb & 1][br] = float2{f16_bits_to_f32(st.h.x), f16_bits_to_f32(st.h.x >> 16)};
      }
#pragma unroll
      for (int i = 0; i < SPT; ++i) {
        const int idx = tid + 256 * i;
        if (idx < 3 * BM) Ss[sb & 1][idx / BM][idx % BM] = st.s[i];
      }
    }
    // codes of sub-blocks 2p (low nibbles) and 2p + 1 (high nibbles), times their scales, as f16
    const uint32_t scw = p < 2 ? sc_lo : sc_hi;
    const int sh = 16 * (p & 1);
    const _Float16 s_a = (_Float16)(float)((scw >> sh) & 0xFFu), s_b = (_Float16)(float)((scw >> (sh + 8)) & 0xFFu);
    const gq_f16x2 sa2 = {s_a, s_a}, sb2 = {s_b, s_b};
    const gq_f16x2 ca2 = {(_Float16)(-1024.f) * s_a, (_Float16)(-1024.f) * s_a};
    const gq_f16x2 cb2 = {(_Float16)(-1024.f) * s_b, (_Float16)(-1024.f) * s_b};
    const uint32_t qw[4] = {st.b.x, st.b.y, st.b.z, st.b.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t cl = qw[i] & 0x0F0F0F0Fu, chh = (qw[i] >> 4) & 0x0F0F0F0Fu;
      // f16 bits 0x64qq = 1024 + q; fma(1024 + q, s, -1024 s) = s q exactly
      lo[2 * i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
          __builtin_bit_cast(gq_f16x2, __builtin_amdgcn_perm(0x64646464u, cl, 0x04010400u)), sa2, ca2));
      lo[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
          __builtin_bit_cast(gq_f16x2, __builtin_amdgcn_perm(0x64646464u, cl, 0x04030402u)), sa2, ca2));
      hi[2 * i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
          __builtin_bit_cast(gq_f16x2, __builtin_amdgcn_perm(0x64646464u, chh, 0x04010400u)), sb2, cb2));
      hi[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
          __builtin_bit_cast(gq_f16x2, __builtin_amdgcn_perm(0x64646464u, chh, 0x04030402u)), sb2, cb2));
    }
    uint16_t* brow = &Bs[buf][br * LDA];
    *reinterpret_cast<uint4*>(brow + 16 * bh) = uint4{lo[0], lo[1], lo[2], lo[3]};
    *reinterpret_cast<uint4*>(brow + 16 * bh + 8) = uint4{lo[4], lo[5], lo[6], lo[7]};
    *reinterpret_cast<uint4*>(brow + 32 + 16 * bh) = uint4{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<uint4*>(brow + 32 + 16 * bh + 8) = uint4{hi[4], hi[5], hi[6], hi[7]};
  };

  gq_f32x4 acc[TI][TJ], d1[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      acc[i][j] = gq_f32x4{0.f, 0.f, 0.f, 0.f};
      d1[i][j] = gq_f32x4{0.f, 0.f, 0.f, 0.f};
    }
  const int fr = lane & 15, fk = 8 * (lane >> 4);
  const uint4 z = {0u, 0u, 0u, 0u};

  load(set[0], 0);
  if (steps > 1) load(set[1], 1);
  stage(set[0], 0);
  if (steps > 2) load(set[0], 2);
  __syncthreads();
  for (int sb = 0; sb < sbs; ++sb) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int ks = 4 * sb + p;
      const int buf = p & 1;
      // stage the next step into the other buffer, then refill its register set
      if (ks + 1 < steps) {
        stage(set[buf ^ 1], ks + 1);
        if (ks + 3 < steps) load(set[buf ^ 1], ks + 3);
      }
      // multiply step ks
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        gq_f16x8 a[TI], b[TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i)
          a[i] = *reinterpret_cast<const gq_f16x8*>(&As[buf][(wm * WTM + 16 * i + fr) * LDA + 32 * gi + fk]);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          b[j] = *reinterpret_cast<const gq_f16x8*>(&Bs[buf][(wn * 64 + 16 * j + fr) * LDA + 32 * gi + fk]);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            d1[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], d1[i][j], 0, 0, 0);
      }
      if (p == 3) {
        // super-block end: min term on the bf16 matrix cores, then y += d D1 - dmin D2
        const int sp = sb & 1;
        gq_bf16x8 bm[TJ];
        float dd[TJ], dm[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          const int col = wn * 64 + 16 * j + fr;
          bm[j] = __builtin_bit_cast(gq_bf16x8, lane < 16 ? Ms[sp][col] : z);
          const float2 dv = Ds[sp][col];
          dd[j] = dv.x;
          dm[j] = dv.y;
        }
#pragma unroll
        for (int i = 0; i < TI; ++i) {
          gq_bf16x8 sa[3];
#pragma unroll
          for (int pl = 0; pl < 3; ++pl)
            sa[pl] = __builtin_bit_cast(gq_bf16x8, lane < 16 ? Ss[sp][pl][wm * WTM + 16 * i + fr] : z);
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            gq_f32x4 d2 = {0.f, 0.f, 0.f, 0.f};
            d2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa[2], bm[j], d2, 0, 0, 0);
            d2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa[1], bm[j], d2, 0, 0, 0);
            d2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa[0], bm[j], d2, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              acc[i][j][v] = fmaf(dd[j], d1[i][j][v], acc[i][j][v]);
              acc[i][j][v] = fmaf(-dm[j], d2[v], acc[i][j][v]);
            }
            d1[i][j] = gq_f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
      __syncthreads();
    }
  }

  // D layout: lane l holds rows 4 (l / 16) + v, column l % 16 of a 16 x 16 tile
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = m0 + wm * WTM + 16 * i + 4 * (lane >> 4) + v;
      if (m >= M) continue;
      const float rs = ws.rsc[m];
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int n = n0 + wn * 64 + 16 * j + (lane & 15);
        if (n < N) y[(size_t)m * N + n] = acc[i][j][v] * rs + (bias ? bias[n] : 0.f);
      }
    }
}

// Launches the activation prep and the GEMM; `workspace` holds
// gemm_q4k_ws_layout(m, k) bytes.
inline int launch_gemm_q4k(const void* w, const void* x, const float* bias, float* y, int m, int n, int k,
                           void* workspace, hipStream_t s) {
  GemmQ4kWs ws;
  gemm_q4k_ws_layout(m, k, static_cast<char*>(workspace), &ws);
  hipLaunchKernelGGL(gemm_prep_kernel, dim3((unsigned)m), dim3(256), 0, s, static_cast<const uint16_t*>(x), m, k, ws);
  if (int rc = check_launch("gemm_prep")) return rc;
  // 64-token tiles: two workgroups per CU (LDS and registers allow it), and
  // measured faster than 128-token tiles at M = 512 and 2048
  const int tiles_n = (n + 127) / 128, tiles_m = (m + 63) / 64;
  hipLaunchKernelGGL(gemm_q4k_kernel<64>, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, s,
                     static_cast<const uint8_t*>(w), ws, bias, y, m, n, k, tiles_m);
  return check_launch("gemm_q4k");
}

}  // namespace draco
