// Prefill GEMM for Q4_K weights on the 32 x 32 x 16 f16 matrix cores (gfx950).
//
// The same arithmetic as gemm_q4k.h (every product exact: B = sc q in f16,
// <= 945; the activations f16 after the per-row power-of-two normalisation of
// gemm_prep_kernel; per super-block one MFMA chain D1 = sum x sc q scaled once
// by d, and the min term D2 = sum_j m_j S_j from bf16 MFMAs over the three
// bf16 planes of the 32-element sums S, scaled once by dmin), on larger
// tiles:
//   * v_mfma_f32_32x32x16_f16: 32 x 32 outputs per instruction, twice the
//     FLOP per LDS fragment byte of 16 x 16 x 32, and its full rate with one
//     wave per SIMD (measured 2.07 PFLOP/s in a pure-MFMA loop, where the
//     16 x 16 x 32 form needs two waves to pass 1.25);
//   * each wave owns a 64 x 64 output tile (2 x 2 MFMA tiles: two A and two B
//     fragment reads feed four MFMAs per 16-deep slice);
//   * a workgroup of WM x WN waves owns a (64 WM tokens) x (64 WN weight rows)
//     tile, so each converted weight code feeds 64 WM tokens.
// Per K step of 64 (half a super-block's sub-block pairs: sub-blocks 2p and
// 2p + 1 of super-block sb at step 4 sb + p) the workgroup stages the f16
// activation tile and the converted f16 sc q tile in LDS, double-buffered
// with the global loads two steps ahead; at a super-block's first step it
// also stages the sums, the mins and d / dmin.  The output is y = acc * 2^t
// (the row's prep scale) + bias.
#pragma once

#include <algorithm>

#include "draco_internal.h"
#include "gemm_q4k.h"
#include "gemv_core.h"
#include "gemv_stream.h"

namespace draco {

typedef _Float16 g2_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 g2_f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 g2_bf16x8 __attribute__((ext_vector_type(8)));
typedef float g2_f32x16 __attribute__((ext_vector_type(16)));
typedef int g2_v4i __attribute__((ext_vector_type(4)));
typedef int g2_v2i __attribute__((ext_vector_type(2)));

// tid again, as a value the compiler cannot prove equal to tid: offsets used
// once per super-block are recomputed there instead of held in registers
// across the loop (the register budget is spent on the tiles)
__device__ __forceinline__ int g2_fresh(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Split K: with part != nullptr the grid holds `splits` workgroups per output
// tile, split s taking super-blocks [s sbps, (s + 1) sbps) and storing its raw
// sums to part[s][M][N]; gemm_split_reduce_kernel adds them in split order.
// Tail split (tail_s > 1): the first tail_full tiles (whole weight-tile
// columns) run whole, and the rest, the partial last round of a grid that
// does not divide evenly over the CUs, in tail_s parts of K each (raw sums to
// part[s][M][N - n_tail] for columns n_tail .. N - 1, added by the reduce
// launch), so every CU finishes the launch with the same amount of work.
// Each XCD gets tail_full / 8 whole tiles, then its share of the parts.
template <int WM, int WN, int NS = 2>
__global__ __launch_bounds__(WM * WN * 64) void gemm_q4k2_kernel(const uint8_t* __restrict__ w, GemmQ4kWs ws,
                                                                 const float* __restrict__ bias,
                                                                 float* __restrict__ y, int M, int N, int K,
                                                                 int tiles_m, int tiles, int sbps,
                                                                 float* __restrict__ part, int tail_full,
                                                                 int tail_s) {
  constexpr int NT = WM * WN * 64;          // threads
  constexpr int BM = 64 * WM, BN = 64 * WN;  // workgroup tile
  constexpr int BK = 64, LDK = BK + 8;       // f16 per LDS row (144 B)
  constexpr int APT = BM * BK / 8 / NT;      // 16-byte activation pieces per thread per step
  constexpr int BPT = BN * 4 / NT;           // 8-byte code pieces per thread per step (1 or 2)
  constexpr int SPT = (3 * BM + NT - 1) / NT;  // 16-byte sum pieces per thread per super-block
  static_assert(APT >= 1 && BPT >= 1, "tile too small for the workgroup");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];
  __shared__ uint4 Ss[2][3][BM];  // [super-block parity][plane][token]: 8 sub-block sums (bf16)
  __shared__ uint4 Ms[2][BN];     // [parity][weight row]: 8 mins (bf16)
  __shared__ float2 Ds[2][BN];    // [parity][weight row]: d, dmin
  __shared__ uint2 Sc[2][BN];     // [parity][weight row]: the eight 6-bit sub-block scales

  // XCD-aware order: workgroups are dealt to the 8 XCDs round robin; renumber
  // so each XCD gets a contiguous run of tiles (the token tiles of one weight
  // tile share that XCD's L2)
  const int nb = gridDim.x;
  int bid = blockIdx.x;
  int split;
  if (tail_s > 1) {
    // (the launch guarantees tail_full % 8 == 0 and nb % 8 == 0)
    const int xcd = bid & 7, k8 = bid >> 3, full8 = tail_full >> 3;
    if (k8 < full8) {
      bid = xcd * full8 + k8;
      split = -1;
    } else {
      const int h = xcd * ((nb - tail_full) >> 3) + (k8 - full8);
      bid = tail_full + h / tail_s;
      split = h - (h / tail_s) * tail_s;
    }
  } else {
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    split = bid / tiles;
    bid -= split * tiles;
  }
  const int tm = bid % tiles_m, tn = bid / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int sbs = K >> 8, groups = K >> 5;
  const int sb0 = split < 0 ? 0 : split * sbps, sb1 = split < 0 ? sbs : min(sb0 + sbps, sbs), ks0 = 4 * sb0;
  const uint32_t row_bytes = (uint32_t)sbs * 144u;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w, (uint32_t)N * row_bytes);
  // activations and sums through buffer resources: 32-bit offsets, and reads
  // past the end (token rows beyond M) return zero
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(ws.xh, (uint32_t)M * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(ws.sp, 3u * (uint32_t)M * (uint32_t)groups * 2u);

  // global data of one step, in a ring of NS register sets (step s in set s % NS)
  static_assert(NS == 2 || NS == 4, "the ring index must be static in the 4-step super-block loop");
  struct Set {
    uint4 a[APT];
    uint2 b[BPT];
  } set[NS];
  // a super-block's header and sums: one copy (loaded with the super-block's
  // first step, at most NS - 1 steps ahead of its staging, which comes first
  // in every iteration)
  struct SbSet {
    uint4 h;
    uint4 s[SPT];
  } sbset;
  // Every thread issues the same loads at every step, also past the last
  // step and for rows / threads with nothing to fetch: offsets past a
  // buffer's end read zero, and those within it (the next row, a later step)
  // only feed LDS images that are never multiplied.  A fixed load count per
  // step lets each wait leave the newer steps' loads in flight.
  auto load = [&](Set& st, int ks) {
    const int k0 = ks * BK, sb = ks >> 2, p = ks & 3;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int idx = tid + NT * i;
      const int row = idx >> 3, c8 = idx & 7;
      const g2_v4i v = __builtin_amdgcn_raw_buffer_load_b128(
          xrs, (uint32_t)(m0 + row) * (uint32_t)K * 2u + (uint32_t)(k0 + 8 * c8) * 2u, 0, 0);
      st.a[i] = uint4{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int idx = tid + NT * i;
      const int br = idx >> 2, bq = idx & 3;
      const int wrow = (int)((uint32_t)min(n0 + br, N - 1) * row_bytes);
      const g2_v2i q = __builtin_amdgcn_raw_buffer_load_b64(wrs, wrow + sb * 144 + 16 + 32 * p + 8 * bq, 0, 0);
      st.b[i] = uint2{(uint32_t)q.x, (uint32_t)q.y};
    }
    if (p == 0) {
      const int tid = g2_fresh(threadIdx.x);
      {
        const uint32_t off = tid < BN ? (uint32_t)min(n0 + tid, N - 1) * row_bytes + (uint32_t)sb * 144u : 0xFFFFFFF0u;
        const g2_v4i hd = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0);
        sbset.h = uint4{(uint32_t)hd.x, (uint32_t)hd.y, (uint32_t)hd.z, (uint32_t)hd.w};
      }
#pragma unroll
      for (int i = 0; i < SPT; ++i) {
        const int idx = tid + NT * i;
        const int pl = idx / BM, row = idx - pl * BM;
        // rows past M read a neighbouring plane or past the end: they feed
        // only output rows that are never stored
        const uint32_t off = idx < 3 * BM ? ((uint32_t)pl * (uint32_t)M + (uint32_t)(m0 + row)) * (uint32_t)groups * 2u +
                                                (uint32_t)sb * 16u
                                          : 0xFFFFFFF0u;
        const g2_v4i v = __builtin_amdgcn_raw_buffer_load_b128(srs, off, 0, 0);
        sbset.s[i] = uint4{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
      }
    }
  };

  // LDS image of step ks (buffer ks & 1) from a register set
  auto stage = [&](const Set& st, int ks) {
    const int buf = ks & 1, sb = ks >> 2, p = ks & 3, par = sb & 1;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int idx = tid + NT * i;
      *reinterpret_cast<uint4*>(&As[buf][(idx >> 3) * LDK + 8 * (idx & 7)]) = st.a[i];
    }
    if (p == 0) {
      const int tid = g2_fresh(threadIdx.x);
      if (tid < BN) {
        const uint32_t s0 = sbset.h.y, s1 = sbset.h.z, s2 = sbset.h.w;
        const uint32_t sc_lo = s0 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
        const uint32_t m_lo = s1 & 0x3F3F3F3Fu;
        const uint32_t m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
        uint32_t mb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t mw = j < 2 ? m_lo : m_hi;
          const int sh = 16 * (j & 1);
          mb[j] = gq_bf16_rne((float)((mw >> sh) & 0xFFu)) | (gq_bf16_rne((float)((mw >> (sh + 8)) & 0xFFu)) << 16);
        }
        Ms[par][tid] = uint4{mb[0], mb[1], mb[2], mb[3]};
        Ds[par][tid] = float2{f16_bits_to_f32(sbset.h.x), f16_bits_to_f32(sbset.h.x >> 16)};
        Sc[par][tid] = uint2{sc_lo, sc_hi};
      }
#pragma unroll
      for (int i = 0; i < SPT; ++i) {
        const int idx = tid + NT * i;
        if (idx < 3 * BM) Ss[par][idx / BM][idx % BM] = sbset.s[i];
      }
    }
  };
  // codes of sub-blocks 2p (low nibbles) and 2p + 1 (high nibbles) times their
  // scales, as f16, into the LDS B image (after the step's scales are staged)
  auto stage_codes = [&](const Set& st, int ks) {
    const int buf = ks & 1, sb = ks >> 2, p = ks & 3, par = sb & 1;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int idx = tid + NT * i;
      const int br = idx >> 2, bq = idx & 3;
      const uint2 scw2 = Sc[par][br];
      const uint32_t scw = p < 2 ? scw2.x : scw2.y;
      const int sh = 16 * (p & 1);
      const _Float16 s_a = (_Float16)(float)((scw >> sh) & 0xFFu), s_b = (_Float16)(float)((scw >> (sh + 8)) & 0xFFu);
      const g2_f16x2 sa2 = {s_a, s_a}, sb2 = {s_b, s_b};
      const g2_f16x2 ca2 = {(_Float16)(-1024.f) * s_a, (_Float16)(-1024.f) * s_a};
      const g2_f16x2 cb2 = {(_Float16)(-1024.f) * s_b, (_Float16)(-1024.f) * s_b};
      const uint32_t qw[2] = {st.b[i].x, st.b[i].y};
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t cl = qw[e] & 0x0F0F0F0Fu, chh = (qw[e] >> 4) & 0x0F0F0F0Fu;
        // f16 bits 0x64qq = 1024 + q; fma(1024 + q, s, -1024 s) = s q exactly
        lo[2 * e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
            __builtin_bit_cast(g2_f16x2, __builtin_amdgcn_perm(0x64646464u, cl, 0x04010400u)), sa2, ca2));
        lo[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
            __builtin_bit_cast(g2_f16x2, __builtin_amdgcn_perm(0x64646464u, cl, 0x04030402u)), sa2, ca2));
        hi[2 * e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
            __builtin_bit_cast(g2_f16x2, __builtin_amdgcn_perm(0x64646464u, chh, 0x04010400u)), sb2, cb2));
        hi[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
            __builtin_bit_cast(g2_f16x2, __builtin_amdgcn_perm(0x64646464u, chh, 0x04030402u)), sb2, cb2));
      }
      uint16_t* brow = &Bs[buf][br * LDK];
      *reinterpret_cast<uint4*>(brow + 8 * bq) = uint4{lo[0], lo[1], lo[2], lo[3]};
      *reinterpret_cast<uint4*>(brow + 32 + 8 * bq) = uint4{hi[0], hi[1], hi[2], hi[3]};
    }
  };

  g2_f32x16 zero16;
#pragma unroll
  for (int v = 0; v < 16; ++v) zero16[v] = 0.f;
  g2_f32x16 acc[2][2], d1[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16;
  // fragment lane roles: row / column l % 32, k slice 8 (l / 32)
  const int fr = lane & 31, fk = 8 * (lane >> 5);
  const uint4 z = {0u, 0u, 0u, 0u};

#pragma unroll
  for (int i = 0; i < NS; ++i) load(set[i], ks0 + i);
  stage(set[0], ks0);
  __syncthreads();
  stage_codes(set[0], ks0);
  load(set[0], ks0 + NS);
  __syncthreads();
  for (int sb = sb0; sb < sb1; ++sb) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int ks = 4 * sb + p;
      const int buf = p & 1;
      // stage the next step into the other buffer, then refill its register
      // set (after the last step this stages an image nobody reads)
      auto stage_next = [&]() {
        Set& nx = set[(p + 1) % NS];
        stage(nx, ks + 1);
        if (((ks + 1) & 3) == 0) __syncthreads();  // the new super-block's scales before the codes
        stage_codes(nx, ks + 1);
        load(nx, ks + 1 + NS);
      };
      // multiply step ks: four 16-deep slices, 2 x 2 MFMA tiles; the next
      // step is staged after the third, while the matrix cores still work
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk == 3) stage_next();
        g2_f16x8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          a[i] = *reinterpret_cast<const g2_f16x8*>(&As[buf][(wm * 64 + 32 * i + fr) * LDK + 16 * kk + fk]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          b[j] = *reinterpret_cast<const g2_f16x8*>(&Bs[buf][(wn * 64 + 32 * j + fr) * LDK + 16 * kk + fk]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)  // a super-block's chain starts from zero
            d1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], p == 0 && kk == 0 ? zero16 : d1[i][j], 0, 0, 0);
      }
      if (p == 3) {
        // super-block end: min term on the bf16 matrix cores (k positions
        // 0..7 of the 16 carry the eight sub-block sums / mins), then
        // acc += d D1 - dmin D2
        const int par = sb & 1;
        g2_bf16x8 bm[2];
        float dd[2], dm[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = wn * 64 + 32 * j + fr;
          bm[j] = __builtin_bit_cast(g2_bf16x8, lane < 32 ? Ms[par][col] : z);
          const float2 dv = Ds[par][col];
          dd[j] = dv.x;
          dm[j] = dv.y;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          g2_bf16x8 sa[3];
#pragma unroll
          for (int pl = 0; pl < 3; ++pl)
            sa[pl] = __builtin_bit_cast(g2_bf16x8, lane < 32 ? Ss[par][pl][wm * 64 + 32 * i + fr] : z);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            // D1 is consumed first, then its registers hold D2
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(dd[j], d1[i][j][v], acc[i][j][v]);
            d1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(sa[2], bm[j], zero16, 0, 0, 0);
            d1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(sa[1], bm[j], d1[i][j], 0, 0, 0);
            d1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(sa[0], bm[j], d1[i][j], 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(-dm[j], d1[i][j][v], acc[i][j][v]);
          }
        }
      }
      __syncthreads();
    }
  }

  // D layout: lane l, register v holds row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = m0 + wm * 64 + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      if (m >= M) continue;
      if (part && split >= 0) {
        // raw sums: columns nt .. N - 1 (all of them unless tail split)
        const int nt = tail_s > 1 ? (tail_full / tiles_m) * 128 : 0;
        float* pr = part + ((size_t)split * M + m) * (size_t)(N - nt);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + wn * 64 + 32 * j + fr;
          if (n < N) pr[n - nt] = acc[i][j][v];
        }
        continue;
      }
      const float rs = ws.rsc[m];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + 32 * j + fr;
        if (n < N) y[(size_t)m * N + n] = acc[i][j][v] * rs + (bias ? bias[n] : 0.f);
      }
    }
}

// y[m, n] = (sum over s in order of part[s][m][n - nt]) * 2^t_m + bias[n] for
// the columns n >= nt that were split: one thread per output, fixed
// summation order (the result does not depend on which split finished first).
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float* __restrict__ part, int splits, int M,
                                                                int N, int nt, const float* __restrict__ rsc,
                                                                const float* __restrict__ bias,
                                                                float* __restrict__ y) {
  const int ns = N - nt;
  const size_t total = (size_t)M * ns;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int m = (int)(i / (size_t)ns), n = nt + (int)(i - (size_t)m * ns);
  float acc = part[i];
  for (int s = 1; s < splits; ++s) acc += part[(size_t)s * total + i];
  y[(size_t)m * N + n] = acc * rsc[m] + (bias ? bias[n] : 0.f);
}

// Split-K plan of the 256 x 128 tiling for an M x N x K problem: `splits`
// workgroups per output tile so that the grid fills the GPU; 0 when the
// tiling should not be used (gemm_q4k.h's 64-token tiles are faster).
// Measured on MI355X (this tiling vs gemm_q4k.h): 14336 x 4096 at M = 512
// (224 tiles, unsplit) 111 vs 177 us; 4096 x 14336 at M = 512 (64 tiles) 285
// vs 209 us unsplit, 110 us in four splits; M = 64 of 4096 x 14336 in eight
// splits 54 vs 190 us.
struct GemmQ4k2Plan {
  int splits = 0;  // 0: not this kernel; 1: no partial sums (unless tail split)
  int sbps = 0;    // super-blocks per split
  size_t part_bytes = 0;
  // tail split: tiles [0, tail_full) whole, the rest in tail_s parts
  int tail_full = 0, tail_s = 0;
};

// Workspace bytes the split-K partial sums of an M-row problem may need
// beyond gemm_q4k_ws_layout: splits are only planned while the tile count
// times the splits stays within the CU count, so S x N <= 128 x CUs / tiles_m.
// The bound is taken at 256 CUs (MI355X), independent of the device present:
// on a device with more CUs the splits are capped by the space given.
// (The tail split of a grid of whole rounds plus a partial one keeps within
// the same bound: its parts times their columns' tiles stay within the CUs.)
inline size_t gemm_q4k2_part_bound(int64_t m) {
  const int64_t tiles_m = (m + 255) / 256;
  return (size_t)m * 128 * (size_t)(256 / tiles_m) * 4;
}

inline GemmQ4k2Plan gemm_q4k2_plan(int m, int n, int k, size_t part_avail) {
  GemmQ4k2Plan pl;
  if ((int64_t)m * k * 2 >= (int64_t(1) << 31)) return pl;  // 32-bit buffer offsets
  const int64_t tiles = (int64_t)((m + 255) / 256) * ((n + 127) / 128);
  const int64_t cus = device_cus();
  if (tiles * 4 >= cus * 3) {
    pl.splits = 1;
    pl.sbps = k / 256;
    // whole rounds plus a partial one: the partial round's tiles in parts of
    // K, so it takes a fraction of a round (14336 x 4096 at M = 2048: 896
    // tiles = 3 rounds + 128 tiles in two parts each).  The split tiles must
    // be whole weight-tile columns, and the whole tiles and the parts divide
    // evenly over the 8 XCDs.
    const int64_t tiles_m = (m + 255) / 256;
    const int64_t full = (tiles / cus) * cus, rest = tiles - full;
    const int sbs = k / 256;
    if (full > 0 && rest > 0 && full % tiles_m == 0 && full % 8 == 0) {
      int ts = (int)std::min<int64_t>(cus / rest, sbs / 2);
      while (ts >= 2 && (rest * ts) % 8 != 0) --ts;
      const int64_t nt = full / tiles_m * 128;
      const size_t bytes = (size_t)ts * m * (size_t)(n - nt) * 4;
      if (ts >= 2 && nt < n && bytes <= part_avail) {
        pl.tail_full = (int)full;
        pl.tail_s = ts;
        pl.sbps = (sbs + ts - 1) / ts;
        pl.part_bytes = bytes;
      }
    }
    return pl;
  }
  const int sbs = k / 256;
  int splits = (int)std::min<int64_t>(cus / tiles, sbs / 2);  // at least two super-blocks per split
  const size_t per = (size_t)m * n * 4;
  if (per > 0) splits = (int)std::min<size_t>((size_t)splits, part_avail / per);
  // split unless gemm_q4k.h's 64-token tiles give more than twice the
  // workgroups (a workgroup here does four times their work per step, at
  // about twice their speed)
  const int64_t tiles_64 = (int64_t)((m + 63) / 64) * ((n + 127) / 128);
  if (splits < 2 || 2 * tiles * splits < tiles_64) return pl;
  pl.sbps = (sbs + splits - 1) / splits;
  pl.splits = (sbs + pl.sbps - 1) / pl.sbps;
  pl.part_bytes = (size_t)pl.splits * per;
  return pl;
}

// Launches the activation prep and the GEMM (and, split, the reduction);
// `workspace` holds gemm_q4k_ws_layout(m, k) bytes followed by
// plan.part_bytes.
inline int launch_gemm_q4k2(const void* w, const void* x, const float* bias, float* y, int m, int n, int k,
                            void* workspace, const GemmQ4k2Plan& plan, hipStream_t s) {
  GemmQ4kWs ws;
  const size_t base = gemm_q4k_ws_layout(m, k, static_cast<char*>(workspace), &ws);
  const bool tail = plan.tail_s > 1;
  float* part = plan.splits > 1 || tail ? reinterpret_cast<float*>(static_cast<char*>(workspace) + base) : nullptr;
  hipLaunchKernelGGL(gemm_prep_kernel, dim3((unsigned)m), dim3(256), 0, s, static_cast<const uint16_t*>(x), m, k, ws);
  if (int rc = check_launch("gemm_prep")) return rc;
  const int tiles_n = (n + 127) / 128, tiles_m = (m + 255) / 256, tiles = tiles_m * tiles_n;
  const int grid = tail ? plan.tail_full + (tiles - plan.tail_full) * plan.tail_s : tiles * plan.splits;
  hipLaunchKernelGGL((gemm_q4k2_kernel<4, 2>), dim3((unsigned)grid), dim3(512), 0, s, static_cast<const uint8_t*>(w),
                     ws, bias, y, m, n, k, tiles_m, tiles, plan.sbps, part, plan.tail_full, plan.tail_s);
  if (int rc = check_launch("gemm_q4k2")) return rc;
  if (!part) return 0;
  const int nt = tail ? plan.tail_full / tiles_m * 128 : 0;
  const size_t total = (size_t)m * (n - nt);
  hipLaunchKernelGGL(gemm_split_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part,
                     tail ? plan.tail_s : plan.splits, m, n, nt, ws.rsc, bias, y);
  return check_launch("gemm_split_reduce");
}

}  // namespace draco
