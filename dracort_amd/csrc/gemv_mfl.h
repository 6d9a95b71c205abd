// Small-batch decode GEMV (2..16 activation rows) for Q4_K and Q6_K with the
// weight tiles staged through LDS.
//
// The chunk math is the persistent matrix-core GEMV's (gemv_mfma.h:
// activations resident in registers for the launch, wave ks taking chunks
// ks, ks + W, ...; one MFMA per scale group against the codes as 128 + code,
// the bias cancelled through the MFMA's C operand), and so are the results,
// bit for bit.  The weights reach the lanes differently.  A lane's share of
// a 16-row tile in the MFMA layout is a few pieces per chunk spread over 16
// rows; loading that straight into registers issues requests that each touch
// 16 rows (measured on MI355X: with the math removed, a 2 x 14336 x 4096
// launch moved 2.9 TB/s where a plain read of the same bytes reaches 5.3).
// Here the tile is read by the whole workgroup as consecutive 16-byte pieces
// of its 16 rows, written to an LDS image with each row padded by 16 bytes
// (rows fall on different banks), and the lanes read their pieces from
// there; see mfl_stream_u for the pipeline.
//
// The same stream serves the split-K form (gemv_mfl_split_kernel): one
// workgroup per CU takes an equal run of (split, tile) units, holds the
// split's activations in registers and writes raw partial sums that
// gemv_split_sum_kernel adds in split order.
#pragma once

#include "gemv_mfma.h"

namespace draco {

// Bytes of one 256-element chunk of a row, and the LDS bytes of one matrix's
// unit image (W chunks of 16 rows, rows padded by 16 bytes).
template <int QT> struct MflChunk { static constexpr int bytes = QT == kQ6_K ? 210 : 144; };
template <int QT>
__host__ __device__ constexpr int mfl_unit_lds(int w) { return 16 * (w * MflChunk<QT>::bytes + 16); }

// Streams ntiles 16-row tiles of NR matrices (Q4_K, or one Q6_K matrix)
// through LDS against the wave's resident activations xr.  A tile's rows
// are `chunks` 256-element chunks long, starting at tile_base(i, r).rowoff
// (matrix r's buffer resource, byte offset of tile i's first row plus any
// chunk offset; rows row_bytes apart).  The tile is read in units of W
// chunks of its 16 rows (unit j: chunks W j .. W j + W - 1, one per wave; U =
// chunks / W units per tile, rounded up; Q6_K units are whole, W chunks of
// 210 bytes being whole 16-byte pieces).  Units alternate between two LDS
// images (`wl`: 2 x NR x mfl_unit_lds<QT>(W) bytes) and two register staging
// slots: a wave multiplies unit v from its image, writes unit v + 1 (landed
// in registers) to the other image, requests unit v + 3 into the freed slot
// and meets the other waves at one barrier per unit.  A tile's partial
// 16 x 16 results go to part[tile parity] and are summed by wave 0 after the
// barrier, while the other waves go on; emit(i, tot) runs on wave 0 with
// tile i's summed result.  Q6_K super-blocks sit at even LDS offsets, so
// each dword field is read as the two aligned dwords around it and realigned
// (v_alignbyte).
// Resident activations of one chunk: bf16 (P = 1), or float32 values as three
// bf16 planes (P = 3, Q4_K; the chunk math against the codes without bias).
template <int QT, int P> struct MflX { typedef typename MfpTypes<QT>::X T; };
template <> struct MflX<kQ4_K, 3> { typedef mf_bf16x8 T[8][3]; };

template <int QT, bool DL, int NR, int W, int U, int P, int NX, class TileBase, class Emit>
__device__ __forceinline__ void mfl_stream_u(const typename MflX<QT, P>::T (&xr)[NX], int chunks, int ntiles,
                                             int row_bytes, TileBase tile_base, Emit emit, uint8_t* __restrict__ wl,
                                             mf_f32x4 (&part)[2][W][NR][64]) {
  constexpr int NT = W * 64;
  static_assert(U >= 1 && U <= NX && NX <= 16 / W, "units per tile");
  static_assert(P == 1 || (P == 3 && QT == kQ4_K), "three planes: Q4_K");
  static_assert(QT == kQ4_K || (QT == kQ6_K && NR == 1 && (W * 210) % 16 == 0), "Q4_K, or one Q6_K matrix");
  constexpr int CB = MflChunk<QT>::bytes;
  constexpr int UB = W * CB;                     // bytes of one row's span in a unit
  constexpr int PPR = UB / 16;                   // 16-byte pieces per row and unit
  constexpr int PPT = (16 * PPR + NT - 1) / NT;  // pieces per thread and matrix
  constexpr int RS = UB + 16, IMG = 16 * RS;     // LDS row stride, image per matrix
  constexpr int QL = DL ? 0 : 2, QH = DL ? 128 : 130, SC = DL ? 192 : 194, D = DL ? 208 : 0;
  const int tid = threadIdx.x, lane = tid & 63;
  const int ks = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, nl = lane & 15;
  const int nunits = ntiles * U;

  // this thread's pieces: row, 16-byte column within the unit's span, LDS destination
  int prow[PPT], pcol[PPT], dst[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int pc = tid + NT * j;
    prow[j] = pc / PPR;
    pcol[j] = pc - prow[j] * PPR;
    dst[j] = pc < 16 * PPR ? prow[j] * RS + (pcol[j] << 4) : -1;
  }
  uint4 stg[2][NR][PPT];
  // unit v into a staging slot; past the last unit (or a column past the
  // row's chunks) an empty resource / an offset past the end reads zero
  auto issue = [&](int v, uint4 (&sl)[NR][PPT]) {
    const int i = min(v / U, ntiles - 1), uj = v - (v / U) * U;
    const int span = (min(chunks - W * uj, W) * CB) >> 4;  // pieces per row in this unit
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const MfRow t = tile_base(i, r);
      const __amdgpu_buffer_rsrc_t rs = v < nunits ? t.rs : make_rsrc(nullptr, 0u);
#pragma unroll
      for (int j = 0; j < PPT; ++j) {
        const bool ok = dst[j] >= 0 && pcol[j] < span;
        const uint32_t off = ok ? (uint32_t)(t.rowoff + prow[j] * row_bytes + uj * UB + (pcol[j] << 4)) : 0x80000000u;
        typedef int v4i __attribute__((ext_vector_type(4)));
        const v4i x4 = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
        sl[r][j] = uint4{(uint32_t)x4.x, (uint32_t)x4.y, (uint32_t)x4.z, (uint32_t)x4.w};
      }
    }
  };
  auto commit = [&](const uint4 (&sl)[NR][PPT], uint8_t* img) {
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int j = 0; j < PPT; ++j)
        if (dst[j] >= 0) *reinterpret_cast<uint4*>(img + r * IMG + dst[j]) = sl[r][j];
  };

  if (ntiles <= 0) return;
  issue(0, stg[0]);
  issue(1, stg[1]);
  // the resident chunks' group sums (Q4_K) once the first weight requests are
  // out: waiting for the activations then overlaps the weights' latency
  float sx[NX][2];
  if constexpr (QT == kQ4_K)
#pragma unroll
    for (int j = 0; j < NX; ++j) {
      if constexpr (P == 1)
        mf_group_sums(xr[j], q, sx[j]);
      else
        mf_group_sums3(xr[j], q, sx[j]);
    }
  commit(stg[0], wl);
  issue(2, stg[0]);
  __syncthreads();
  mf_f32x4 acc[NR];
  // units in pairs so that the staging slot and image (v % 2) and, for U = 2,
  // the unit within its tile are compile-time constants
  for (int v0 = 0; v0 < nunits; v0 += 2) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const int v = v0 + sl;
      const int i = U == 2 ? v0 / 2 : v;  // tile
      const int uj = U == 2 ? sl : 0;     // unit within the tile
      const bool live = v < nunits;
      const bool last = uj == U - 1;
      const int pi = i & 1;  // partial-tile buffer of this tile
      if (live) {
        if (uj == 0)
#pragma unroll
          for (int r = 0; r < NR; ++r) acc[r] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
        const int xj = U == 2 ? sl : 0;  // the resident chunk of this unit
        if (W * uj + ks < chunks) {
          const uint8_t* img = wl + sl * NR * IMG;
          if constexpr (QT == kQ4_K) {
            MfChunk<kQ4_K> wc[NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
              const uint8_t* rp = img + r * IMG + nl * RS + ks * CB;
              wc[r].head = *reinterpret_cast<const uint4*>(rp);
#pragma unroll
              for (int p = 0; p < 4; ++p) {
                const uint2 t = *reinterpret_cast<const uint2*>(rp + 16 + 32 * p + 8 * q);
                wc[r].qs[p][0] = t.x;
                wc[r].qs[p][1] = t.y;
              }
            }
            if constexpr (P == 1)
              mf_chunk_q4k_sx<NR>(xr[xj], wc, q, acc, sx[xj]);
            else
              mf_chunk_q4k_sx3<NR>(xr[xj], wc, q, acc, sx[xj]);
          } else {
            const uint8_t* rp = img + nl * RS;
            const int base = ks * CB;
            // the four bytes at row offset o (even) from the aligned dwords around them
            auto dw = [&](int o) -> uint32_t {
              const uint32_t* w = reinterpret_cast<const uint32_t*>(rp + (o & ~3));
              return __builtin_amdgcn_alignbyte(w[1], w[0], (uint32_t)(o & 3));
            };
            MfQ6 wc[1];
#pragma unroll
            for (int n = 0; n < 2; ++n)
#pragma unroll
              for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                  wc[0].ql[4 * n + 2 * tb + h] = dw(base + QL + 64 * n + 32 * tb + 16 * h + 4 * q);
#pragma unroll
            for (int n = 0; n < 2; ++n)
#pragma unroll
              for (int h = 0; h < 2; ++h) wc[0].qh[2 * n + h] = dw(base + QH + 32 * n + 16 * h + 4 * q);
            wc[0].sc = uint4{dw(base + SC), dw(base + SC + 4), dw(base + SC + 8), dw(base + SC + 12)};
            wc[0].d = dw(base + D) & 0xFFFFu;
            mf_chunk_q6<1>(xr[xj], wc, acc);
          }
        }
        if (last)
#pragma unroll
          for (int r = 0; r < NR; ++r) part[pi][ks][r][lane] = acc[r];
      }
      // the other image was last read by unit v - 1, which every wave finished
      // before the previous barrier
      if (v + 1 < nunits) {
        commit(stg[sl ^ 1], wl + (sl ^ 1) * NR * IMG);  // unit v + 1
        issue(v + 3, stg[sl ^ 1]);                     // an empty resource past the last unit
      }
      __syncthreads();  // unit v + 1 in LDS; after a tile's last unit, its partial tiles written
      if (live && last && ks == 0) {
        // part[pi] is next written two tiles later, after a barrier wave 0 reaches only after this
        mf_f32x4 tot[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          tot[r] = part[pi][0][r][lane];
#pragma unroll
          for (int w = 1; w < W; ++w) {
            const mf_f32x4 pp = part[pi][w][r][lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) tot[r][e] += pp[e];
          }
        }
        emit(i, tot);
      }
    }
  }
}

template <int QT, bool DL, int NR, int W, class TileBase, class Emit>
__device__ __forceinline__ void mfl_stream(const typename MfpTypes<QT>::X (&xr)[16 / W], int chunks, int ntiles,
                                           int row_bytes, TileBase tile_base, Emit emit, uint8_t* __restrict__ wl,
                                           mf_f32x4 (&part)[2][W][NR][64]) {
  if (chunks > W)
    mfl_stream_u<QT, DL, NR, W, 2, 1, 16 / W>(xr, chunks, ntiles, row_bytes, tile_base, emit, wl, part);
  else
    mfl_stream_u<QT, DL, NR, W, 1, 1, 16 / W>(xr, chunks, ntiles, row_bytes, tile_base, emit, wl, part);
}

// The Q4_K form (the MoE up projection's stream).
template <int NR, int W, class TileBase, class Emit>
__device__ __forceinline__ void mfl_stream_q4k(const typename MfpTypes<kQ4_K>::X (&xr)[16 / W], int chunks,
                                               int ntiles, int row_bytes, TileBase tile_base, Emit emit,
                                               uint8_t* __restrict__ wl, mf_f32x4 (&part)[2][W][NR][64]) {
  mfl_stream<kQ4_K, false, NR, W>(xr, chunks, ntiles, row_bytes, tile_base, emit, wl, part);
}

// The decode GEMV of 2..16 bf16 token rows over Q4_K (or single Q6_K)
// matrices with K <= 4096 (gemv_mfp_kernel's jobs, modes and results).
template <int QT, bool DL, int MODE, int W>
__global__ __launch_bounds__(W * 64) void gemv_mfl_kernel(StreamJob job) {
  constexpr int NR = MODE == kSwiGLU ? 2 : 1;
  static_assert(QT == kQ4_K || (QT == kQ6_K && NR == 1), "Q4_K, or one Q6_K matrix per row");
  __shared__ __attribute__((aligned(16))) uint8_t wl[2 * NR * mfl_unit_lds<QT>(W)];
  __shared__ mf_f32x4 part[2][W][NR][64];
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, nl = lane & 15;
  const int k = job.k, M = job.m;
  const int chunks = k >> 8;
  const int ntiles = job.rows >> 4;
  const int my_tiles = ntiles > (int)blockIdx.x ? (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;

  typename MfpTypes<QT>::X xr[16 / W];
  mfp_load_x<QT, W>(static_cast<const uint16_t*>(job.x) + (size_t)min(nl, M - 1) * k, chunks, ks, q, xr);

  int c1 = INT_MAX, c2 = INT_MAX, c3 = INT_MAX;
  if constexpr (MODE == kPlain) {
    if (job.n_mats > 1) c1 = job.n[0];
    if (job.n_mats > 2) c2 = c1 + job.n[1];
    if (job.n_mats > 3) c3 = c2 + job.n[2];
  }
  const uint8_t *w0 = job.w[0], *w1 = job.w[1], *w2 = job.w[2], *w3 = job.w[3];
  const int n0 = job.n[0], n1 = job.n[1], n2 = job.n[2], n3 = job.n[3];
  float *y0 = job.y[0], *y1 = job.y[1], *y2 = job.y[2], *y3 = job.y[3];
  uint16_t *b0 = job.yb[0], *b1 = job.yb[1], *b2 = job.yb[2], *b3 = job.yb[3];
  float* const resid = job.resid;
  uint16_t* const resid_bf16 = job.resid_bf16;
  const float* const bias = job.bias;
  const int row_bytes = job.row_bytes;
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
  auto tile_base = [=](int i, int r) {
    int mat, lrow;
    locate(16 * ((int)blockIdx.x + i * (int)gridDim.x), mat, lrow);
    const int mm = NR == 2 ? r : mat;
    const uint8_t* wp = pick(mm, w0, w1, w2, w3);
    const int nn = pick(mm, n0, n1, n2, n3);
    return MfRow{make_rsrc(wp, (uint32_t)((int64_t)nn * row_bytes)), lrow * row_bytes};
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
  mfl_stream<QT, DL, NR, W>(xr, chunks, my_tiles, row_bytes, tile_base, emit, wl, part);
}

// Split-K small-batch GEMV for one matrix with long rows (the batch-16 down
// projection): K in splits of W chunks, units (split s, 16-row tile t) in
// split-major order, workgroup b of G taking units [U b / G, U (b + 1) / G)
// -- every CU the same number of tiles, the runs crossing a split boundary at
// most once.  For each split of its run the workgroup loads that split's
// activations (16 token rows x W chunks, one chunk per wave, rows past M
// repeating row M - 1) into registers once and streams its tiles through
// mfl_stream_u; each tile's raw 16 x 16 sums go to part[s] (M x n floats per
// split), which gemv_split_sum_kernel adds in split order.  Q6_K needs
// whole-W-chunk splits (K a multiple of 2048); n a multiple of 16.
template <int QT, bool DL, int W>
__global__ __launch_bounds__(W * 64) void gemv_mfl_split_kernel(StreamJob job) {
  constexpr int CB = MflChunk<QT>::bytes;
  __shared__ __attribute__((aligned(16))) uint8_t wl[2 * mfl_unit_lds<QT>(W)];
  __shared__ mf_f32x4 part[2][W][1][64];
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, nl = lane & 15;
  const int k = job.k, M = job.m, chunks = k >> 8;
  const int n = job.n[0], tiles = n >> 4, row_bytes = job.row_bytes;
  const int splits = (chunks + W - 1) / W;
  const int units = splits * tiles;
  const int G = gridDim.x, b = blockIdx.x;
  const int u1 = (int)((int64_t)units * (b + 1) / G);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(job.w[0], (uint32_t)((int64_t)n * row_bytes));
  const uint16_t* const x = static_cast<const uint16_t*>(job.x);
  float* const out = job.part;
  for (int u = (int)((int64_t)units * b / G); u < u1;) {
    const int s = u / tiles, t0 = u - s * tiles;
    const int nt = min(u1 - u, tiles - t0);
    const int c0 = W * s, nch = min(W, chunks - c0);
    typename MfpTypes<QT>::X xr[16 / W];
    mfp_load_x<QT, W>(x + (size_t)min(nl, M - 1) * k + c0 * 256, nch, ks, q, xr);
    auto tile_base = [=](int i, int) { return MfRow{rs, (t0 + i) * 16 * row_bytes + c0 * CB}; };
    auto emit = [=](int i, const mf_f32x4 (&tot)[1]) {
      float* const pp = out + (size_t)s * M * n + 16 * (t0 + i) + nl;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (4 * q + v < M) pp[(size_t)(4 * q + v) * n] = tot[0][v];
    };
    mfl_stream_u<QT, DL, 1, W, 1, 1, 16 / W>(xr, nch, nt, row_bytes, tile_base, emit, wl, part);
    u += nt;
  }
}

// Whether gemv_mfl_split_kernel takes a split launch of this job.
inline bool mfl_split_ok(int qtype, const StreamJob& job) {
  return job.n_mats == 1 && job.rows % 16 == 0 && job.split_chunks == 8 &&
         (qtype == kQ4_K || (qtype == kQ6_K && job.k % 2048 == 0));
}

template <int QT, bool DL, int MODE, int W>
static int launch_gemv_mfl(const StreamJob& job, int blocks_per_cu, hipStream_t s) {
  if (job.k > 4096 || job.k % (QT == kQ6_K ? 2048 : 256) != 0 || job.rows % 16 != 0)
    return set_error(DRACO_EINVAL_SHAPE, "LDS-staged matrix-core GEMV takes K <= 4096 and whole 16-row tiles");
  const int tiles = job.rows / 16;
  const int blocks = std::max(1, std::min(tiles, device_cus() * blocks_per_cu));
  hipLaunchKernelGGL((gemv_mfl_kernel<QT, DL, MODE, W>), dim3(blocks), dim3(W * 64), 0, s, job);
  return check_launch("gemv_mfl");
}

// A split launch (job.part from gemv_split_bytes) through gemv_mfl_split_kernel,
// one workgroup per CU (or per unit when there are fewer), then the ordered sum.
template <int QT, bool DL, int MODE>
static int launch_gemv_mfl_split(const StreamJob& job, hipStream_t s) {
  const int splits = (job.k / 256 + 7) / 8;
  const int units = splits * (job.rows / 16);
  hipLaunchKernelGGL((gemv_mfl_split_kernel<QT, DL, 8>), dim3(std::max(1, std::min(units, device_cus()))), dim3(512),
                     0, s, job);
  if (int rc = check_launch("gemv_mfl_split")) return rc;
  const size_t total = (size_t)job.m * job.n[0];
  float* const y = MODE == kResid ? job.resid : job.y[0];
  uint16_t* const yb = MODE == kResid ? job.resid_bf16 : job.yb[0];
  hipLaunchKernelGGL(gemv_split_sum_kernel<MODE>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, job.part,
                     splits, job.m, job.n[0], y, yb, job.bias);
  return check_launch("gemv_split_sum");
}

template <int MODE>
static int gemv_mfma_dispatch(int qtype, bool d_last, const StreamJob& job, bool xbf16, hipStream_t s) {
  // long rows split over K with a workspace: the LDS-staged split form
  // (measured on MI355X at 16 rows, 4096 x 14336 Q6_K: see gemv_mfl_split_kernel)
  if constexpr (MODE != kSwiGLU) {
    if (xbf16 && job.part && mfl_split_ok(qtype, job)) {
      if (qtype == kQ6_K)
        return d_last ? launch_gemv_mfl_split<kQ6_K, true, MODE>(job, s) : launch_gemv_mfl_split<kQ6_K, false, MODE>(job, s);
      return launch_gemv_mfl_split<kQ4_K, false, MODE>(job, s);
    }
  }
  // bf16 rows of at most 16 chunks: the persistent form (activations resident
  // in registers), one 512-thread workgroup per CU (measured best: 14336 x 4096
  // Q4_K at M = 16 18 us vs 30 us for the one-tile-per-workgroup form)
  // (SwiGLU's two weight sets fit the 512-thread register budget for Q4_K only)
  if (xbf16 && job.k <= 4096 && (MODE != kSwiGLU || qtype == kQ4_K)) {
    if constexpr (MODE != kSwiGLU) {
      // Q6_K rows of whole 16-byte pieces (K a multiple of 2048) through LDS
      // as well; other lengths read their tiles straight into registers
      if (qtype == kQ6_K && job.k % 2048 == 0)
        return d_last ? launch_gemv_mfl<kQ6_K, true, MODE, 8>(job, 1, s)
                      : launch_gemv_mfl<kQ6_K, false, MODE, 8>(job, 1, s);
      if (qtype == kQ6_K)
        return d_last ? launch_gemv_mfp<kQ6_K, true, MODE, 8>(job, 1, s)
                      : launch_gemv_mfp<kQ6_K, false, MODE, 8>(job, 1, s);
    }
    // Q4_K: the LDS-staged form above, bit-identical and faster (measured at
    // 16 rows: gate/up 33.1 -> 28.4 us, q/k/v 12.6 -> 11.5, o 11.1 -> 9.6)
    if (qtype == kQ4_K) return launch_gemv_mfl<kQ4_K, false, MODE, 8>(job, 1, s);
    if constexpr (MODE != kSwiGLU) return launch_gemv_mfp<kQ4_0, false, MODE, 8>(job, 1, s);
  }
  if (qtype == kQ6_K)
    return d_last ? launch_gemv_mfma<kQ6_K, true, true, MODE>(job, s) : launch_gemv_mfma<kQ6_K, false, true, MODE>(job, s);
  if (qtype == kQ4_K)
    return xbf16 ? launch_gemv_mfma<kQ4_K, false, true, MODE>(job, s)
                 : launch_gemv_mfma<kQ4_K, false, false, MODE>(job, s);
  return xbf16 ? launch_gemv_mfma<kQ4_0, false, true, MODE>(job, s) : launch_gemv_mfma<kQ4_0, false, false, MODE>(job, s);
}

}  // namespace draco
