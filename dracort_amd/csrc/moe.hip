// Sparse MoE FFN over GGUF-quantized experts on gfx950.
//
// Replaces TopKRouter.forward (draco/models/moe/router.py:81-120) and
// ExpertGroup.forward / Expert.forward (draco/models/moe/expert.py:47-49,
// 77-116) with four launches and no host synchronization:
//
//  1. moe_route_kernel (one workgroup): per token, top-k of the router logits
//     (ties -> lower expert index), softmax over the k logits, renormalised by
//     their sum (router.py:106-111); slots sorted by expert id.  Tokens are
//     then grouped by expert: counts, exclusive offsets, and for every expert
//     its tokens in ascending order (a block-wide ballot/popcount scan, so
//     the grouping is deterministic).
//  2. moe_up_kernel: grid (row blocks of the intermediate dim, experts).  Each
//     wave runs the register GEMV core on W_gate[e] and W_up[e] for the
//     expert's gathered tokens (16 at a time) and writes
//     h = silu(gate) * up in float32.
//  3. moe_down_kernel: the same core on W_down[e] over h, one output row per
//     (expert, token) assignment.
//  4. moe_combine_kernel: y[t] = sum over the token's slots in ascending
//     expert order of weight * down_out, the reference's index_add_ order.
//
// Q4_K and Q4_0 experts with 256-divisible dims take the matrix-core forms of
// steps 2 and 3 (moe_up_mfma_kernel, moe_down_mfma_kernel): a workgroup owns
// one 16-row weight tile of one expert, four waves split K, and each gathered
// tile of 16 tokens is one 16 x 16 MFMA output tile (the decode GEMV's
// mf_accumulate), so an expert's weights are read once per 16 tokens instead
// of once per token row of the register core.
#include "draco_internal.h"
#include "gemv_core.h"
#include "gemv_mfl.h"

namespace draco {

constexpr int kMaxExperts = 64;
constexpr int kMaxTopK = 8;
constexpr int kMoeMT = 16;

struct ExpertPtrs {
  const uint8_t* p[kMaxExperts];
};

struct MoeWs {
  int* sel_e;       // [T*k] expert of each slot, slots ascending by expert
  float* sel_w;     // [T*k] routing weight of each slot
  int* slot_pos;    // [T*k] assignment row of each slot
  int* assign_tok;  // [T*k] token of each assignment row, grouped by expert
  int* counts;      // [E]
  int* offsets;     // [E + 1]
  float* h;         // [T*k, inter]  silu(gate) * up (register-core path)
  uint16_t* hp;     // [3][T*k, inter] the same as three bf16 planes (matrix-core path)
  size_t hp_plane;  // elements per plane: T*k*inter
  float* yk;        // [T*k, hidden] expert outputs
  float* yks;       // [splits][T*k, hidden] the matrix-core down projection's split sums
  int tk;           // T*k
};

static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// K splits of the LDS-staged down projection (eight 256-element chunks each).
static int moe_down_splits(int64_t I) { return (int)((I / 256 + 7) / 8); }

static size_t moe_ws_layout(int64_t T, int64_t H, int64_t I, int E, int k, char* base, MoeWs* ws) {
  const size_t tk = (size_t)T * k;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  MoeWs w;
  w.sel_e = (int*)take(tk * 4);
  w.sel_w = (float*)take(tk * 4);
  w.slot_pos = (int*)take(tk * 4);
  w.assign_tok = (int*)take(tk * 4);
  w.counts = (int*)take((size_t)E * 4);
  w.offsets = (int*)take((size_t)(E + 1) * 4);
  w.h = (float*)take(tk * (size_t)I * 4);
  w.hp = (uint16_t*)take(3 * tk * (size_t)I * 2);
  w.hp_plane = tk * (size_t)I;
  w.yk = (float*)take(tk * (size_t)H * 4);
  w.yks = (float*)take((size_t)moe_down_splits(I) * tk * (size_t)H * 4);
  w.tk = (int)tk;
  if (ws) *ws = w;
  return off;
}

// Top-k of one token's logits (ties: the lower expert id), softmax over the
// k, renormalised, slots sorted by expert id.  EM > 0: at most EM experts, the
// expert loop unrolled (lg may then be a register array).
template <int EM = 0>
__device__ __forceinline__ void moe_topk(const float* __restrict__ lg, int E, int k, int (&idx)[kMaxTopK],
                                         float (&ex)[kMaxTopK]) {
  float val[kMaxTopK];
  uint64_t taken = 0;
  for (int j = 0; j < k; ++j) {
    int best = -1;
    float bv = 0.f;
#pragma unroll
    for (int e = 0; e < (EM > 0 ? EM : E); ++e) {
      if (EM > 0 && e >= E) break;
      if (taken >> e & 1ull) continue;
      const float v = lg[e];
      if (best < 0 || v > bv) { best = e; bv = v; }
    }
    taken |= 1ull << best;
    idx[j] = best;
    val[j] = bv;
  }
  float s = 0.f;
  for (int j = 0; j < k; ++j) { ex[j] = __expf(val[j] - val[0]); s += ex[j]; }
  float s2 = 0.f;
  for (int j = 0; j < k; ++j) { ex[j] = ex[j] / s; s2 += ex[j]; }
  for (int j = 0; j < k; ++j) ex[j] = ex[j] / s2;
  for (int a = 1; a < k; ++a) {  // insertion sort by expert id
    int ie = idx[a];
    float we = ex[a];
    int b = a - 1;
    while (b >= 0 && idx[b] > ie) { idx[b + 1] = idx[b]; ex[b + 1] = ex[b]; --b; }
    idx[b + 1] = ie;
    ex[b + 1] = we;
  }
}

__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                        MoeWs ws) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int offs[kMaxExperts + 1];
  __shared__ int running[kMaxExperts];
  __shared__ int wave_tot[4];
  __shared__ int wcnt[4][kMaxExperts];  // single-pass grouping: slots of expert e per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  if (T <= 256) {
    // one token per thread, its slots in registers: the same routing and the
    // same grouping (tokens of expert e in ascending token order) as the
    // general path below, with one ballot per expert and wave instead of a
    // pass with barriers per expert
    const int t = tid;
    int idx[kMaxTopK];
    float ex[kMaxTopK];
    if (t < T) {
      if (E <= 16) {
        float lr[16];  // the token's logits, loaded once (unrolled: static register indices)
        const float* lg = logits + (size_t)t * E;
#pragma unroll
        for (int e = 0; e < 16; ++e) lr[e] = e < E ? lg[e] : 0.f;
        moe_topk<16>(lr, E, k, idx, ex);
      } else {
        moe_topk(logits + (size_t)t * E, E, k, idx, ex);
      }
      for (int j = 0; j < k; ++j) {
        ws.sel_e[t * k + j] = idx[j];
        ws.sel_w[t * k + j] = ex[j];
      }
    }
    int rk[kMaxTopK] = {};
    for (int e = 0; e < E; ++e) {
      bool has = false;
#pragma unroll
      for (int j = 0; j < kMaxTopK; ++j) has |= t < T && j < k && idx[j] == e;
      const uint64_t mask = __ballot(has);
      const int r = __popcll(mask & ((1ull << lane) - 1ull));
#pragma unroll
      for (int j = 0; j < kMaxTopK; ++j)
        if (t < T && j < k && idx[j] == e) rk[j] = r;
      if (lane == 0) wcnt[wave][e] = __popcll(mask);
    }
    __syncthreads();
    if (tid == 0) {
      int acc = 0;
      for (int e = 0; e < E; ++e) {
        offs[e] = acc;
        acc += wcnt[0][e] + wcnt[1][e] + wcnt[2][e] + wcnt[3][e];
      }
      offs[E] = acc;
    }
    __syncthreads();
    if (tid < E) {
      ws.counts[tid] = offs[tid + 1] - offs[tid];
      ws.offsets[tid] = offs[tid];
    }
    if (tid == 0) ws.offsets[E] = offs[E];
    if (t < T)
#pragma unroll
      for (int j = 0; j < kMaxTopK; ++j) {
        if (j >= k) break;
        const int e = idx[j];
        int before = 0;
        for (int w = 0; w < wave; ++w) before += wcnt[w][e];
        const int pos = offs[e] + before + rk[j];
        ws.assign_tok[pos] = t;
        ws.slot_pos[t * k + j] = pos;
      }
    return;
  }

  // 1. top-k, softmax, renormalise, sort slots by expert
  for (int t = tid; t < T; t += 256) {
    int idx[kMaxTopK];
    float ex[kMaxTopK];
    moe_topk(logits + (size_t)t * E, E, k, idx, ex);
    for (int j = 0; j < k; ++j) {
      ws.sel_e[t * k + j] = idx[j];
      ws.sel_w[t * k + j] = ex[j];
    }
  }
  for (int e = tid; e < E; e += 256) { cnt[e] = 0; running[e] = 0; }
  __syncthreads();

  // 2. per-expert counts and exclusive offsets
  for (int s = tid; s < T * k; s += 256) atomicAdd(&cnt[ws.sel_e[s]], 1);
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) { offs[e] = acc; acc += cnt[e]; }
    offs[E] = acc;
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) { ws.counts[e] = cnt[e]; ws.offsets[e] = offs[e]; }
  if (tid == 0) ws.offsets[E] = offs[E];

  // 3. deterministic grouping: tokens of expert e in ascending token order
  for (int cb = 0; cb < T; cb += 256) {
    const int t = cb + tid;
    for (int e = 0; e < E; ++e) {
      int js = -1;
      if (t < T)
        for (int j = 0; j < k; ++j)
          if (ws.sel_e[t * k + j] == e) js = j;
      const bool flag = js >= 0;
      const uint64_t mask = __ballot(flag);
      const int rank = __popcll(mask & ((1ull << lane) - 1ull));
      if (lane == 0) wave_tot[wave] = __popcll(mask);
      __syncthreads();
      int before = 0, total = 0;
      for (int w = 0; w < 4; ++w) {
        if (w < wave) before += wave_tot[w];
        total += wave_tot[w];
      }
      if (flag) {
        const int pos = offs[e] + running[e] + before + rank;
        ws.assign_tok[pos] = t;
        ws.slot_pos[t * k + js] = pos;
      }
      __syncthreads();
      if (tid == 0) running[e] += total;
      __syncthreads();
    }
  }
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.f + __expf(-g)); }

template <int QT, bool XBF16, int R>
__global__ __launch_bounds__(256) void moe_up_kernel(ExpertPtrs wg, ExpertPtrs wu, const void* __restrict__ x,
                                                     int H, int I, MoeWs ws) {
  const int e = blockIdx.y;
  const int cnt = ws.counts[e];
  if (cnt == 0) return;
  const int off = ws.offsets[e];
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
  if (n0 >= I) return;
  const int64_t row_bytes = (int64_t)(H / Fmt<QT>::QK) * Fmt<QT>::BYTES;
  const size_t xstride = XBF16 ? (size_t)H * 2 : (size_t)H * 4;
  const uint8_t* xb = static_cast<const uint8_t*>(x);
  for (int t0 = 0; t0 < cnt; t0 += kMoeMT) {
    const int mt = min(kMoeMT, cnt - t0);
    const int* toks = ws.assign_tok + off + t0;
    auto xrow = [&](int mi) { return (const void*)(xb + (size_t)toks[mi] * xstride); };
    float ag[R][kMoeMT], au[R][kMoeMT];
    gemv_accumulate<QT, false, kMoeMT, XBF16, R>(wg.p[e], row_bytes, n0, I, H, mt, xrow, ag);
    gemv_accumulate<QT, false, kMoeMT, XBF16, R>(wu.p[e], row_bytes, n0, I, H, mt, xrow, au);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mi = 0; mi < kMoeMT; ++mi) {
        const float g = wave_sum(ag[r][mi]);
        const float u = wave_sum(au[r][mi]);
        if (lane == 0 && mi < mt && n0 + r < I) ws.h[(size_t)(off + t0 + mi) * I + n0 + r] = silu_f(g) * u;
      }
  }
}

template <int QT, int R>
__global__ __launch_bounds__(256) void moe_down_kernel(ExpertPtrs wd, int H, int I, MoeWs ws) {
  const int e = blockIdx.y;
  const int cnt = ws.counts[e];
  if (cnt == 0) return;
  const int off = ws.offsets[e];
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
  if (n0 >= H) return;
  const int64_t row_bytes = (int64_t)(I / Fmt<QT>::QK) * Fmt<QT>::BYTES;
  for (int t0 = 0; t0 < cnt; t0 += kMoeMT) {
    const int mt = min(kMoeMT, cnt - t0);
    const float* hb = ws.h + (size_t)(off + t0) * I;
    auto xrow = [&](int mi) { return (const void*)(hb + (size_t)mi * I); };
    float acc[R][kMoeMT];
    gemv_accumulate<QT, false, kMoeMT, false, R>(wd.p[e], row_bytes, n0, H, I, mt, xrow, acc);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mi = 0; mi < kMoeMT; ++mi) {
        const float v = wave_sum(acc[r][mi]);
        if (lane == 0 && mi < mt && n0 + r < H) ws.yk[(size_t)(off + t0 + mi) * H + n0 + r] = v;
      }
  }
}

// h[off + t0 + m, :] = silu(x_t W_gate[e]^T) * (x_t W_up[e]^T) for the
// expert's tokens t = assign_tok[off + t0 + m], 16 tokens per pass.
template <int QT, bool XBF16>
__global__ __launch_bounds__(256) void moe_up_mfma_kernel(ExpertPtrs wg, ExpertPtrs wu, const void* __restrict__ x,
                                                          int H, int I, MoeWs ws) {
  __shared__ mf_f32x4 part[4][2][64];
  const int e = blockIdx.y;
  const int cnt = ws.counts[e];
  if (cnt == 0) return;
  const int off = ws.offsets[e];
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, nl = lane & 15;
  const int row0 = blockIdx.x * 16;  // I is a multiple of 16 and the grid covers it exactly
  const uint32_t row_bytes = (uint32_t)(H / Fmt<QT>::QK) * Fmt<QT>::BYTES;
  const __amdgpu_buffer_rsrc_t rs[2] = {make_rsrc(wg.p[e], (uint32_t)I * row_bytes),
                                        make_rsrc(wu.p[e], (uint32_t)I * row_bytes)};
  const int rowoff = (int)((uint32_t)(row0 + nl) * row_bytes);
  const size_t xstride = (size_t)H * (XBF16 ? 2 : 4);
  for (int t0 = 16 * (int)blockIdx.z; t0 < cnt; t0 += 16 * (int)gridDim.z) {
    const int mt = min(16, cnt - t0);
    // lanes of token rows past the expert's count repeat its last token
    const int tok = ws.assign_tok[off + t0 + min(nl, mt - 1)];
    const void* xrow = static_cast<const uint8_t*>(x) + (size_t)tok * xstride;
    mf_f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    mf_accumulate<QT, XBF16, 2>(rs, rowoff, xrow, q, ks, H >> 8, acc);
    part[ks][0][lane] = acc[0];
    part[ks][1][lane] = acc[1];
    __syncthreads();
    if (ks == 0) {
      mf_f32x4 g = part[0][0][lane], u = part[0][1][lane];
#pragma unroll
      for (int j = 1; j < 4; ++j) {
        const mf_f32x4 pg = part[j][0][lane], pu = part[j][1][lane];
#pragma unroll
        for (int v = 0; v < 4; ++v) { g[v] += pg[v]; u[v] += pu[v]; }
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = 4 * q + v;  // D layout: lane l holds token rows 4 (l / 16) + v, weight row l % 16
        if (m < mt) {
          uint16_t a, b, c;
          mf_split3(silu_f(g[v]) * u[v], a, b, c);
          const size_t o = (size_t)(off + t0 + m) * I + row0 + nl;
          ws.hp[o] = a;
          ws.hp[ws.hp_plane + o] = b;
          ws.hp[2 * ws.hp_plane + o] = c;
        }
      }
    }
    __syncthreads();
  }
}

// Persistent form of the up projection for Q4_K experts with hidden <= 4096,
// one 512-thread workgroup per CU.  The work -- every 16-token tile of every
// expert (expert e has ceil(counts[e] / 16) of them, known only on the
// device) times the I / 16 row tiles of its gate / up matrices -- is cut
// into gridDim.x runs of equally many row tiles in (expert, token tile, row
// tile) order, one run per workgroup, so every CU streams the same number of
// tiles whatever the routing (a grid of one workgroup per (expert, token
// tile) slice left the slices of crowded experts to a second round).  A run
// spans few token tiles; for each the workgroup loads the 16 gathered
// tokens' activations into registers (eight waves split the hidden
// dimension) and streams its row tiles through LDS (mfl_stream_q4k).
__global__ __launch_bounds__(512) void moe_up_mfp_kernel(ExpertPtrs wg, ExpertPtrs wu,
                                                         const uint16_t* __restrict__ x, int H, int I, int E,
                                                         MoeWs ws) {
  constexpr int W = 8;
  __shared__ __attribute__((aligned(16))) uint8_t wl[2 * 2 * mfl_unit_lds<kQ4_K>(W)];
  __shared__ mf_f32x4 part[2][W][2][64];
  __shared__ int tb[kMaxExperts + 1];  // token tiles of the experts before e
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, nl = lane & 15;
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) {
      tb[e] = acc;
      acc += (ws.counts[e] + 15) >> 4;
    }
    tb[E] = acc;
  }
  __syncthreads();
  const int chunks = H >> 8, rt = I >> 4;
  const int64_t work = (int64_t)tb[E] * rt;
  const int64_t lo = work * (int64_t)blockIdx.x / (int64_t)gridDim.x;
  const int64_t hi = work * ((int64_t)blockIdx.x + 1) / (int64_t)gridDim.x;
  const int row_bytes = (H / 256) * 144;
  const uint32_t mat_bytes = (uint32_t)I * (uint32_t)row_bytes;
  uint16_t* const hp = ws.hp;
  const size_t plane = ws.hp_plane;
  for (int64_t idx = lo; idx < hi;) {
    // this segment: token tile `item` (expert e, tokens t0 ..), row tiles r0 .. r0 + nr
    const int item = __builtin_amdgcn_readfirstlane((int)(idx / rt));
    const int r0 = __builtin_amdgcn_readfirstlane((int)(idx - (int64_t)item * rt));
    const int nr = __builtin_amdgcn_readfirstlane((int)min((int64_t)(rt - r0), hi - idx));
    int e = 0;
    while (tb[e + 1] <= item) ++e;  // item < tb[E]; experts without tokens are skipped
    e = __builtin_amdgcn_readfirstlane(e);
    const int t0 = 16 * (item - tb[e]);
    const int off = ws.offsets[e];
    const int mt = min(16, ws.counts[e] - t0);
    const int tok = ws.assign_tok[off + t0 + min(nl, mt - 1)];
    const uint8_t* const gp = wg.p[e];
    const uint8_t* const upp = wu.p[e];
    typename MfpTypes<kQ4_K>::X xr[16 / W];
    mfp_load_x<kQ4_K, W>(x + (size_t)tok * H, chunks, ks, q, xr);
    auto tile_base = [=](int i, int r) {
      const int row = 16 * (r0 + i);
      return MfRow{make_rsrc(r == 0 ? gp : upp, mat_bytes), row * row_bytes};
    };
    auto emit = [=](int i, const mf_f32x4 (&tot)[2]) {
      const int col = 16 * (r0 + i) + nl;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = 4 * q + v;  // D layout: lane l holds token rows 4 (l / 16) + v, weight row l % 16
        if (m < mt) {
          uint16_t a, b, c;
          mf_split3(silu_f(tot[0][v]) * tot[1][v], a, b, c);
          const size_t o = (size_t)(off + t0 + m) * I + col;
          hp[o] = a;
          hp[plane + o] = b;
          hp[2 * plane + o] = c;
        }
      }
    };
    mfl_stream_q4k<2, W>(xr, chunks, nr, row_bytes, tile_base, emit, wl, part);
    idx += nr;
  }
}

// yk[off + t0 + m, :] = h[off + t0 + m, :] W_down[e]^T, 16 assignment rows per
// pass; h arrives as the three bf16 planes the up kernels wrote (three MFMAs
// per group against exact codes, no split here).
//
// NR 16-row weight tiles per workgroup share each wave's activation fragments
// (the h planes, re-read from L2 / the Infinity Cache by every row tile of
// the expert: 16 tokens x 14336 x 3 planes x 2 B = 1.4 MB per tile against
// 129 KB of Q4_K weights), which cuts that traffic NR-fold; launched with
// NR = 4 (Mixtral shape: 503, 287, 238 us for NR = 1, 2, 4; the extra
// accumulators spill to AGPRs, not to scratch).
template <int QT, int NR>
__global__ __launch_bounds__(256) void moe_down_mfma_kernel(ExpertPtrs wd, int H, int I, MoeWs ws) {
  __shared__ mf_f32x4 part[4][NR][64];
  const int e = blockIdx.y;
  const int cnt = ws.counts[e];
  if (cnt == 0) return;
  const int off = ws.offsets[e];
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, nl = lane & 15;
  const int row0 = blockIdx.x * 16 * NR;  // H is a multiple of 16 NR and the grid covers it exactly
  const uint32_t row_bytes = (uint32_t)(I / Fmt<QT>::QK) * Fmt<QT>::BYTES;
  __amdgpu_buffer_rsrc_t rs[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) rs[r] = make_rsrc(wd.p[e] + (size_t)(row0 + 16 * r) * row_bytes, 16u * row_bytes);
  const int rowoff = (int)((uint32_t)nl * row_bytes);
  for (int t0 = 16 * (int)blockIdx.z; t0 < cnt; t0 += 16 * (int)gridDim.z) {
    const int mt = min(16, cnt - t0);
    const uint16_t* xrow = ws.hp + (size_t)(off + t0 + min(nl, mt - 1)) * I;
    mf_f32x4 acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
    mf_accumulate<QT, false, NR, true>(rs, rowoff, xrow, q, ks, I >> 8, acc, ws.hp_plane);
#pragma unroll
    for (int r = 0; r < NR; ++r) part[ks][r][lane] = acc[r];
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        mf_f32x4 tot = part[0][r][lane];
#pragma unroll
        for (int j = 1; j < 4; ++j) {
          const mf_f32x4 p = part[j][r][lane];
#pragma unroll
          for (int v = 0; v < 4; ++v) tot[v] += p[v];
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = 4 * q + v;
          if (m < mt) ws.yk[(size_t)(off + t0 + m) * H + row0 + 16 * r + nl] = tot[v];
        }
      }
    }
    __syncthreads();
  }
}

// The down projection split along K, on the small-batch GEMV's LDS stream:
// units (token tile of an expert, split of eight chunks, 16-row tile of
// W_down[e]) in that order, one workgroup per CU taking an equal run.  For
// each (token tile, split) of its run a workgroup holds that split's h planes
// (16 assignment rows x 8 chunks x 3 bf16 planes, one chunk per wave) in
// registers and streams the row tiles through LDS (mfl_stream_u, three-plane
// chunk math against exact codes); each tile's raw sums go to yks[split], and
// moe_combine_split_kernel adds the splits in order.  Q4_K, H and I multiples
// of 256.
__global__ __launch_bounds__(512) void moe_down_mfl_kernel(ExpertPtrs wd, int H, int I, int E, MoeWs ws) {
  constexpr int W = 8;
  __shared__ __attribute__((aligned(16))) uint8_t wl[2 * mfl_unit_lds<kQ4_K>(W)];
  __shared__ mf_f32x4 part[2][W][1][64];
  __shared__ int tb[kMaxExperts + 1];  // token tiles of the experts before e
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, nl = lane & 15;
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) {
      tb[e] = acc;
      acc += (ws.counts[e] + 15) >> 4;
    }
    tb[E] = acc;
  }
  __syncthreads();
  const int chunks = I >> 8, splits = (chunks + W - 1) / W, rt = H >> 4;
  const int per = splits * rt;  // units per token tile
  const int units = tb[E] * per;
  const int G = gridDim.x, b = blockIdx.x;
  const int u1 = (int)((int64_t)units * (b + 1) / G);
  const int row_bytes = chunks * 144;
  const uint32_t mat_bytes = (uint32_t)H * (uint32_t)row_bytes;
  const size_t tk = (size_t)ws.tk;  // assignment rows
  for (int u = (int)((int64_t)units * b / G); u < u1;) {
    const int item = u / per, rem = u - item * per;
    const int s = rem / rt, r0 = rem - s * rt;
    const int nt = min(u1 - u, rt - r0);
    int e = 0;
    while (tb[e + 1] <= item) ++e;  // item < tb[E]; experts without tokens are skipped
    e = __builtin_amdgcn_readfirstlane(e);
    const int t0 = 16 * (item - tb[e]);
    const int off = ws.offsets[e];
    const int mt = min(16, ws.counts[e] - t0);
    const int c0 = W * s, nch = min(W, chunks - c0);
    mf_bf16x8 xr[1][8][3];
    {
      const uint16_t* xrow = ws.hp + (size_t)(off + t0 + min(nl, mt - 1)) * I;
      const int cc = min(c0 + ks, chunks - 1);
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const uint16_t* xp = xrow + cc * 256 + mf_pos<kQ4_K>(g, q);
#pragma unroll
        for (int j = 0; j < 3; ++j)
          xr[0][g][j] = __builtin_bit_cast(mf_bf16x8, *reinterpret_cast<const uint4*>(xp + j * ws.hp_plane));
      }
    }
    const uint8_t* const wp = wd.p[e];
    auto tile_base = [=](int i, int) {
      return MfRow{make_rsrc(wp, mat_bytes), (r0 + i) * 16 * row_bytes + c0 * 144};
    };
    float* const out = ws.yks + ((size_t)s * tk + off + t0) * H + nl;
    auto emit = [=](int i, const mf_f32x4 (&tot)[1]) {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (4 * q + v < mt) out[(size_t)(4 * q + v) * H + 16 * (r0 + i)] = tot[0][v];
    };
    mfl_stream_u<kQ4_K, false, 1, W, 1, 3, 1>(xr, nch, nt, row_bytes, tile_base, emit, wl, part);
    u += nt;
  }
}

// y[t] = sum over the token's k slots, in order, of w * (the slot's split sums
// added in split order); four consecutive outputs per thread (H a multiple of 4).
__global__ __launch_bounds__(256) void moe_combine_split_kernel(float* __restrict__ y, int H, int k, int splits,
                                                                MoeWs ws) {
  const int t = blockIdx.y;
  const int n = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (n >= H) return;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < k; ++j) {
    const int p = ws.slot_pos[t * k + j];
    const float w = ws.sel_w[t * k + j];
    float4 v = *reinterpret_cast<const float4*>(ws.yks + (size_t)p * H + n);
    for (int s = 1; s < splits; ++s) {
      const float4 u = *reinterpret_cast<const float4*>(ws.yks + ((size_t)s * ws.tk + p) * H + n);
      v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
    }
    acc.x = acc.x + v.x * w; acc.y = acc.y + v.y * w; acc.z = acc.z + v.z * w; acc.w = acc.w + v.w * w;
  }
  *reinterpret_cast<float4*>(y + (size_t)t * H + n) = acc;
}

__global__ __launch_bounds__(256) void moe_combine_kernel(float* __restrict__ y, int H, int k, MoeWs ws) {
  const int t = blockIdx.y;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= H) return;
  float acc = 0.f;
  for (int j = 0; j < k; ++j) {
    const int p = ws.slot_pos[t * k + j];
    const float contrib = ws.yk[(size_t)p * H + n] * ws.sel_w[t * k + j];
    acc = acc + contrib;
  }
  y[(size_t)t * H + n] = acc;
}

template <int QT>
static int launch_moe(const ExpertPtrs& wg, const ExpertPtrs& wu, const ExpertPtrs& wd, const float* logits,
                      const void* x, bool xbf16, float* y, int T, int H, int I, int E, int k, const MoeWs& ws,
                      hipStream_t s) {
  constexpr int R = 1;
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(256), 0, s, logits, T, E, k, ws);
  if (int rc = check_launch("moe_route")) return rc;
  if constexpr (QT == kQ4_K || QT == kQ4_0) {
    // matrix-core experts: K a whole number of 256-element chunks, whole
    // 16-row tiles, 32-bit buffer offsets within one expert matrix
    const int64_t up_bytes = (int64_t)I * (H / Fmt<QT>::QK) * Fmt<QT>::BYTES;
    const int64_t down_bytes = (int64_t)H * (I / Fmt<QT>::QK) * Fmt<QT>::BYTES;
    if (H % 256 == 0 && I % 256 == 0 && up_bytes < ((int64_t)1 << 31) && down_bytes < ((int64_t)1 << 31)) {
      // z: an expert's 16-token tiles side by side (an expert holds at most T
      // tokens; slices past its count exit at once), so a crowded expert does
      // not serialize its tiles
      const unsigned zt = (unsigned)std::min((T + 15) / 16, 8);
      if (QT == kQ4_K && xbf16 && H <= 4096) {
        // one workgroup per CU, the routed work split evenly over them
        hipLaunchKernelGGL(moe_up_mfp_kernel, dim3((unsigned)device_cus()), dim3(512), 0, s, wg, wu,
                           static_cast<const uint16_t*>(x), H, I, E, ws);
      } else if (xbf16)
        hipLaunchKernelGGL((moe_up_mfma_kernel<QT, true>), dim3((unsigned)(I / 16), (unsigned)E, zt), dim3(256), 0, s,
                           wg, wu, x, H, I, ws);
      else
        hipLaunchKernelGGL((moe_up_mfma_kernel<QT, false>), dim3((unsigned)(I / 16), (unsigned)E, zt), dim3(256), 0, s,
                           wg, wu, x, H, I, ws);
      if (int rc = check_launch("moe_up_mfma")) return rc;
      if constexpr (QT == kQ4_K) {
        // down split along K over one workgroup per CU, then the ordered split sums in the combine
        hipLaunchKernelGGL(moe_down_mfl_kernel, dim3((unsigned)device_cus()), dim3(512), 0, s, wd, H, I, E, ws);
        if (int rc = check_launch("moe_down_mfl")) return rc;
        hipLaunchKernelGGL(moe_combine_split_kernel, dim3((unsigned)((H / 4 + 255) / 256), (unsigned)T), dim3(256), 0,
                           s, y, H, k, moe_down_splits(I), ws);
        return check_launch("moe_combine");
      }
      hipLaunchKernelGGL((moe_down_mfma_kernel<QT, 4>), dim3((unsigned)(H / 64), (unsigned)E, zt), dim3(256), 0, s, wd,
                         H, I, ws);
      if (int rc = check_launch("moe_down_mfma")) return rc;
      hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((H + 255) / 256), (unsigned)T), dim3(256), 0, s, y,
                         H, k, ws);
      return check_launch("moe_combine");
    }
  }
  const dim3 gup((unsigned)((I + 4 * R - 1) / (4 * R)), (unsigned)E);
  if (xbf16)
    hipLaunchKernelGGL((moe_up_kernel<QT, true, R>), gup, dim3(256), 0, s, wg, wu, x, H, I, ws);
  else
    hipLaunchKernelGGL((moe_up_kernel<QT, false, R>), gup, dim3(256), 0, s, wg, wu, x, H, I, ws);
  if (int rc = check_launch("moe_up")) return rc;
  const dim3 gdown((unsigned)((H + 4 * R - 1) / (4 * R)), (unsigned)E);
  hipLaunchKernelGGL((moe_down_kernel<QT, R>), gdown, dim3(256), 0, s, wd, H, I, ws);
  if (int rc = check_launch("moe_down")) return rc;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((H + 255) / 256), (unsigned)T), dim3(256), 0, s, y, H,
                     k, ws);
  return check_launch("moe_combine");
}

}  // namespace draco

using namespace draco;

extern "C" size_t draco_gguf_moe_workspace_size(int64_t tokens, int64_t hidden, int64_t inter, int n_experts,
                                                int top_k) {
  if (tokens < 1 || hidden < 1 || inter < 1 || n_experts < 1 || top_k < 1) return 0;
  return moe_ws_layout(tokens, hidden, inter, n_experts, top_k, nullptr, nullptr);
}

extern "C" int draco_gguf_moe_ffn(int ggml_type, const void* const* w_gate, const void* const* w_up,
                                  const void* const* w_down, size_t expert_w_bytes, const float* router_logits,
                                  const void* x, int x_dtype, float* y, int64_t tokens, int64_t hidden, int64_t inter,
                                  int n_experts, int top_k, void* workspace, size_t workspace_bytes, void* stream) {
  int qk = 0, bb = 0;
  if (int rc = draco_gguf_block_info(ggml_type, &qk, &bb)) return rc;
  if (ggml_type & DRACO_GGUF_GGML_ORDER)
    return set_error(DRACO_EINVAL_QTYPE, "MoE experts take reference-layout blocks only");
  if (n_experts < 1 || n_experts > kMaxExperts)
    return set_error(DRACO_EINVAL_SHAPE, "n_experts must be in 1..%d, got %d", kMaxExperts, n_experts);
  if (top_k < 1 || top_k > kMaxTopK || top_k > n_experts)
    return set_error(DRACO_EINVAL_SHAPE, "top_k must be in 1..min(%d, n_experts), got %d", kMaxTopK, top_k);
  if (tokens < 1 || tokens * top_k > (1 << 30) || hidden < 1 || inter < 1 || hidden > (1 << 30) ||
      inter > (1 << 30))
    return set_error(DRACO_EINVAL_SHAPE, "invalid MoE dims tokens=%lld hidden=%lld inter=%lld",
                     (long long)tokens, (long long)hidden, (long long)inter);
  if (hidden % qk || inter % qk)
    return set_error(DRACO_EINVAL_SHAPE, "hidden (%lld) and inter (%lld) must be multiples of the block size %d",
                     (long long)hidden, (long long)inter, qk);
  const uint64_t need_w = (uint64_t)(inter * (hidden / qk)) * (uint64_t)bb;
  if (expert_w_bytes < need_w)
    return set_error(DRACO_EINVAL_SHAPE, "expert weights hold %zu bytes, [%lld, %lld] needs %llu", expert_w_bytes,
                     (long long)inter, (long long)hidden, (unsigned long long)need_w);
  if (x_dtype != DRACO_DTYPE_F32 && x_dtype != DRACO_DTYPE_BF16)
    return set_error(DRACO_EINVAL_ARG, "unknown activation dtype %d", x_dtype);
  if (!w_gate || !w_up || !w_down) return set_error(DRACO_EINVAL_ARG, "expert pointer arrays must not be NULL");
  auto bad = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) != 0; };
  if (bad(router_logits) || bad(x) || bad(y) || bad(workspace))
    return set_error(DRACO_EINVAL_ARG, "router_logits, x, y and workspace must be non-NULL and 16-byte aligned");
  ExpertPtrs wg{}, wu{}, wd{};
  for (int e = 0; e < n_experts; ++e) {
    if (bad(w_gate[e]) || bad(w_up[e]) || bad(w_down[e]))
      return set_error(DRACO_EINVAL_ARG, "expert %d weight pointer is NULL or misaligned", e);
    wg.p[e] = static_cast<const uint8_t*>(w_gate[e]);
    wu.p[e] = static_cast<const uint8_t*>(w_up[e]);
    wd.p[e] = static_cast<const uint8_t*>(w_down[e]);
  }
  MoeWs ws;
  const size_t need = moe_ws_layout(tokens, hidden, inter, n_experts, top_k, static_cast<char*>(workspace), &ws);
  if (workspace_bytes < need)
    return set_error(DRACO_EWORKSPACE, "MoE workspace needs %zu bytes, got %zu", need, workspace_bytes);
  const bool xbf16 = x_dtype == DRACO_DTYPE_BF16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int T = (int)tokens, H = (int)hidden, I = (int)inter;
  switch (ggml_type) {
    case kQ8_0: return launch_moe<kQ8_0>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ4_0: return launch_moe<kQ4_0>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ4_1: return launch_moe<kQ4_1>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ5_0: return launch_moe<kQ5_0>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ5_1: return launch_moe<kQ5_1>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ8_K: return launch_moe<kQ8_K>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ2_K: return launch_moe<kQ2_K>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ3_K: return launch_moe<kQ3_K>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ4_K: return launch_moe<kQ4_K>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ5_K: return launch_moe<kQ5_K>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    case kQ6_K: return launch_moe<kQ6_K>(wg, wu, wd, router_logits, x, xbf16, y, T, H, I, n_experts, top_k, ws, s);
    default: return set_error(DRACO_EINVAL_QTYPE, "unsupported ggml type %d", ggml_type);
  }
}
