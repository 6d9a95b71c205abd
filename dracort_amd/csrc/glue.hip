// Decode-step glue on gfx950: RMSNorm and single-token attention over a
// float16 KV cache (RoPE and the cache append fused in).
//
// RMSNorm replaces rms_norm (draco/runtime/cpu/ops.py:15-19): one workgroup
// per row, float32 sum of squares, y = x / sqrt(mean(x^2) + eps) * w written as
// float32 and / or bfloat16 (the decode GEMVs' input).
//
// Decode attention replaces CPUAttentionBackend.decode -> prefill with one
// query (draco/runtime/cpu/attention.py:35-81) plus apply_rope
// (draco/runtime/cpu/ops.py:73-92) on q and k:
//   * cache layout [batch][kv head][position][head_dim] float16 (head-major:
//     a head's keys are consecutive, so a workgroup's key reads are
//     contiguous); position p of sequence b holds token p;
//   * grid (split, kv head, sequence) of one-wave workgroups: a wave takes
//     32 consecutive positions (more, in steps of 32, only when the cache
//     holds over 32768) of one kv head for the G = Hq / Hkv query heads that
//     share it (GQA) and writes its partial softmax state (max, sum of
//     exponentials, weighted value sum) per query head;
//   * RoPE reads the cos / sin tables the reference builds (build_rope_cache,
//     [max_positions][head_dim / 2] float32) at the token's position;
//   * the new token's k / v are rotated, rounded to float16 and used directly
//     by the workgroup whose range holds their position, which also stores
//     them in the cache (no other workgroup reads that position);
//   * only the waves whose range holds keys (positions 0 .. p) do any work;
//     a second launch, one workgroup per (sequence, query head), merges their
//     partial states (max over the splits, rescaled sums) and writes the
//     output.
//
// Shapes outside the fast kernels' set (head_dim other than 64 / 128, or a
// query-head group other than 1, 2, 4 or 8: small test models, unusual GQA
// ratios) run decode_attention_generic_kernel instead: one workgroup per
// (query head, sequence) in three passes over the cached positions -- scores
// into the workspace, exponentials and their sum, then the weighted value sum
// -- with the same RoPE, float16 rounding of the new key / value and cache
// store as the fast kernels.
#include <math.h>

#include "draco_internal.h"
#include "gemv_core.h"

namespace draco {

// Max over the 64 lanes, result in every lane (DPP within rows of 16, then two exchanges).
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// Sum over aligned groups of N (8 or 16) lanes, result in every lane of the group.
template <int N>
__device__ __forceinline__ float group_sum_dpp(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  if constexpr (N == 16) v += dpp_f<0x140>(v);
  return v;
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// One row per workgroup.  NV > 0: the row (n <= 1024 NV) is loaded in one
// batch into registers (every load in flight at once); NV = 0: any n, in a loop.
template <int NV>
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       float eps, float* __restrict__ y, uint16_t* __restrict__ yb,
                                                       int n) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * n;
  auto emit = [&](int i, float4 v, float denom) {
    const float4 g = *reinterpret_cast<const float4*>(w + i);
    const float4 o = make_float4(v.x / denom * g.x, v.y / denom * g.y, v.z / denom * g.z, v.w / denom * g.w);
    const size_t at = (size_t)blockIdx.x * n + i;
    if (y) *reinterpret_cast<float4*>(y + at) = o;
    if (yb) {
      const uint32_t lo = f32_to_bf16_bits(o.x) | ((uint32_t)f32_to_bf16_bits(o.y) << 16);
      const uint32_t hi = f32_to_bf16_bits(o.z) | ((uint32_t)f32_to_bf16_bits(o.w) << 16);
      *reinterpret_cast<uint2*>(yb + at) = make_uint2(lo, hi);
    }
  };
  if constexpr (NV > 0) {
    float4 v[NV];
    float ss = 0.f;
#pragma unroll
    for (int r = 0; r < NV; ++r) {
      const int i = threadIdx.x * 4 + 1024 * r;
      v[r] = i < n ? *reinterpret_cast<const float4*>(xr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int r = 0; r < NV; ++r) ss += v[r].x * v[r].x + v[r].y * v[r].y + v[r].z * v[r].z + v[r].w * v[r].w;
    const float denom = sqrtf(block_sum_256(ss, red) / (float)n + eps);
#pragma unroll
    for (int r = 0; r < NV; ++r) {
      const int i = threadIdx.x * 4 + 1024 * r;
      if (i < n) emit(i, v[r], denom);
    }
  } else {
    float ss = 0.f;
    for (int i = threadIdx.x * 4; i < n; i += 1024) {
      const float4 v = *reinterpret_cast<const float4*>(xr + i);
      ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    const float denom = sqrtf(block_sum_256(ss, red) / (float)n + eps);
    for (int i = threadIdx.x * 4; i < n; i += 1024) emit(i, *reinterpret_cast<const float4*>(xr + i), denom);
  }
}

int rms_norm_launch(const float* x, const float* w, float eps, float* y, uint16_t* yb, int64_t m, int64_t n,
                    hipStream_t s) {
  if (n <= 4096)
    hipLaunchKernelGGL(rms_norm_kernel<4>, dim3((unsigned)m), dim3(256), 0, s, x, w, eps, y, yb, (int)n);
  else if (n <= 16384)
    hipLaunchKernelGGL(rms_norm_kernel<16>, dim3((unsigned)m), dim3(256), 0, s, x, w, eps, y, yb, (int)n);
  else
    hipLaunchKernelGGL(rms_norm_kernel<0>, dim3((unsigned)m), dim3(256), 0, s, x, w, eps, y, yb, (int)n);
  return check_launch("rms_norm");
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
constexpr int kAttnKeys = 32;     // positions per wave and step
constexpr int kMaxSplits = 1024;  // wave splits per (sequence, kv head)
constexpr int kMaxGroup = 8;      // query heads per kv head (1, 2, 4 or 8)
constexpr int kMaxPositions = 1 << 17;

struct AttnArgs {
  const float* q;          // [B, Hq * D]
  const float* k;          // [B, Hkv * D]
  const float* v;          // [B, Hkv * D]
  uint16_t* kc;            // [B, Hkv, P, D] float16
  uint16_t* vc;
  const int* positions;    // [B]
  void* out;               // [B, Hq * D] float32 or bfloat16
  float* part;             // [B, Hkv, S, G, D + 4] partial softmax states: m, l, 0, 0, o[D]
  const float* cos_t;      // [P, D / 2] RoPE tables, NULL: no rotation
  const float* sin_t;
  int hq, hkv, max_pos;
  int splits;              // waves per (sequence, kv head)
  int steps;               // kAttnKeys-position steps per wave
  float scale;
  int out_bf16;
};

// The split geometry for a cache of max_pos positions: each wave takes
// `steps` consecutive runs of kAttnKeys positions, at most kMaxSplits waves.
struct AttnSplit {
  int steps, splits;
};
inline AttnSplit attn_split(int64_t max_pos) {
  const int64_t runs = (max_pos + kAttnKeys - 1) / kAttnKeys;
  const int steps = (int)((runs + kMaxSplits - 1) / kMaxSplits);
  return {steps, (int)((runs + steps - 1) / steps)};
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Sum over the lanes that share a lane index modulo LK (the key slots of a
// wave), result in every lane.
template <int LK>
__device__ __forceinline__ float slot_sum(float v) {
#pragma unroll
  for (int m = LK; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}
template <int LK>
__device__ __forceinline__ float slot_max(float v) {
#pragma unroll
  for (int m = LK; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ void f16x8_to_f32(const uint4 w, float (&f)[8]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = f16_to_f32((uint16_t)(ws[e] & 0xFFFFu));
    f[2 * e + 1] = f16_to_f32((uint16_t)(ws[e] >> 16));
  }
}

// One wave per workgroup; grid (split, kv head, sequence).  The wave takes
// positions [split * steps * 32, +steps * 32) of (sequence, kv head) for its G
// query heads.  Lane mapping per 16-byte load: LK = D / 8 lanes per key (8
// dimensions each), 64 / LK keys per load, NPW loads per lane cover 32 keys;
// every key and value load of a step is issued before any math.  Scores are
// summed over a key's LK lanes with DPP (every lane of the key holds it),
// softmax statistics over the wave's keys with lane exchanges, and the value
// sums are accumulated per lane over its key slot, rescaled across steps
// (online softmax) and summed over the slots at the end.  No workgroup
// barrier anywhere: a wave with no keys returns at once.
template <int D, int G>
__global__ __launch_bounds__(64) void decode_attention_kernel(AttnArgs a) {
  constexpr int HALF = D / 2;
  constexpr int LK = D / 8;
  constexpr int KPL = 64 / LK;
  constexpr int NPW = kAttnKeys / KPL;
  __shared__ float qs[G][D];  // rotated queries of the group
  __shared__ float kn[D];     // the new token's rotated key (float16-rounded)
  __shared__ float vn[D];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int pos = a.positions[b];
  const bool valid = pos >= 0 && pos < a.max_pos;  // else no cache access; the output is NaN
  const int n_keys = valid ? pos + 1 : 0;
  const int span = kAttnKeys * a.steps;
  const int j0 = split * span;
  if (j0 >= n_keys) return;
  const int jend = min(j0 + span, n_keys);
  const size_t head = ((size_t)b * a.hkv + h) * (size_t)a.max_pos * D;
  const int dl = lane % LK, slot = lane / LK;

  // the query (and new key / value) elements and RoPE factors first: they
  // come from L2 and are rotated while the cache loads are in flight
  constexpr int QE = (G * HALF + 63) / 64;  // (g, i) pairs per lane
  float q1[QE], q2[QE], qc[QE], qn[QE];
  const float* qb = a.q + (size_t)b * a.hq * D + (size_t)h * G * D;
#pragma unroll
  for (int u = 0; u < QE; ++u) {
    const int e = min(lane + 64 * u, G * HALF - 1);
    const int g = e / HALF, i = e - g * HALF;
    q1[u] = qb[g * D + i];
    q2[u] = qb[g * D + i + HALF];
    qc[u] = a.cos_t ? a.cos_t[(size_t)pos * HALF + i] : 1.f;
    qn[u] = a.cos_t ? a.sin_t[(size_t)pos * HALF + i] : 0.f;
  }
  const bool owner = pos >= j0 && pos < jend;
  const int io = min(lane, HALF - 1);
  float k1 = 0.f, k2 = 0.f, v1 = 0.f, v2 = 0.f;
  if (owner) {
    const float* kp = a.k + ((size_t)b * a.hkv + h) * D;
    const float* vp = a.v + ((size_t)b * a.hkv + h) * D;
    k1 = kp[io];
    k2 = kp[io + HALF];
    v1 = vp[io];
    v2 = vp[io + HALF];
  }
  uint4 kw[NPW], vw[NPW];
#pragma unroll
  for (int r = 0; r < NPW; ++r) {
    const int jj = slot + KPL * r;
    const size_t at = head + (size_t)(j0 + (j0 + jj < jend ? jj : 0)) * D + 8 * dl;
    kw[r] = *reinterpret_cast<const uint4*>(a.kc + at);
    vw[r] = *reinterpret_cast<const uint4*>(a.vc + at);
  }
#pragma unroll
  for (int u = 0; u < QE; ++u) {
    const int e = lane + 64 * u;
    if (e < G * HALF) {
      const int g = e / HALF, i = e - g * HALF;
      qs[g][i] = q1[u] * qc[u] - q2[u] * qn[u];
      qs[g][i + HALF] = q2[u] * qc[u] + q1[u] * qn[u];
    }
  }
  if (owner && lane < HALF) {
    // (x1, x2) -> (x1 c - x2 s, x2 c + x1 s), the reference's apply_rope pair
    // (ops.py:82-92), then the float16 cache dtype
    const float c = qc[0], sn = qn[0];  // lane < HALF: pair i = lane, the same factors as q's
    const uint16_t kh1 = f32_to_f16(k1 * c - k2 * sn), kh2 = f32_to_f16(k2 * c + k1 * sn);
    const uint16_t vh1 = f32_to_f16(v1), vh2 = f32_to_f16(v2);
    kn[lane] = f16_to_f32(kh1);
    kn[lane + HALF] = f16_to_f32(kh2);
    vn[lane] = f16_to_f32(vh1);
    vn[lane + HALF] = f16_to_f32(vh2);
    a.kc[head + (size_t)pos * D + lane] = kh1;
    a.kc[head + (size_t)pos * D + lane + HALF] = kh2;
    a.vc[head + (size_t)pos * D + lane] = vh1;
    a.vc[head + (size_t)pos * D + lane + HALF] = vh2;
  }
  __syncthreads();  // one wave: orders the LDS writes before the reads
  float qr[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) qr[g][e] = qs[g][8 * dl + e];

  float m[G], l[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  }
  for (int js = j0;;) {
    const int jn = min(kAttnKeys, jend - js);  // keys of this step
    float s[G][NPW];
#pragma unroll
    for (int r = 0; r < NPW; ++r) {
      const int jj = slot + KPL * r;
      float kv[8];
      if (js + jj == pos) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kv[e] = kn[8 * dl + e];
      } else {
        f16x8_to_f32(kw[r], kv);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dot = fmaf(qr[g][e], kv[e], dot);
        dot = group_sum_dpp<LK>(dot);
        s[g][r] = jj < jn ? dot * a.scale : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = s[g][0];
#pragma unroll
      for (int r = 1; r < NPW; ++r) mx = fmaxf(mx, s[g][r]);
      const float mn = fmaxf(m[g], slot_max<LK>(mx));
      const float corr = expf(m[g] - mn);  // 0 on the first step
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < NPW; ++r) {
        s[g][r] = expf(s[g][r] - mn);
        ps += s[g][r];
      }
      l[g] = l[g] * corr + slot_sum<LK>(ps);  // one lane per key slot in each exchange
      m[g] = mn;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= corr;
    }
#pragma unroll
    for (int r = 0; r < NPW; ++r) {
      const int jj = slot + KPL * r;
      float vv[8];
      if (js + jj == pos) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vv[e] = vn[8 * dl + e];
      } else {
        f16x8_to_f32(vw[r], vv);
      }
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(s[g][r], vv[e], o[g][e]);
    }
    js += kAttnKeys;
    if (js >= jend) break;
#pragma unroll
    for (int r = 0; r < NPW; ++r) {
      const int jj = slot + KPL * r;
      const size_t at = head + (size_t)(js + (js + jj < jend ? jj : 0)) * D + 8 * dl;
      kw[r] = *reinterpret_cast<const uint4*>(a.kc + at);
      vw[r] = *reinterpret_cast<const uint4*>(a.vc + at);
    }
  }
  // value sums over the key slots; slot 0's lanes write the partial state
  float* part = a.part + (((size_t)b * a.hkv + h) * a.splits + split) * G * (D + 4);
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = slot_sum<LK>(o[g][e]);
    if (slot == 0) {
      float4* dst = reinterpret_cast<float4*>(part + g * (D + 4) + 4 + 8 * dl);
      dst[0] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
      dst[1] = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
      if (dl == 0) *reinterpret_cast<float4*>(part + g * (D + 4)) = make_float4(m[g], l[g], 0.f, 0.f);
    }
  }
}

// Merges the partial states of the `used` waves of one query head of
// sequence b (a second launch: the kernel boundary makes the partials
// visible).  Grid (query head, sequence).  Thread t takes dimensions
// 4 (t % (D / 4)) .. + 3 of the splits s = t / (D / 4) (mod the phases) and
// merges them as it loads them (running max, rescaled sums), so every load
// of the launch is issued at once; the phases meet in LDS.
template <int D, int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(AttnArgs a) {
  constexpr int TQ = D / 4;      // threads per split row (float4 each)
  constexpr int NPH = 256 / TQ;  // split phases
  __shared__ float pm[NPH], pl[NPH];
  __shared__ float4 acc[NPH][TQ];
  const int qh = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int h = qh / G, g = qh - h * G;
  const int pos = a.positions[b];
  const bool valid = pos >= 0 && pos < a.max_pos;
  const int span = kAttnKeys * a.steps;
  const int used = valid ? (pos + span) / span : 0;
  const size_t stride = (size_t)G * (D + 4);
  const float* base = a.part + (((size_t)b * a.hkv + h) * a.splits * G + g) * (D + 4);
  const int dq = t % TQ, ph = t / TQ;
  float M = -INFINITY, L = 0.f;
  float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
  for (int sp = ph; sp < used; sp += NPH) {
    const float* p = base + sp * stride;
    const float2 ml = *reinterpret_cast<const float2*>(p);
    const float4 o4 = *reinterpret_cast<const float4*>(p + 4 + 4 * dq);
    const float mn = fmaxf(M, ml.x);
    const float co = expf(M - mn), cn = expf(ml.x - mn);
    L = fmaf(L, co, ml.y * cn);
    s4.x = fmaf(s4.x, co, o4.x * cn);
    s4.y = fmaf(s4.y, co, o4.y * cn);
    s4.z = fmaf(s4.z, co, o4.z * cn);
    s4.w = fmaf(s4.w, co, o4.w * cn);
    M = mn;
  }
  if (dq == 0) {
    pm[ph] = M;
    pl[ph] = L;
  }
  acc[ph][dq] = s4;
  __syncthreads();
  if (t < D) {
    float mg = pm[0];
#pragma unroll
    for (int p = 1; p < NPH; ++p) mg = fmaxf(mg, pm[p]);
    const int q4 = t / 4, c = t & 3;
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int p = 0; p < NPH; ++p) {
      const float w = pm[p] == -INFINITY ? 0.f : expf(pm[p] - mg);  // a phase without splits weighs 0
      const float4 v = acc[p][q4];
      num = fmaf(c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w, w, num);
      den = fmaf(pl[p], w, den);
    }
    const float r = valid ? num / den : __builtin_nanf("");
    const size_t at = (size_t)b * a.hq * D + (size_t)qh * D + t;
    if (a.out_bf16)
      static_cast<uint16_t*>(a.out)[at] = f32_to_bf16_bits(r);
    else
      static_cast<float*>(a.out)[at] = r;
  }
}

__device__ __forceinline__ float block_max_256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Any even head_dim D <= 256 and any group G = Hq / Hkv.  Workgroup (query
// head qh, sequence b), 256 threads; a.part holds this workgroup's scores,
// [B][Hq][max_pos] floats.  Every workgroup of kv head qh / G rotates the new
// key itself (the same arithmetic as the fast kernel, so the same bits) and
// uses it for position pos; the group's first query head stores k / v.
__global__ __launch_bounds__(256) void decode_attention_generic_kernel(AttnArgs a, int D, int G) {
  __shared__ float qs[256], kn[256], vn[256], acc[256];
  __shared__ float red[4];
  const int qh = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int h = qh / G, HALF = D / 2;
  const int pos = a.positions[b];
  const size_t at = (size_t)b * a.hq * D + (size_t)qh * D;
  if (pos < 0 || pos >= a.max_pos) {  // no cache access; NaN output (uniform branch)
    if (t < D) {
      if (a.out_bf16)
        static_cast<uint16_t*>(a.out)[at + t] = 0x7FC0u;
      else
        static_cast<float*>(a.out)[at + t] = __builtin_nanf("");
    }
    return;
  }
  const size_t head = ((size_t)b * a.hkv + h) * (size_t)a.max_pos * D;
  if (t < HALF) {
    const float c = a.cos_t ? a.cos_t[(size_t)pos * HALF + t] : 1.f;
    const float sn = a.cos_t ? a.sin_t[(size_t)pos * HALF + t] : 0.f;
    const float* qp = a.q + at;
    const float q1 = qp[t], q2 = qp[t + HALF];
    qs[t] = q1 * c - q2 * sn;
    qs[t + HALF] = q2 * c + q1 * sn;
    const float* kp = a.k + ((size_t)b * a.hkv + h) * D;
    const float* vp = a.v + ((size_t)b * a.hkv + h) * D;
    const float k1 = kp[t], k2 = kp[t + HALF];
    const uint16_t kh1 = f32_to_f16(k1 * c - k2 * sn), kh2 = f32_to_f16(k2 * c + k1 * sn);
    const uint16_t vh1 = f32_to_f16(vp[t]), vh2 = f32_to_f16(vp[t + HALF]);
    kn[t] = f16_to_f32(kh1);
    kn[t + HALF] = f16_to_f32(kh2);
    vn[t] = f16_to_f32(vh1);
    vn[t + HALF] = f16_to_f32(vh2);
    if (qh % G == 0) {
      a.kc[head + (size_t)pos * D + t] = kh1;
      a.kc[head + (size_t)pos * D + t + HALF] = kh2;
      a.vc[head + (size_t)pos * D + t] = vh1;
      a.vc[head + (size_t)pos * D + t + HALF] = vh2;
    }
  }
  __syncthreads();
  float* sc = a.part + ((size_t)b * a.hq + qh) * (size_t)a.max_pos;
  // 1. scores q . k / sqrt(D) of positions 0 .. pos
  float mx = -INFINITY;
  for (int j = t; j <= pos; j += 256) {
    float sj = 0.f;
    if (j == pos) {
      for (int d = 0; d < D; ++d) sj = fmaf(qs[d], kn[d], sj);
    } else {
      const uint16_t* kr = a.kc + head + (size_t)j * D;
      for (int d = 0; d < D; ++d) sj = fmaf(qs[d], f16_to_f32(kr[d]), sj);
    }
    sj *= a.scale;
    sc[j] = sj;
    mx = fmaxf(mx, sj);
  }
  mx = block_max_256(mx, red);
  // 2. exponentials and their sum (each thread rewrites only its own scores)
  float sum = 0.f;
  for (int j = t; j <= pos; j += 256) {
    const float e = expf(sc[j] - mx);
    sc[j] = e;
    sum += e;
  }
  sum = block_sum_256(sum, red);  // its barriers also order the score writes before pass 3
  // 3. weighted value sums: thread group g = t / D takes positions g, g + NG, ...
  const int NG = 256 / D, g = t / D, d = t - g * D;
  float o = 0.f;
  if (g < NG) {
    for (int j = g; j <= pos; j += NG) {
      const float vj = j == pos ? vn[d] : f16_to_f32(a.vc[head + (size_t)j * D + d]);
      o = fmaf(sc[j], vj, o);
    }
  }
  acc[t] = o;
  __syncthreads();
  if (t < D) {
    float tot = 0.f;
    for (int gg = 0; gg < NG; ++gg) tot += acc[gg * D + t];
    const float r = tot / sum;
    if (a.out_bf16)
      static_cast<uint16_t*>(a.out)[at + t] = f32_to_bf16_bits(r);
    else
      static_cast<float*>(a.out)[at + t] = r;
  }
}

// The fast kernels take head_dim 64 / 128 with 1, 2, 4 or 8 query heads per kv head.
inline bool attn_fast_shape(int hq, int hkv, int head_dim) {
  const int g = hq / hkv;
  return (head_dim == 64 || head_dim == 128) && g <= kMaxGroup && (g & (g - 1)) == 0;
}

size_t decode_attention_ws(int64_t batch, int hq, int hkv, int head_dim, int64_t max_pos) {
  if (!attn_fast_shape(hq, hkv, head_dim)) return (size_t)batch * hq * max_pos * sizeof(float);
  const AttnSplit sp = attn_split(max_pos);
  return (size_t)batch * hkv * sp.splits * (hq / hkv) * (head_dim + 4) * sizeof(float);
}

int decode_attention_launch(const float* q, const float* k, const float* v, uint16_t* kc, uint16_t* vc,
                            const int* positions, int64_t batch, int hq, int hkv, int head_dim, int64_t max_pos,
                            const float* cos_t, const float* sin_t, void* out, int out_bf16, void* workspace,
                            hipStream_t s) {
  AttnArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.kc = kc;
  a.vc = vc;
  a.positions = positions;
  a.out = out;
  a.part = static_cast<float*>(workspace);
  a.hq = hq;
  a.hkv = hkv;
  a.max_pos = (int)max_pos;
  const AttnSplit sp = attn_split(max_pos);
  a.splits = sp.splits;
  a.steps = sp.steps;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.scale = (float)(1.0 / sqrt((double)head_dim));
  a.out_bf16 = out_bf16;
  const int g = hq / hkv;
  if (!attn_fast_shape(hq, hkv, head_dim)) {
    hipLaunchKernelGGL(decode_attention_generic_kernel, dim3((unsigned)hq, (unsigned)batch), dim3(256), 0, s, a,
                       head_dim, g);
    return check_launch("decode_attention_generic");
  }
  const dim3 grid((unsigned)a.splits, (unsigned)hkv, (unsigned)batch);
  const dim3 mgrid((unsigned)hq, (unsigned)batch);
#define DRACO_ATTN_LAUNCH(D_, G_)                                                                \
  hipLaunchKernelGGL((decode_attention_kernel<D_, G_>), grid, dim3(64), 0, s, a);               \
  if (int rc = check_launch("decode_attention")) return rc;                                    \
  hipLaunchKernelGGL((decode_merge_kernel<D_, G_>), mgrid, dim3(256), 0, s, a)
  if (head_dim == 128) {
    switch (g) {
      case 1: DRACO_ATTN_LAUNCH(128, 1); break;
      case 2: DRACO_ATTN_LAUNCH(128, 2); break;
      case 4: DRACO_ATTN_LAUNCH(128, 4); break;
      case 8: DRACO_ATTN_LAUNCH(128, 8); break;
      default: return set_error(DRACO_EINVAL_SHAPE, "query heads per kv head must be 1, 2, 4 or 8, got %d", g);
    }
  } else {
    switch (g) {
      case 1: DRACO_ATTN_LAUNCH(64, 1); break;
      case 2: DRACO_ATTN_LAUNCH(64, 2); break;
      case 4: DRACO_ATTN_LAUNCH(64, 4); break;
      case 8: DRACO_ATTN_LAUNCH(64, 8); break;
      default: return set_error(DRACO_EINVAL_SHAPE, "query heads per kv head must be 1, 2, 4 or 8, got %d", g);
    }
  }
#undef DRACO_ATTN_LAUNCH
  return check_launch("decode_attention_merge");
}

}  // namespace draco

using namespace draco;

extern "C" {

int draco_gguf_rms_norm(const float* x, const float* weight, float eps, float* y, void* y_bf16, int64_t m, int64_t n,
                        void* stream) {
  if (m < 1 || m > ((int64_t)1 << 30) || n < 4 || n % 4 != 0 || n > ((int64_t)1 << 30))
    return set_error(DRACO_EINVAL_SHAPE, "rms_norm needs m >= 1 rows of n (multiple of 4) elements, got [%lld, %lld]",
                     (long long)m, (long long)n);
  auto bad = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) != 0; };
  if (bad(x) || bad(weight)) return set_error(DRACO_EINVAL_ARG, "x and weight must be non-NULL and 16-byte aligned");
  if (!y && !y_bf16) return set_error(DRACO_EINVAL_ARG, "rms_norm needs y and / or y_bf16");
  if ((y && bad(y)) || (y_bf16 && (reinterpret_cast<uintptr_t>(y_bf16) & 7u)))
    return set_error(DRACO_EINVAL_ARG, "y must be 16-byte and y_bf16 8-byte aligned");
  if (!(eps >= 0.f)) return set_error(DRACO_EINVAL_ARG, "eps must be >= 0");
  return rms_norm_launch(x, weight, eps, y, static_cast<uint16_t*>(y_bf16), m, n, static_cast<hipStream_t>(stream));
}

size_t draco_gguf_decode_attention_workspace_size(int64_t batch, int n_q_heads, int n_kv_heads, int head_dim,
                                                  int64_t max_positions) {
  if (batch < 1 || n_kv_heads < 1 || n_q_heads < n_kv_heads || n_q_heads % n_kv_heads || head_dim < 1 ||
      max_positions < 1)
    return 0;
  return decode_attention_ws(batch, n_q_heads, n_kv_heads, head_dim, max_positions);
}

int draco_gguf_decode_attention(const float* q, const float* k, const float* v, void* k_cache, void* v_cache,
                                const int32_t* positions, int64_t batch, int n_q_heads, int n_kv_heads, int head_dim,
                                int64_t max_positions, const float* rope_cos, const float* rope_sin, void* out,
                                int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 1 || batch > 65535 || n_kv_heads < 1 || n_q_heads > 65535 || n_q_heads < n_kv_heads ||
      n_q_heads % n_kv_heads)
    return set_error(DRACO_EINVAL_SHAPE,
                     "decode attention needs 1 <= batch <= 65535 and n_q_heads (<= 65535) a multiple of n_kv_heads; "
                     "got batch %lld, %d / %d heads",
                     (long long)batch, n_q_heads, n_kv_heads);
  if (head_dim < 2 || head_dim > 256 || head_dim % 2)
    return set_error(DRACO_EINVAL_SHAPE, "decode attention takes an even head_dim of 2..256, got %d", head_dim);
  if (max_positions < 1 || max_positions * head_dim * (int64_t)n_kv_heads * batch > ((int64_t)1 << 40) ||
      max_positions > kMaxPositions)
    return set_error(DRACO_EINVAL_SHAPE, "invalid max_positions %lld", (long long)max_positions);
  if ((rope_cos == nullptr) != (rope_sin == nullptr))
    return set_error(DRACO_EINVAL_ARG, "rope_cos and rope_sin must both be given or both be NULL");
  if (out_dtype != DRACO_DTYPE_F32 && out_dtype != DRACO_DTYPE_BF16)
    return set_error(DRACO_EINVAL_ARG, "unknown output dtype %d", out_dtype);
  auto bad = [](const void* p, uintptr_t a) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & (a - 1)) != 0; };
  if (bad(q, 4) || bad(k, 4) || bad(v, 4) || bad(positions, 4) || bad(out, 4) ||
      (rope_cos && (bad(rope_cos, 4) || bad(rope_sin, 4))))
    return set_error(DRACO_EINVAL_ARG, "q, k, v, positions and out must be non-NULL and 4-byte aligned");
  if (bad(k_cache, 16) || bad(v_cache, 16) || bad(workspace, 256))
    return set_error(DRACO_EINVAL_ARG, "caches must be 16-byte and the workspace 256-byte aligned");
  const size_t need = decode_attention_ws(batch, n_q_heads, n_kv_heads, head_dim, max_positions);
  if (workspace_bytes < need)
    return set_error(DRACO_EWORKSPACE, "decode attention workspace needs %zu bytes, got %zu", need, workspace_bytes);
  return decode_attention_launch(q, k, v, static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                                 positions, batch, n_q_heads, n_kv_heads, head_dim, max_positions, rope_cos, rope_sin,
                                 out, out_dtype == DRACO_DTYPE_BF16, workspace, static_cast<hipStream_t>(stream));
}

}  // extern "C"
