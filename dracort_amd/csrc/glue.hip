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
//   * grid (split, kv head, sequence): a workgroup takes 256 consecutive
//     positions of one kv head for the G = Hq / Hkv query heads that share it
//     (GQA), one key per thread, and writes its partial softmax state (max,
//     sum of exponentials, weighted value sum) per query head;
//   * RoPE reads the cos / sin tables the reference builds (build_rope_cache,
//     [max_positions][head_dim / 2] float32) at the token's position;
//   * the new token's k / v are rotated, rounded to float16 and used directly
//     by the workgroup whose range holds their position, which also stores
//     them in the cache (no other workgroup reads that position);
//   * only the workgroups whose range holds keys (positions 0 .. p) do any
//     work; a second launch, one workgroup per (sequence, kv head), merges
//     their partial states (max over the splits, rescaled sums) and writes the
//     output.
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
constexpr int kAttnChunk = 256;  // positions per workgroup
constexpr int kMaxSplits = 512;  // splits per (sequence, kv head): max_positions <= 131072
constexpr int kMaxGroup = 8;     // query heads per kv head (1, 2, 4 or 8)

struct AttnArgs {
  const float* q;          // [B, Hq * D]
  const float* k;          // [B, Hkv * D]
  const float* v;          // [B, Hkv * D]
  uint16_t* kc;            // [B, Hkv, P, D] float16
  uint16_t* vc;
  const int* positions;    // [B]
  void* out;               // [B, Hq * D] float32 or bfloat16
  float* part;             // [B, Hkv, S, G, D + 2] partial softmax states
  const float* cos_t;      // [P, D / 2] RoPE tables, NULL: no rotation
  const float* sin_t;
  int hq, hkv, max_pos, splits;
  float scale;
  int out_bf16;
};

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// (x1, x2) -> (x1 c - x2 s, x2 c + x1 s), the reference's apply_rope pair (ops.py:82-92)
__device__ __forceinline__ void rope_pair(const AttnArgs& a, int pos, int i, int half, float& x1, float& x2) {
  if (!a.cos_t) return;
  const float c = a.cos_t[(size_t)pos * half + i], s = a.sin_t[(size_t)pos * half + i];
  const float r1 = x1 * c - x2 * s, r2 = x2 * c + x1 * s;
  x1 = r1;
  x2 = r2;
}

template <int D, int G>
__global__ __launch_bounds__(256) void decode_attention_kernel(AttnArgs a) {
  constexpr int HALF = D / 2;
  constexpr int LK = D / 8;            // lanes per key: each holds 8 dimensions (one 16-byte load)
  constexpr int KS = 256 / LK;         // keys per pass of the workgroup
  constexpr int NP = kAttnChunk / KS;  // passes over the chunk
  constexpr bool EARLY_V = G <= 4;     // value loads issued with the key loads (register budget)
  __shared__ float qs[G][D];           // rotated queries of the group
  __shared__ float kn[D];              // the new token's rotated key (float16-rounded)
  __shared__ float vn[D];
  __shared__ float ps[G][kAttnChunk];
  __shared__ float red[G][4];
  __shared__ float accs[KS][D];        // one query head's value sums per key slot

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x;
  const int pos = a.positions[b];
  const bool valid = pos >= 0 && pos < a.max_pos;  // else no cache access; the output is NaN
  const int n_keys = valid ? pos + 1 : 0;
  const int used = (n_keys + kAttnChunk - 1) / kAttnChunk;  // workgroups holding keys
  const int j0 = split * kAttnChunk;
  const int jn = min(kAttnChunk, n_keys - j0);  // keys of this workgroup (<= 0: none)
  if (split >= used || jn <= 0) return;  // no keys
  const size_t head = ((size_t)b * a.hkv + h) * (size_t)a.max_pos * D;
  float* part = a.part + (((size_t)b * a.hkv + h) * a.splits + split) * G * (D + 2);
  // thread t: dimensions 8 * (t % LK) .. + 7 of key slot t / LK of each pass
  const int dl = t % LK, slot = t / LK;

  if (jn > 0) {
    // every key (and value) load of the chunk first: their addresses need only the position
    uint4 kw[NP], vw[EARLY_V ? NP : 1];
#pragma unroll
    for (int r = 0; r < NP; ++r) {
      const int jj = slot + KS * r;
      const size_t at = head + (size_t)(j0 + (jj < jn ? jj : 0)) * D + 8 * dl;
      kw[r] = *reinterpret_cast<const uint4*>(a.kc + at);
      if constexpr (EARLY_V) vw[r] = *reinterpret_cast<const uint4*>(a.vc + at);
    }
    // queries (and, for the workgroup holding the new position, k / v), rotated
    for (int e = t; e < G * HALF; e += 256) {
      const int g = e / HALF, i = e - g * HALF;
      const float* qp = a.q + (size_t)b * a.hq * D + (size_t)(h * G + g) * D;
      float x1 = qp[i], x2 = qp[i + HALF];
      rope_pair(a, pos, i, HALF, x1, x2);
      qs[g][i] = x1;
      qs[g][i + HALF] = x2;
    }
    const bool owner = pos >= j0 && pos < j0 + kAttnChunk;
    if (owner) {
      for (int i = t; i < HALF; i += 256) {
        const float* kp = a.k + ((size_t)b * a.hkv + h) * D;
        const float* vp = a.v + ((size_t)b * a.hkv + h) * D;
        float x1 = kp[i], x2 = kp[i + HALF];
        rope_pair(a, pos, i, HALF, x1, x2);
        const uint16_t k1 = f32_to_f16(x1), k2 = f32_to_f16(x2);
        const uint16_t v1 = f32_to_f16(vp[i]), v2 = f32_to_f16(vp[i + HALF]);
        kn[i] = f16_to_f32(k1);
        kn[i + HALF] = f16_to_f32(k2);
        vn[i] = f16_to_f32(v1);
        vn[i + HALF] = f16_to_f32(v2);
        a.kc[head + (size_t)pos * D + i] = k1;
        a.kc[head + (size_t)pos * D + i + HALF] = k2;
        a.vc[head + (size_t)pos * D + i] = v1;
        a.vc[head + (size_t)pos * D + i + HALF] = v2;
      }
    }
    __syncthreads();

    float qr[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) qr[g][e] = qs[g][8 * dl + e];

    // scores (the new position's key comes from LDS)
#pragma unroll
    for (int r = 0; r < NP; ++r) {
      const int jj = slot + KS * r;
      float kv[8];
      if (j0 + jj == pos) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kv[e] = kn[8 * dl + e];
      } else {
        const uint32_t ws[4] = {kw[r].x, kw[r].y, kw[r].z, kw[r].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kv[2 * e] = f16_to_f32((uint16_t)(ws[e] & 0xFFFFu));
          kv[2 * e + 1] = f16_to_f32((uint16_t)(ws[e] >> 16));
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dot = fmaf(qr[g][e], kv[e], dot);
        dot = group_sum_dpp<LK>(dot);  // the key's LK lanes
        if (dl == 0) ps[g][jj] = jj < jn ? dot * a.scale : -INFINITY;
      }
    }
    if constexpr (!EARLY_V) {
#pragma unroll
      for (int r = 0; r < NP; ++r) {
        const int jj = slot + KS * r;
        kw[r] = *reinterpret_cast<const uint4*>(a.vc + head + (size_t)(j0 + (jj < jn ? jj : 0)) * D + 8 * dl);
      }
    }
    __syncthreads();

    // max and sum of exponentials per query head (thread t < chunk <-> key t)
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float v = wave_max_dpp(t < kAttnChunk ? ps[g][t] : -INFINITY);
      if ((t & 63) == 0) red[g][t >> 6] = v;
    }
    __syncthreads();
    float pv[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = fmaxf(fmaxf(red[g][0], red[g][1]), fmaxf(red[g][2], red[g][3]));
      pv[g] = t < jn ? expf(ps[g][t] - m[g]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (t < kAttnChunk) ps[g][t] = pv[g];
      const float v = wave_sum_dpp(pv[g]);
      if ((t & 63) == 0) red[g][t >> 6] = v;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) l[g] = red[g][0] + red[g][1] + red[g][2] + red[g][3];

    // weighted value sums, the same lane mapping
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
#pragma unroll
    for (int r = 0; r < NP; ++r) {
      const int jj = slot + KS * r;
      const uint4 w = EARLY_V ? vw[EARLY_V ? r : 0] : kw[r];
      float vv[8];
      if (j0 + jj == pos) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vv[e] = vn[8 * dl + e];
      } else {
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vv[2 * e] = f16_to_f32((uint16_t)(ws[e] & 0xFFFFu));
          vv[2 * e + 1] = f16_to_f32((uint16_t)(ws[e] >> 16));
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = jj < jn ? ps[g][jj] : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(p, vv[e], o[g][e]);
      }
    }
    // sum over the KS key slots through LDS, one query head at a time
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) accs[slot][8 * dl + e] = o[g][e];
      __syncthreads();
      if (t < D) {
        float v = 0.f;
#pragma unroll
        for (int k2 = 0; k2 < KS; ++k2) v += accs[k2][t];
        part[g * (D + 2) + 2 + t] = v;
      }
      __syncthreads();
    }
    if (t < G) {
      part[t * (D + 2)] = m[t];
      part[t * (D + 2) + 1] = l[t];
    }
  }
}

// Merges the partial states of the `used` workgroups of (sequence b, kv head h)
// (a second launch: the kernel boundary makes the partials visible).
template <int D, int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(AttnArgs a) {
  __shared__ float ms[kMaxSplits][G];  // split maxima, then their weights exp(m_s - M)
  __shared__ float ls[kMaxSplits][G];
  __shared__ float mg[G], dg[G];
  const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int pos = a.positions[b];
  const bool valid = pos >= 0 && pos < a.max_pos;
  const int used = valid ? (pos + kAttnChunk) / kAttnChunk : 0;
  const float* base = a.part + ((size_t)b * a.hkv + h) * a.splits * G * (D + 2);
  for (int i = t; i < used * G; i += 256) {
    const int sp = i / G, g = i - sp * G;
    ms[sp][g] = base[(sp * G + g) * (D + 2)];
    ls[sp][g] = base[(sp * G + g) * (D + 2) + 1];
  }
  __syncthreads();
  if (t < G) {
    float mx = -INFINITY;
    for (int sp = 0; sp < used; ++sp) mx = fmaxf(mx, ms[sp][t]);
    mg[t] = mx;
  }
  __syncthreads();
  for (int i = t; i < used * G; i += 256) {
    const int sp = i / G, g = i - sp * G;
    ms[sp][g] = expf(ms[sp][g] - mg[g]);
  }
  __syncthreads();
  if (t < G) {
    float den = 0.f;
    for (int sp = 0; sp < used; ++sp) den = fmaf(ls[sp][t], ms[sp][t], den);
    dg[t] = den;
  }
  __syncthreads();
  for (int e = t; e < G * D; e += 256) {
    const int g = e / D, d = e - g * D;
    float num = 0.f;
#pragma unroll 8
    for (int sp = 0; sp < used; ++sp) num = fmaf(base[(sp * G + g) * (D + 2) + 2 + d], ms[sp][g], num);
    const float r = valid ? num / dg[g] : __builtin_nanf("");
    const size_t at = (size_t)b * a.hq * D + (size_t)(h * G + g) * D + d;
    if (a.out_bf16)
      static_cast<uint16_t*>(a.out)[at] = f32_to_bf16_bits(r);
    else
      static_cast<float*>(a.out)[at] = r;
  }
}

size_t decode_attention_ws(int64_t batch, int hq, int hkv, int head_dim, int64_t max_pos) {
  const int64_t splits = (max_pos + kAttnChunk - 1) / kAttnChunk;
  return (size_t)batch * hkv * splits * (hq / hkv) * (head_dim + 2) * sizeof(float);
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
  a.splits = (int)((max_pos + kAttnChunk - 1) / kAttnChunk);
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.scale = (float)(1.0 / sqrt((double)head_dim));
  a.out_bf16 = out_bf16;
  const dim3 grid((unsigned)a.splits, (unsigned)hkv, (unsigned)batch);
  const int g = hq / hkv;
  const dim3 mgrid((unsigned)hkv, (unsigned)batch);
#define DRACO_ATTN_LAUNCH(D_, G_)                                                                \
  hipLaunchKernelGGL((decode_attention_kernel<D_, G_>), grid, dim3(256), 0, s, a);              \
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
  if (batch < 1 || batch > 65535 || n_kv_heads < 1 || n_kv_heads > 65535 || n_q_heads < n_kv_heads ||
      n_q_heads % n_kv_heads || n_q_heads / n_kv_heads > kMaxGroup ||
      ((n_q_heads / n_kv_heads) & (n_q_heads / n_kv_heads - 1)))
    return set_error(DRACO_EINVAL_SHAPE,
                     "decode attention needs 1 <= batch <= 65535, n_q_heads = 1, 2, 4 or 8 (<= %d) x n_kv_heads; got "
                     "batch %lld, %d / %d heads",
                     kMaxGroup, (long long)batch, n_q_heads, n_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return set_error(DRACO_EINVAL_SHAPE, "decode attention takes head_dim 64 or 128, got %d", head_dim);
  if (max_positions < 1 || max_positions * head_dim * (int64_t)n_kv_heads * batch > ((int64_t)1 << 40) ||
      max_positions > (int64_t)kMaxSplits * kAttnChunk)
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
