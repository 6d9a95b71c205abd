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
//   * the last workgroup of a (sequence, kv head) to finish -- found with a
//     device-scope counter, no waiting -- merges the partial states and writes
//     the output; it resets the counter, so the workspace needs zeroing once.
#include <math.h>

#include "draco_internal.h"
#include "gemv_core.h"

namespace draco {

__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum_dpp(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       float eps, float* __restrict__ y, uint16_t* __restrict__ yb,
                                                       int n) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * n;
  float ss = 0.f;
  for (int i = threadIdx.x * 4; i < n; i += 1024) {
    const float4 v = *reinterpret_cast<const float4*>(xr + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  const float denom = sqrtf(block_sum_256(ss, red) / (float)n + eps);
  for (int i = threadIdx.x * 4; i < n; i += 1024) {
    const float4 v = *reinterpret_cast<const float4*>(xr + i);
    const float4 g = *reinterpret_cast<const float4*>(w + i);
    const float4 o = make_float4(v.x / denom * g.x, v.y / denom * g.y, v.z / denom * g.z, v.w / denom * g.w);
    const size_t at = (size_t)blockIdx.x * n + i;
    if (y) *reinterpret_cast<float4*>(y + at) = o;
    if (yb) {
      const uint32_t lo = f32_to_bf16_bits(o.x) | ((uint32_t)f32_to_bf16_bits(o.y) << 16);
      const uint32_t hi = f32_to_bf16_bits(o.z) | ((uint32_t)f32_to_bf16_bits(o.w) << 16);
      *reinterpret_cast<uint2*>(yb + at) = make_uint2(lo, hi);
    }
  }
}

int rms_norm_launch(const float* x, const float* w, float eps, float* y, uint16_t* yb, int64_t m, int64_t n,
                    hipStream_t s) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)m), dim3(256), 0, s, x, w, eps, y, yb, (int)n);
  return check_launch("rms_norm");
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
constexpr int kAttnChunk = 256;  // positions per workgroup
constexpr int kMaxGroup = 8;     // query heads per kv head

struct AttnArgs {
  const float* q;          // [B, Hq * D]
  const float* k;          // [B, Hkv * D]
  const float* v;          // [B, Hkv * D]
  uint16_t* kc;            // [B, Hkv, P, D] float16
  uint16_t* vc;
  const int* positions;    // [B]
  void* out;               // [B, Hq * D] float32 or bfloat16
  float* part;             // [B, Hkv, S, G, D + 2]
  unsigned* count;         // [B, Hkv]
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

template <int D>
__global__ __launch_bounds__(256) void decode_attention_kernel(AttnArgs a) {
  constexpr int HALF = D / 2;
  __shared__ float qs[kMaxGroup][D];     // rotated queries of the group
  __shared__ float kn[D];                // the new token's rotated key (float16-rounded)
  __shared__ float vn[D];
  __shared__ float ps[kMaxGroup][kAttnChunk];
  __shared__ float red[kMaxGroup][4];
  constexpr int SETS = 256 / D;  // thread sets splitting the keys of the value sums
  __shared__ float accs[SETS - 1][kMaxGroup][D];
  __shared__ int last;

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int G = a.hq / a.hkv;
  const int t = threadIdx.x;
  const int pos = a.positions[b];
  const bool valid = pos >= 0 && pos < a.max_pos;  // else no cache access; the output is NaN
  const int n_keys = valid ? pos + 1 : 0;
  const int j0 = split * kAttnChunk;
  const int jn = min(kAttnChunk, n_keys - j0);  // keys of this workgroup (<= 0: none)
  const size_t head = ((size_t)b * a.hkv + h) * (size_t)a.max_pos * D;
  float* part = a.part + (((size_t)b * a.hkv + h) * a.splits + split) * G * (D + 2);

  if (jn > 0) {
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

    // scores: thread t <-> key j0 + t
    float sc[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) sc[g] = -INFINITY;
    if (t < jn) {
      const int j = j0 + t;
      float dot[kMaxGroup];
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) dot[g] = 0.f;
      if (j == pos) {
        for (int i = 0; i < D; ++i) {
#pragma unroll
          for (int g = 0; g < kMaxGroup; ++g)
            if (g < G) dot[g] = fmaf(qs[g][i], kn[i], dot[g]);
        }
      } else {
        const uint4* kp = reinterpret_cast<const uint4*>(a.kc + head + (size_t)j * D);
        for (int c = 0; c < D / 8; ++c) {
          const uint4 w = kp[c];
          const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float k0 = f16_to_f32((uint16_t)(ws[e] & 0xFFFFu)), k1 = f16_to_f32((uint16_t)(ws[e] >> 16));
            const int i = 8 * c + 2 * e;
#pragma unroll
            for (int g = 0; g < kMaxGroup; ++g)
              if (g < G) dot[g] = fmaf(qs[g][i + 1], k1, fmaf(qs[g][i], k0, dot[g]));
          }
        }
      }
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) sc[g] = dot[g] * a.scale;
    }
    // max and sum of exponentials per query head
    float m[kMaxGroup], l[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      if (g >= G) break;
      float v = sc[g];
      v = fmaxf(v, __shfl_xor(v, 1, 64));
      v = fmaxf(v, __shfl_xor(v, 2, 64));
      v = fmaxf(v, __shfl_xor(v, 4, 64));
      v = fmaxf(v, __shfl_xor(v, 8, 64));
      v = fmaxf(v, __shfl_xor(v, 16, 64));
      v = fmaxf(v, __shfl_xor(v, 32, 64));
      if ((t & 63) == 0) red[g][t >> 6] = v;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      if (g >= G) break;
      m[g] = fmaxf(fmaxf(red[g][0], red[g][1]), fmaxf(red[g][2], red[g][3]));
      const float p = t < jn ? expf(sc[g] - m[g]) : 0.f;
      ps[g][t] = p;
      sc[g] = p;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      if (g >= G) break;
      float v = wave_sum_dpp(sc[g]);
      if ((t & 63) == 0) red[g][t >> 6] = v;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      if (g >= G) break;
      l[g] = red[g][0] + red[g][1] + red[g][2] + red[g][3];
    }
    // weighted value sums: thread t <-> dimension t % D, keys split over the thread sets
    const int d = t % D, set = t / D;
    float o[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) o[g] = 0.f;
    for (int jj = set; jj < jn; jj += SETS) {
      const int j = j0 + jj;
      const float vv = j == pos ? vn[d] : f16_to_f32(a.vc[head + (size_t)j * D + d]);
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g)
        if (g < G) o[g] = fmaf(ps[g][jj], vv, o[g]);
    }
    if (set > 0) {
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g)
        if (g < G) accs[set - 1][g][d] = o[g];
    }
    __syncthreads();
    if (set == 0) {
      for (int r = 0; r < SETS - 1; ++r) {
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g)
          if (g < G) o[g] += accs[r][g][d];
      }
    }
    if (set == 0) {
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) {
        if (g >= G) break;
        part[g * (D + 2) + 2 + d] = o[g];
        if (d == 0) {
          part[g * (D + 2)] = m[g];
          part[g * (D + 2) + 1] = l[g];
        }
      }
    }
  }

  // the last workgroup of (b, h) merges the partial states
  __threadfence();
  __syncthreads();
  if (t == 0) {
    const unsigned done = atomicAdd(a.count + (size_t)b * a.hkv + h, 1u);
    last = done == (unsigned)a.splits - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  const int used = (n_keys + kAttnChunk - 1) / kAttnChunk;  // splits that hold keys
  const float* base = a.part + ((size_t)b * a.hkv + h) * a.splits * G * (D + 2);
  for (int e = t; e < G * D; e += 256) {
    const int g = e / D, d = e - g * D;
    float mx = -INFINITY;
    for (int s = 0; s < used; ++s) mx = fmaxf(mx, base[(s * G + g) * (D + 2)]);
    float num = 0.f, den = 0.f;
    for (int s = 0; s < used; ++s) {
      const float* p = base + (s * G + g) * (D + 2);
      const float f = expf(p[0] - mx);
      den = fmaf(p[1], f, den);
      num = fmaf(p[2 + d], f, num);
    }
    const float r = valid ? num / den : __builtin_nanf("");
    const size_t at = (size_t)b * a.hq * D + (size_t)(h * G + g) * D + d;
    if (a.out_bf16)
      static_cast<uint16_t*>(a.out)[at] = f32_to_bf16_bits(r);
    else
      static_cast<float*>(a.out)[at] = r;
  }
  if (t == 0) atomicExch(a.count + (size_t)b * a.hkv + h, 0u);
}

size_t decode_attention_ws(int64_t batch, int hq, int hkv, int head_dim, int64_t max_pos) {
  const int64_t splits = (max_pos + kAttnChunk - 1) / kAttnChunk;
  const size_t part = (size_t)batch * hkv * splits * (hq / hkv) * (head_dim + 2) * sizeof(float);
  const size_t count = (size_t)batch * hkv * sizeof(unsigned);
  return ((count + 255) & ~(size_t)255) + part;
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
  a.count = static_cast<unsigned*>(workspace);
  const size_t count = (size_t)batch * hkv * sizeof(unsigned);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((count + 255) & ~(size_t)255));
  a.hq = hq;
  a.hkv = hkv;
  a.max_pos = (int)max_pos;
  a.splits = (int)((max_pos + kAttnChunk - 1) / kAttnChunk);
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.scale = (float)(1.0 / sqrt((double)head_dim));
  a.out_bf16 = out_bf16;
  const dim3 grid((unsigned)a.splits, (unsigned)hkv, (unsigned)batch);
  if (head_dim == 128)
    hipLaunchKernelGGL(decode_attention_kernel<128>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(decode_attention_kernel<64>, grid, dim3(256), 0, s, a);
  return check_launch("decode_attention");
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
      n_q_heads % n_kv_heads || n_q_heads / n_kv_heads > kMaxGroup)
    return set_error(DRACO_EINVAL_SHAPE,
                     "decode attention needs 1 <= batch <= 65535, n_q_heads a multiple (<= %d x) of n_kv_heads; got "
                     "batch %lld, %d / %d heads",
                     kMaxGroup, (long long)batch, n_q_heads, n_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return set_error(DRACO_EINVAL_SHAPE, "decode attention takes head_dim 64 or 128, got %d", head_dim);
  if (max_positions < 1 || max_positions * head_dim * (int64_t)n_kv_heads * batch > ((int64_t)1 << 40) ||
      max_positions > (1 << 24))
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
