/*
 * draco_gguf.h -- C ABI of libdraco_gguf.so, the MI355X (gfx950) GGUF
 * quantized-matmul library.
 *
 * Plain C types only: device pointers are `const void*` / `float*` into HBM
 * (e.g. torch tensor data_ptr()), sizes are int64_t, the stream is a
 * hipStream_t passed as `void*` (NULL = the null stream).
 *
 * Conventions (all entry points):
 *  - Caller-allocated buffers; the library never allocates or frees caller
 *    memory.  Pointers are borrowed for the duration of the enqueued work.
 *  - Every call only ENQUEUES work on `stream` and returns; nothing here
 *    synchronizes the device.
 *  - Return 0 on success or a negative DRACO_E* code; the calling thread's
 *    draco_gguf_last_error() then holds a message.
 *  - Weight buffers hold GGUF blocks in their native packed layout: an [N, K]
 *    weight is N rows of K/QK blocks, rows contiguous, blocks along K
 *    (reference: draco/format/gguf.py:630-648).  Weight, activation and output
 *    pointers must be 16-byte aligned.  Weight entry points also take the
 *    byte size of the weight buffer; a buffer shorter than the shape needs
 *    (a truncated payload) is rejected with DRACO_EINVAL_SHAPE before any
 *    launch.
 *  - ggml_type is the GGUF type id, optionally OR-ed with
 *    DRACO_GGUF_GGML_ORDER for Q2_K / Q3_K / Q6_K blocks stored in upstream
 *    ggml field order instead of the reference's, which puts the float16
 *    scales first:
 *      Q2_K  reference d, dmin, qs[64], scales[16]   ggml scales, qs, d, dmin
 *      Q3_K  reference d, scales[12], qs[64], hmask  ggml hmask, qs, scales, d
 *      Q6_K  reference d, ql, qh, scales[16]         ggml ql, qh, scales, d
 */
#ifndef DRACO_GGUF_H
#define DRACO_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids handled here: every block type of the reference's
 * _BLOCK_LAYOUTS (reference: draco/format/gguf.py:57-87). */
#define DRACO_GGML_TYPE_Q4_0 2
#define DRACO_GGML_TYPE_Q4_1 3
#define DRACO_GGML_TYPE_Q5_0 6
#define DRACO_GGML_TYPE_Q5_1 7
#define DRACO_GGML_TYPE_Q8_0 8
#define DRACO_GGML_TYPE_Q2_K 10
#define DRACO_GGML_TYPE_Q3_K 11
#define DRACO_GGML_TYPE_Q4_K 12
#define DRACO_GGML_TYPE_Q5_K 13
#define DRACO_GGML_TYPE_Q6_K 14
#define DRACO_GGML_TYPE_Q8_K 15
/* Layout flag: upstream ggml field order of Q2_K / Q3_K / Q6_K blocks. */
#define DRACO_GGUF_GGML_ORDER 0x100
/* Older name of the same flag (it first applied to Q6_K only). */
#define DRACO_GGUF_Q6K_D_LAST DRACO_GGUF_GGML_ORDER

/* Activation dtypes. */
#define DRACO_DTYPE_F32 0
#define DRACO_DTYPE_BF16 1

/* Return codes. */
#define DRACO_OK 0
#define DRACO_EINVAL_QTYPE (-1) /* unsupported ggml type               */
#define DRACO_EINVAL_SHAPE (-2) /* K % QK != 0, non-positive or too-large dims, M out of range */
#define DRACO_EINVAL_ARG (-3)   /* null / misaligned pointer, bad dtype */
#define DRACO_EHIP (-4)         /* HIP launch or runtime error          */
#define DRACO_EWORKSPACE (-5)   /* workspace missing or too small       */

/* ABI version of this header (bumped on any signature change). */
int draco_gguf_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* draco_gguf_last_error(void);

/*
 * Block geometry of a ggml type: elements per block and bytes per block.
 * Replaces the lookup in _BLOCK_LAYOUTS (draco/format/gguf.py:75-87).
 */
int draco_gguf_block_info(int ggml_type, int* qk, int* block_bytes);

/*
 * out[n_rows, k] (float32) = dequantize(blocks), bit-exact to the reference
 * float32 dequant.  Blocks may run across rows when k is not a multiple of
 * the block size, as long as n_rows * k is (the reference's rule, at most
 * 2^30 values in that case).  Replaces _dequantize(qtype, payload, n)
 * (draco/format/gguf.py:272-497) as called by GGUFReader.get_tensor
 * (draco/format/gguf.py:820-834).
 */
int draco_gguf_dequant_f32(int ggml_type, const void* blocks, size_t blocks_bytes, float* out, int64_t n_rows,
                           int64_t k, void* stream);

/*
 * Decode GEMV with the dequantization fused in:
 *   y[m, n] = x[m, k] . W[n, k]^T (+ bias[n]),  1 <= m <= 16.
 * x is float32 or bfloat16 (x_dtype), y and bias (nullable) float32;
 * accumulation is float32.  Replaces _dequantize followed by
 * GenericGemmKernel.matmul_f32 (draco/runtime/cpu/kernels/generic.py:32-33)
 * inside _linear (draco/runtime/cpu/executor.py:47-79), and
 * QuantizationBackend.quantized_linear (draco/quantization/base.py:86-99).
 */
int draco_gguf_gemv(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype, const float* bias,
                    float* y, int64_t m, int64_t n, int64_t k, void* stream);

/*
 * Several decode GEMVs sharing one activation, in one launch (e.g. the q, k
 * and v projections of a layer):
 *   y_i[m, n_i] = x[m, k] . W_i[n_i, k]^T   for i < n_mats (1..4),
 * every W_i of the same ggml type and row length k, w_bytes[i] its buffer
 * size.  y[i] (float32) and y_bf16[i] (bfloat16 copy, round to nearest even)
 * may each be NULL but not both; y and y_bf16 themselves may be NULL arrays.
 * 1 <= m <= 16.  x must not overlap any output.  Replaces _qkv
 * (draco/runtime/cpu/executor.py:243-271), three _linear calls sharing x.
 */
int draco_gguf_gemv_multi(int ggml_type, int n_mats, const void* const* w, const size_t* w_bytes,
                          const int64_t* n, float* const* y, void* const* y_bf16, const void* x, int x_dtype,
                          int64_t m, int64_t k, void* stream);

/*
 * Gate and up projections with the SwiGLU product fused in:
 *   y[m, n] = silu(x . W_gate^T) * (x . W_up^T),  silu(g) = g / (1 + e^-g),
 * W_gate and W_up [n, k] of one ggml type, each w_bytes long; y float32 and/or
 * y_bf16 (either may be NULL, not both); 1 <= m <= 16; x must not overlap an
 * output.  Replaces the gate/up _linear calls and swiglu of _mlp
 * (draco/runtime/cpu/executor.py:208-224, draco/runtime/cpu/ops.py:19-27).
 */
int draco_gguf_gemv_swiglu(int ggml_type, const void* w_gate, const void* w_up, size_t w_bytes, const void* x,
                           int x_dtype, float* y, void* y_bf16, int64_t m, int64_t n, int64_t k, void* stream);

/*
 * Projection plus residual add, in place:
 *   resid[m, n] += x . W^T,  then resid_bf16 = bf16(resid) if not NULL.
 * 1 <= m <= 16; x must not overlap resid or resid_bf16.  Replaces _o_proj /
 * the down projection of _mlp and the residual adds of forward_step
 * (draco/runtime/cpu/executor.py:208-224, 273-277, 308-329).
 */
int draco_gguf_gemv_residual(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype, float* resid,
                             void* resid_bf16, int64_t m, int64_t n, int64_t k, void* stream);

/*
 * draco_gguf_gemv_residual with a workspace (device memory, 256-byte
 * aligned): launches with few 16-row tiles and long rows (K > 4096, e.g. the
 * down projection at 8..16 tokens) then split K over several workgroups per
 * tile, store the partial sums to the workspace and add them in a fixed
 * order in a second launch (the result does not depend on scheduling).  The
 * bytes needed are draco_gguf_gemv_residual_workspace_size(type, m, n, k) (0:
 * this launch is not split; a smaller workspace, or NULL, runs unsplit).
 * Same reference call sites as draco_gguf_gemv_residual.
 */
size_t draco_gguf_gemv_residual_workspace_size(int ggml_type, int64_t m, int64_t n, int64_t k);
int draco_gguf_gemv_residual_ws(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype,
                                float* resid, void* resid_bf16, int64_t m, int64_t n, int64_t k, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * Workspace bytes draco_gguf_gemm / draco_gguf_linear use for m token rows of
 * length k with this weight type (0 when the type's GEMM needs none).  Q4_K
 * requires m * k * 2 + 3 * m * (k / 32) * 2 + m * 4 bytes (rounded up to 256
 * per part: the activations as float16, their 32-element sums, the row
 * scales); the size returned adds m * 128 * (256 / ceil(m / 256)) * 4
 * bytes of room for split-K partial sums, which shapes with too few output
 * tiles to fill the GPU, and the partial last round of a grid that does not
 * divide evenly over the CUs, use when the workspace given holds them.
 */
size_t draco_gguf_gemm_workspace_size(int ggml_type, int64_t m, int64_t k);

/*
 * Prefill GEMM with the dequantization fused in (bf16 activations, MFMA,
 * float32 accumulate and output):
 *   y[m, n] = x_bf16[m, k] . W[n, k]^T (+ bias[n]),  m >= 1.
 * Same reference call sites as draco_gguf_gemv, for prompt-sized M.
 * `workspace` (device memory, 256-byte aligned, workspace_bytes =
 * draco_gguf_gemm_workspace_size) selects the float16 matrix-core kernels for
 * Q4_K; NULL runs the workspace-free kernel (three bf16 weight planes,
 * slower).  A workspace below the required part (the size without the
 * split-K room) is an error (DRACO_EWORKSPACE); one without the room runs
 * unsplit.
 */
int draco_gguf_gemm(int ggml_type, const void* w, size_t w_bytes, const void* x_bf16, const float* bias, float* y,
                    int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes, void* stream);

/*
 * _linear for any M: draco_gguf_gemv for m <= 16, draco_gguf_gemm (with the
 * workspace, which may be NULL) for larger m with bf16 activations, and
 * 16-row GEMV tiles for larger m with float32 activations.  Replaces _linear
 * (draco/runtime/cpu/executor.py:47-79).
 */
int draco_gguf_linear(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype, const float* bias,
                      float* y, int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                      void* stream);

/*
 * draco_gguf_linear that allocates nothing and takes no workspace.  No
 * counterpart in the reference: this entry point is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The Q4_K prefill GEMM's workspace lives
 * in a static device array of DRACO_GGUF_NOALLOC_SCRATCH_BYTES per GPU (held
 * by each GPU the library runs on until the process ends), enough for
 * m = 2048 rows of k = 14336; a call needing more (see
 * draco_gguf_gemm_workspace_size) fails with DRACO_EWORKSPACE before any
 * launch.  The array of the calling thread's current device is used, so the
 * stream must belong to that device; its address is looked up on the first
 * call on each device (make that first call outside graph capture).  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (concurrent streams, threads or processes' graphs replayed together) race.
 * Nothing in the array needs to start at zero (each call writes what it reads).
 */
#define DRACO_GGUF_NOALLOC_SCRATCH_BYTES (64u << 20)
int draco_gguf_linear_noalloc(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype,
                              const float* bias, float* y, int64_t m, int64_t n, int64_t k, void* stream);

/*
 * Workspace bytes draco_gguf_moe_ffn needs for `tokens` tokens.
 */
size_t draco_gguf_moe_workspace_size(int64_t tokens, int64_t hidden, int64_t inter, int n_experts, int top_k);

/*
 * Sparse MoE FFN over GGUF experts:
 *   (idx, w) = top_k(router_logits[t, :]); w = softmax(w); w /= sum(w)
 *   y[t] = sum over the token's experts e, in ascending e, of
 *          w_e * W_down[e] . (silu(W_gate[e] . x[t]) * (W_up[e] . x[t]))
 * w_gate / w_up ([inter, hidden]) and w_down ([hidden, inter]) are HOST arrays
 * of n_experts device pointers, each buffer at least expert_w_bytes long; x is [tokens, hidden] bfloat16 or float32,
 * router_logits [tokens, n_experts] float32, y [tokens, hidden] float32.
 * Routing and grouping run on the device (no host synchronization).
 * Replaces TopKRouter.forward (draco/models/moe/router.py:81-120) and
 * ExpertGroup.forward (draco/models/moe/expert.py:77-116).
 */
int draco_gguf_moe_ffn(int ggml_type, const void* const* w_gate, const void* const* w_up,
                       const void* const* w_down, size_t expert_w_bytes, const float* router_logits, const void* x, int x_dtype,
                       float* y, int64_t tokens, int64_t hidden, int64_t inter, int n_experts, int top_k,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * draco_gguf_gemv_multi / draco_gguf_gemv_swiglu whose input is
 * RMSNorm(x): x [m, k] float32, norm_w [k] float32,
 *   x_norm = bf16(x / sqrt(mean(x^2) + eps) * norm_w)   ([m, k], written)
 * and the GEMV runs on x_norm.  For single-token bf16-eligible launches of
 * Q4_K / Q6_K (k <= 4096) the norm runs in the GEMV's own prologue (no extra
 * launch); otherwise it is a separate RMSNorm launch.  Replaces _norm
 * (draco/runtime/cpu/executor.py:199-206) followed by _qkv / _mlp.
 */
int draco_gguf_gemv_multi_rmsnorm(int ggml_type, int n_mats, const void* const* w, const size_t* w_bytes,
                                  const int64_t* n, float* const* y, void* const* y_bf16, const float* x,
                                  const float* norm_w, float eps, void* x_norm, int64_t m, int64_t k, void* stream);

int draco_gguf_gemv_swiglu_rmsnorm(int ggml_type, const void* w_gate, const void* w_up, size_t w_bytes,
                                   const float* x, const float* norm_w, float eps, void* x_norm, float* y,
                                   void* y_bf16, int64_t m, int64_t n, int64_t k, void* stream);

/*
 * RMSNorm of m rows of n float32 values (n a multiple of 4):
 *   y[r, i] = x[r, i] / sqrt(mean_j(x[r, j]^2) + eps) * weight[i]
 * into float32 y and / or bfloat16 y_bf16 (either may be NULL, not both).
 * Replaces rms_norm (draco/runtime/cpu/ops.py:15-19) as the executor's _norm
 * (draco/runtime/cpu/executor.py:199-206) calls it.
 */
int draco_gguf_rms_norm(const float* x, const float* weight, float eps, float* y, void* y_bf16, int64_t m, int64_t n,
                        void* stream);

/*
 * Workspace bytes draco_gguf_decode_attention needs (0 for invalid sizes):
 * the partial softmax states of the position splits.
 */
size_t draco_gguf_decode_attention_workspace_size(int64_t batch, int n_q_heads, int n_kv_heads, int head_dim,
                                                  int64_t max_positions);

/*
 * One decode token per sequence b (batch sequences): rotate q [b, n_q_heads *
 * head_dim] and k [b, n_kv_heads * head_dim] (float32) with RoPE at
 * position p = positions[b] (device int32, 0 <= p < max_positions) using
 * the tables rope_cos / rope_sin [max_positions][head_dim / 2] (float32, as
 * build_rope_cache makes them, draco/runtime/cpu/ops.py:73-79; both NULL:
 * no rotation), store k and v in the float16 caches
 * k_cache / v_cache [batch][n_kv_heads][max_positions][head_dim] at that
 * position, and write the attention of q over positions 0 .. p of its
 * sequence (query head h reads kv head h / (n_q_heads / n_kv_heads);
 * scores q.k / sqrt(head_dim), softmax, weighted sum of v) to out
 * [b, n_q_heads * head_dim], float32 or bfloat16 (out_dtype).  Any even
 * head_dim of 2..256, n_q_heads a multiple of n_kv_heads, max_positions <=
 * 131072.  head_dim 64 or 128 with 1, 2, 4 or 8 query heads per kv head run
 * two launches (partial attention per position split, then the merge); other
 * shapes one workgroup per (query head, sequence) whose workspace holds the
 * scores (draco_gguf_decode_attention_workspace_size gives either size).
 * A position outside [0, max_positions) touches no cache memory and yields
 * NaN outputs.
 * Replaces apply_rope (draco/runtime/cpu/ops.py:73-92) on q / k and
 * CPUAttentionBackend.decode (draco/runtime/cpu/attention.py:35-81) with its
 * CPUKVCache append (float16 storage, draco/runtime/cpu/kv_cache.py:19-28).
 */
int draco_gguf_decode_attention(const float* q, const float* k, const float* v, void* k_cache, void* v_cache,
                                const int32_t* positions, int64_t batch, int n_q_heads, int n_kv_heads, int head_dim,
                                int64_t max_positions, const float* rope_cos, const float* rope_sin, void* out,
                                int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Executor pieces for the tensors of a GGUF model that are not
 * block-quantized, and the glue between projections that were not fused.
 *
 * draco_gguf_dense_linear: y[m, n] = x[m, k] . W[n, k]^T (+ bias[n]) for a
 * float weight, ggml_type F32 (0), F16 (1) or BF16 (30); x float32 or
 * bfloat16 (x_dtype), float32 accumulation; accumulate != 0 adds the result
 * into y (the residual add).  Replaces _linear on a tensor with
 * quantization=None: get_tensor(dequantize=True) then matmul_f32
 * (draco/runtime/cpu/executor.py:47-52, 77-78,
 * draco/runtime/cpu/kernels/generic.py:32-33).
 */
int draco_gguf_dense_linear(int ggml_type, const void* w, size_t w_bytes, const void* x, int x_dtype,
                            const float* bias, float* y, int64_t m, int64_t n, int64_t k, int accumulate,
                            void* stream);

/*
 * Embedding gather: out[i, :] (float32) = row ids[i] of the [n_rows, k]
 * table w, for i < n_ids (<= 65535); ids are device int32.  Block-quantized
 * tables (k a multiple of the block size) are dequantized bit-exactly as
 * draco_gguf_dequant_f32 does; F32 / F16 / BF16 tables are converted.  An id
 * outside [0, n_rows) gives a row of NaN.  Replaces embed[token_ids] after
 * get_tensor(embed_name, dequantize=True) in _initial_hidden
 * (draco/runtime/cpu/executor.py:279-288).
 */
int draco_gguf_get_rows(int ggml_type, const void* w, size_t w_bytes, int64_t n_rows, int64_t k, const int32_t* ids,
                        int64_t n_ids, float* out, void* stream);

/*
 * y = silu(gate) * up over n float32 values into float32 y and / or bfloat16
 * y_bf16 (either may be NULL, not both): swiglu (draco/runtime/cpu/ops.py:19-27)
 * for gate / up projections computed by separate launches.
 */
int draco_gguf_swiglu(const float* gate, const float* up, float* y, void* y_bf16, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DRACO_GGUF_H */
