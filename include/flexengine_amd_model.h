/*
 * flexengine_amd_model.h -- C ABI of the decoder-layer kernels around the
 * paged attention (same library, libfe_paged.so; same conventions as
 * flexengine_amd.h: device pointers, caller-owned buffers, asynchronous on
 * `stream`, no host synchronisation, no allocation, graph-capturable; returns
 * 0, a negative FE_ERR_* code, or a positive hipError_t).
 *
 * These are the caller side of the hot path: the per-layer work of
 * FlexEngine's Qwen2Adapter decode step (src/flexengine/inference/models/
 * qwen2.py:139-186) other than the attention, fused so that a graph-replayed
 * step issues about nine launches per layer.
 *
 * "Sourced" inputs: an argument pair (ptr, splits) names a matrix
 * [rows][cols] that is either fp16 rows (splits == 0; a row stride argument,
 * where present, gives the element distance between rows) or the fp32
 * partial products written by fe_gemm_skinny (splits > 0:
 * [splits][rows][cols] floats, summed by the consumer and rounded to fp16).
 */
#ifndef FLEXENGINE_AMD_MODEL_H
#define FLEXENGINE_AMD_MODEL_H

#include "flexengine_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Fused residual add + RMSNorm over rows of `hidden` (<= 8192) elements:
 *   r = fp16(x + residual)            (residual may be NULL: r = fp16(x))
 *   residual_out = r                  (may be NULL)
 *   out = fp16(weight * fp16(r * rsqrt(mean(r^2) + eps)))
 * x is sourced (x_splits).  Replaces the residual adds and the RMSNorm calls of
 * qwen2.py:97,129-130,150,183-185 (HF Qwen2RMSNorm; the reference's optional
 * Triton RMSNorm is src/flexengine/inference/kernels/rmsnorm.py:9-35).
 */
int fe_rmsnorm(const void* x, int x_splits, const void* residual, void* residual_out,
               const void* weight, void* out, int rows, int hidden, float eps,
               fe_stream_t stream);

/*
 * RoPE on a fused projection row [q: Hq*D | k: Hkv*D | v: Hkv*D] (sourced:
 * qkv, qkv_splits; `bias` [(Hq+2Hkv)*D] fp16 is added to summed partials, may
 * be NULL), writing q_out [rows, Hq, D], k_out and v_out [rows, Hkv, D]:
 *   angle = float(positions[row]) * inv_freq[i]            (fp32)
 *   c, s  = fp16(cos(angle)), fp16(sin(angle))
 *   out[i] = x[i]*c - x[i+D/2]*s,  out[i+D/2] = x[i+D/2]*c + x[i]*s
 * with each product and sum rounded to fp16 as PyTorch's fp16 ops do.
 * positions are int64 (the engine's position tensor).  Replaces
 * Qwen2Adapter._rope and rotate_half (qwen2.py:15-17,73-77) and the q/k/v
 * views of qwen2.py:152-155.
 */
int fe_rope_qkv(const void* qkv, int64_t row_stride, int qkv_splits, const void* bias,
                const int64_t* positions, const float* inv_freq, void* q_out, void* k_out,
                void* v_out, int rows, int num_q_heads, int kv_heads, int head_dim,
                fe_stream_t stream);

/*
 * SiLU-gated product of a fused [gate: I | up: I] row (sourced):
 *   out[row][e] = fp16(fp16(silu(gate[e])) * up[e])        out: [rows, I]
 * Replaces act_fn(gate_proj(x)) * up_proj(x) of the HF Qwen2MLP called at
 * qwen2.py:130,184.
 */
int fe_silu_mul(const void* gate_up, int64_t row_stride, int splits, void* out, int rows,
                int inter, fe_stream_t stream);

/*
 * Number of K slices fe_gemm_skinny uses for a weight of N rows and K columns.
 */
int fe_gemm_skinny_splits(int N, int K);

/*
 * Skinny GEMM for decode-sized batches (M <= 32, K a multiple of 32, x and W
 * 16-byte aligned):
 *   partials[s][m][o] = sum over k in slice s of x[m][k] * W[o][k]
 * x: fp16 [M, K]; W: fp16 [N, K] (PyTorch Linear weight layout); partials:
 * fp32 [splits][M][N] with splits = fe_gemm_skinny_splits(N, K).  Consumers
 * take (partials, splits) as a sourced input.  Replaces the q/k/v, o, gate/up
 * and down projections and the LM head of the decode step (qwen2.py:152-154,
 * 183-186) for small batches.
 */
int fe_gemm_skinny(const void* x, int M, int K, const void* W, int N, float* partials,
                   int splits, fe_stream_t stream);

/*
 * Decode-step projections with their element-wise neighbours fused
 * (M <= 64 rows, K a multiple of 32, x and W 16-byte aligned; the workgroups
 * of a 16-row output tile
 * reduce K among themselves -- split-K partial tiles meet in `workspace` and the
 * last workgroup adds them in split order -- so results are final fp16 values,
 * deterministic from call to call).  workspace: at least
 * fe_gemm_fused_workspace_size(M, N, K) bytes, 256-byte aligned, zero-filled
 * before its first use; every call leaves it ready for the next (calls that
 * overlap in time need separate workspaces).
 *
 * Optional RMSNorm prologue, shared by fe_gemm_f16, fe_gemm_silu and
 * fe_gemm_rope: with x_ss == NULL the operand is x [M, K] itself; otherwise x
 * is the un-normalised residual stream r [M, K] and x_ss [ss_tiles][M] the
 * per-tile sums of r^2 written by fe_gemm_resid, and the operand is
 *   fp16(norm_w * fp16(r * rsqrt(sum_t x_ss[t][m] / K + eps)))
 * (transformers' Qwen2RMSNorm, as fe_rmsnorm computes it).
 */

/* Workspace bytes of the fused projections for an [N, K] weight and M rows. */
size_t fe_gemm_fused_workspace_size(int M, int N, int K);

/* out [M, N] = fp16(operand @ W^T + bias); bias [N] may be NULL.  The LM head
 * with the final norm (qwen2.py:185-186). */
int fe_gemm_f16(const void* x, const float* x_ss, int ss_tiles, const void* norm_w, float eps,
                int M, int K, const void* W, int N, const void* bias, void* out,
                void* workspace, size_t workspace_bytes, fe_stream_t stream);

/* r = fp16(fp16(x @ W^T) + residual), written to out [M, N] (may alias
 * nothing the call reads), and out_ss [ceil(N/16)][M] = sum of r^2 over each
 * 16-column tile: the o and down projections with the residual adds of
 * qwen2.py:129-130,183-184, producing the next RMSNorm's input. */
int fe_gemm_resid(const void* x, int M, int K, const void* W, int N, const void* residual,
                  void* out, float* out_ss, void* workspace, size_t workspace_bytes,
                  fe_stream_t stream);

/* fe_gemm_resid followed by the RMSNorm of its result, in one launch: writes
 * r to out [M, N] and out_ss as fe_gemm_resid does, and norm_out [M, N] =
 * fp16(norm_w * fp16(r * rsqrt(mean(r^2) + eps))) (transformers'
 * Qwen2RMSNorm, as fe_rmsnorm computes it; the mean from the tile sums).  The
 * workgroup that finishes the last output tile normalises every row, so the
 * residual add and the post-attention / next input norm of qwen2.py:129-134
 * cost one launch.  N a multiple of 16, at most 2048; out, norm_w and
 * norm_out 16-byte aligned; workspace as for the other fused projections
 * (always required: it holds the launch-wide ticket). */
int fe_gemm_resid_rmsnorm(const void* x, int M, int K, const void* W, int N,
                          const void* residual, void* out, float* out_ss, const void* norm_w,
                          float eps, void* norm_out, void* workspace, size_t workspace_bytes,
                          fe_stream_t stream);

/* W = [gate; up] ([2I, K]); out [M, I] = fp16(fp16(silu(g)) * u) with
 * g, u = fp16 of the gate / up products: the gate/up projection and act_fn
 * product of HF Qwen2MLP (qwen2.py:130,184). */
int fe_gemm_silu(const void* x, const float* x_ss, int ss_tiles, const void* norm_w, float eps,
                 int M, int K, const void* W, int N, void* out, void* workspace,
                 size_t workspace_bytes, fe_stream_t stream);

/* W = [q; k; v] ([(Hq + 2 Hkv) * D, K]) with bias; writes q_out [M, Hq, D],
 * k_out and v_out [M, Hkv, D] with RoPE on q and k exactly as fe_rope_qkv
 * computes it (positions int64 [M], inv_freq fp32 [D/2]; D a multiple of 16):
 * the q/k/v projection, split and _rope of qwen2.py:67-77,152-155. */
int fe_gemm_rope(const void* x, const float* x_ss, int ss_tiles, const void* norm_w, float eps,
                 int M, int K, const void* W, const void* bias, const int64_t* positions,
                 const float* inv_freq, int num_q_heads, int kv_heads, int head_dim,
                 void* q_out, void* k_out, void* v_out, void* workspace,
                 size_t workspace_bytes, fe_stream_t stream);

/*
 * out [M, N] = fp16(x [M, K] @ W^T + bias) for 33..64 rows (any M <= 64; K a
 * multiple of 32; x and W 16-byte aligned; bias [N] may be NULL): the four
 * waves of a workgroup take four
 * 16-row weight tiles over the same keys and share each 128-key chunk of x
 * through LDS.  workspace: at least fe_gemm_rows64_workspace_size(M, N, K)
 * bytes, 256-byte aligned, zero-filled before its first use (split-K tickets
 * that every call leaves at zero, then partial tiles).  Replaces the library
 * GEMM for the batch-64 decode step's deep projection (K >= 4 N: the MLP down
 * projection, qwen2.py:183-184), where it measured faster; wide projections
 * stay on the library GEMM.
 */
size_t fe_gemm_rows64_workspace_size(int M, int N, int K);
int fe_gemm_rows64(const void* x, int M, int K, const void* W, int N, const void* bias,
                   void* out, void* workspace, size_t workspace_bytes, fe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLEXENGINE_AMD_MODEL_H */
