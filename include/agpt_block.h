/*
 * agpt_block.h — C ABI of the kernels around the trie-attention path in one
 * training step (libagpt_attn.so, gfx950): the projection epilogue (bias +
 * RoPE), the row norms (RMSNorm / LayerNorm) and the RMSProp update.
 *
 * Shares the conventions of agpt_attn.h: int status (AGPT_OK = 0) with the
 * message in agpt_last_error(), DEVICE pointers owned by the caller, work
 * ordered on the stream passed in (NULL = default stream), deterministic
 * results.
 */
#ifndef AGPT_BLOCK_H
#define AGPT_BLOCK_H

#include <stdint.h>

#include "agpt_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* In place on x [T, n_heads*head_dim] fp32 (a projection's output): adds
 * bias [n_heads*head_dim] (NULL = none) to every row, then, when cos_t is
 * not NULL, rotates each head's pairs (2i, 2i+1) by the angle of row t's
 * position positions[t] (clamped to rope_seq_len-1):
 *     x0' = x0 c - x1 s,  x1' = x0 s + x1 c,  c/s = table[pos, 2i].
 * Replaces cuda_bias_add + launch_rope_batched (agpt_train.cu:4676-4687,
 * kernel :1305-1326), fused into one pass over x. positions holds one entry
 * per row t (the reference passes one per (row, head), all equal). */
int agpt_bias_rope(float* x, const float* bias, const int32_t* positions, const float* cos_t,
                   const float* sin_t, int rope_seq_len, int64_t T, int n_heads, int head_dim,
                   void* stream);

/* The same epilogue over a fused projection: qkv [T, 3D] holds the q | k | v
 * column blocks of one GEMM (D = n_heads*head_dim), bias [3D] or NULL.
 * Writes contiguous q, k, v [T, D]: bias on all three, RoPE (as
 * agpt_bias_rope) on q and k. One pass instead of three copies and three
 * in-place passes. */
int agpt_bias_rope_split(const float* qkv, const float* bias, const int32_t* positions,
                         const float* cos_t, const float* sin_t, int rope_seq_len, int64_t T,
                         int n_heads, int head_dim, float* q, float* k, float* v, void* stream);

/* RMSProp without momentum over n fp32 parameters:
 *     s = beta s + (1 - beta) g^2,   p -= lr g / (sqrt(s) + eps).
 * Replaces cuda_rmsprop_bulk (the µGPT extern of agpt_train.cu:69, called at
 * :5153-5156 with eps 1e-8); its body is not in the reference, so the update
 * follows the textbook rule above (as torch.optim.RMSprop with alpha = beta,
 * momentum 0, centered False). grads are read only. */
int agpt_rmsprop(float* params, const float* grads, float* sq_avg, float lr, float beta, float eps,
                 int64_t n, void* stream);

/* Row norms over x [T, d_model] fp32 (d_model 64, 128, 256 or 512), the
 * LN1 / LN2 / final-norm sites of agpt_train.cu:4671, 4826, 4800:
 *   LayerNorm (b != NULL): y = (x - mean) rstd w + b, rstd = 1/sqrt(var + eps)
 *   RMSNorm   (b == NULL): y = x rstd w,            rstd = 1/sqrt(mean(x^2) + eps)
 * Saves mean [T] (LayerNorm only) and rstd [T] for the backward. Replaces
 * µGPT's cuda_layer_norm_forward (extern, agpt_train.cu:50-52), which saves
 * the normalised rows instead. */
int agpt_norm_fwd(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
                  int64_t T, int d_model, float eps, void* stream);

/* Backward of agpt_norm_fwd: dx [T, d_model], dw [d_model], and db
 * [d_model] when db != NULL (LayerNorm). dres [T, d_model] (NULL = none) is
 * added into dx: the gradient a residual stream brings to the same x, so the
 * caller needs no separate add where x also feeds a residual connection. dw / db are sums over rows in a
 * fixed order (per-workgroup partials in `workspace`, at least
 * agpt_norm_workspace_floats(d_model) floats, then a column sum): two calls
 * give identical bytes. All pointers 16-byte aligned. Replaces
 * cuda_layer_norm_backward (agpt_train.cu:53-55). */
int agpt_norm_bwd(const float* dy, const float* dres, const float* x, const float* w, const float* mean, const float* rstd,
                  float* dx, float* dw, float* db, float* workspace, int64_t workspace_floats, int64_t T,
                  int d_model, void* stream);

/* Backward of the FFN's ReLU and its bias gradient in one pass over
 * [T, width] fp32 (width 64, 128, 256 or 512): dh = dy where h > 0 else 0
 * (h = the ReLU's output), db [width] = sum over rows of dh in a fixed order
 * (per-workgroup partials in `workspace`, at least
 * agpt_norm_workspace_floats(width) floats, then a column sum). dh may be dy
 * (in place, as the reference). All pointers 16-byte aligned. Replaces
 * cuda_relu_backward (µGPT extern, agpt_train.cu:59; called at :4893) plus
 * launch_bias_grad_accum over its output (:1774-1796, called at :4903),
 * which the reference scales and adds into the bias gradient: the caller
 * scales / accumulates db. */
int agpt_relu_bwd(const float* dy, const float* h, float* dh, float* db, float* workspace,
                  int64_t workspace_floats, int64_t T, int width, void* stream);

/* Workspace floats agpt_norm_bwd and agpt_relu_bwd need for d_model / width. */
int64_t agpt_norm_workspace_floats(int d_model);

#ifdef __cplusplus
}
#endif

#endif /* AGPT_BLOCK_H */
