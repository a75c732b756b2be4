/*
 * block_oracle.h — TEST INFRASTRUCTURE ONLY. Plain-C restatement of the
 * projection epilogue (bias add + RoPE, agpt_train.cu:4676-4687 and
 * rope_batched_kernel :1305-1326) and of the textbook RMSProp update that
 * stands in for the absent µGPT cuda_rmsprop_bulk. Used by tests/ as the
 * checker; nothing in the product links or calls it. HOST arrays.
 */
#ifndef AGPT_BLOCK_ORACLE_H
#define AGPT_BLOCK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void oracle_bias_rope(float* x, const float* bias, const int32_t* positions, const float* cos_t,
                      const float* sin_t, int rope_seq_len, int64_t T, int n_heads, int head_dim);

void oracle_rmsprop(float* params, const float* grads, float* sq_avg, float lr, float beta, float eps,
                    int64_t n);

/* LayerNorm (b != NULL) / RMSNorm (b == NULL) over rows of x [T, D]:
 * two-pass mean and variance in double, rounded once to float for rstd. */
void oracle_norm_fwd(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
                     int64_t T, int D, float eps);
/* The backward from the same saved mean / rstd, sums in double. */
void oracle_norm_bwd(const float* dy, const float* x, const float* w, const float* mean, const float* rstd,
                     float* dx, float* dw, float* db, int64_t T, int D);

#ifdef __cplusplus
}
#endif

#endif
