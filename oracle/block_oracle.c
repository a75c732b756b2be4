/*
 * block_oracle.c — TEST INFRASTRUCTURE ONLY (the checker, never the
 * product). Only tests/ load it (through oracle/liboracle.so).
 *
 * oracle_bias_rope: cuda_bias_add (row + bias) followed by
 * rope_batched_kernel (agpt_train.cu:1305-1326) over each (row, head) slice,
 * the position of row t taken for all its heads. oracle_rmsprop: the
 * textbook RMSProp without momentum (the µGPT body is absent). Compiled with
 * -ffp-contract=off. Pinning: tests/test_block_oracle.py (rotation by a
 * known angle, norm preservation, the inverse rotation of the trie oracle
 * undoing it, torch.optim.RMSprop on the same tensors).
 */
#include "block_oracle.h"

#include <math.h>

void oracle_bias_rope(float* x, const float* bias, const int32_t* positions, const float* cos_t,
                      const float* sin_t, int rope_seq_len, int64_t T, int n_heads, int head_dim) {
  const int D = n_heads * head_dim;
  for (int64_t t = 0; t < T; t++) {
    float* row = x + t * D;
    if (bias)
      for (int j = 0; j < D; j++) row[j] += bias[j];
    if (!cos_t) continue;
    int pos = positions[t];
    if (pos < 0) pos = 0;
    if (pos > rope_seq_len - 1) pos = rope_seq_len - 1;
    for (int h = 0; h < n_heads; h++) {
      float* xh = row + h * head_dim;
      for (int half_i = 0; half_i < head_dim / 2; half_i++) {
        int j0 = 2 * half_i, j1 = j0 + 1;
        float x0 = xh[j0], x1 = xh[j1];
        float c = cos_t[pos * head_dim + j0];
        float s = sin_t[pos * head_dim + j0];
        xh[j0] = x0 * c - x1 * s;
        xh[j1] = x0 * s + x1 * c;
      }
    }
  }
}

void oracle_rmsprop(float* params, const float* grads, float* sq_avg, float lr, float beta, float eps,
                    int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    float g = grads[i];
    sq_avg[i] = beta * sq_avg[i] + (1.0f - beta) * (g * g);
    params[i] -= lr * (g / (sqrtf(sq_avg[i]) + eps));
  }
}
