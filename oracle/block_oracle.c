/*
 * block_oracle.c — TEST INFRASTRUCTURE ONLY (the checker, never the
 * product). Only tests/ load it (through oracle/liboracle.so).
 *
 * oracle_norm_fwd / _bwd: LayerNorm and RMSNorm with the saved mean /
 * rstd convention of agpt_norm_fwd (µGPT's layer norm is absent).
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
#include <stdlib.h>

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

void oracle_norm_fwd(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
                     int64_t T, int D, float eps) {
  for (int64_t t = 0; t < T; t++) {
    const float* r = x + t * D;
    double mu = 0.0;
    if (b) {
      for (int j = 0; j < D; j++) mu += r[j];
      mu /= D;
    }
    double q = 0.0;
    for (int j = 0; j < D; j++) q += (r[j] - mu) * (r[j] - mu);
    float rs = (float)(1.0 / sqrt(q / D + eps));
    for (int j = 0; j < D; j++) {
      double v = (r[j] - mu) * rs * w[j];
      if (b) v += b[j];
      y[t * D + j] = (float)v;
    }
    rstd[t] = rs;
    if (b) mean[t] = (float)mu;
  }
}

void oracle_norm_bwd(const float* dy, const float* x, const float* w, const float* mean, const float* rstd,
                     float* dx, float* dw, float* db, int64_t T, int D) {
  for (int j = 0; j < D; j++) {
    dw[j] = 0.0f;
    if (db) db[j] = 0.0f;
  }
  double* acw = (double*)calloc((size_t)D, sizeof(double));
  double* acb = (double*)calloc((size_t)D, sizeof(double));
  for (int64_t t = 0; t < T; t++) {
    const double mu = db ? mean[t] : 0.0, r = rstd[t];
    double s1 = 0.0, s2 = 0.0;
    for (int j = 0; j < D; j++) {
      double xh = (x[t * D + j] - mu) * r, g = (double)dy[t * D + j] * w[j];
      s1 += g;
      s2 += g * xh;
      acw[j] += (double)dy[t * D + j] * xh;
      acb[j] += dy[t * D + j];
    }
    s1 = db ? s1 / D : 0.0;
    s2 /= D;
    for (int j = 0; j < D; j++) {
      double xh = (x[t * D + j] - mu) * r;
      dx[t * D + j] = (float)(r * ((double)dy[t * D + j] * w[j] - s1 - xh * s2));
    }
  }
  for (int j = 0; j < D; j++) {
    dw[j] = (float)acw[j];
    if (db) db[j] = (float)acb[j];
  }
  free(acw);
  free(acb);
}
