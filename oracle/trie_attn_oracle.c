/*
 * trie_attn_oracle.c — TEST INFRASTRUCTURE ONLY (the checker, never the
 * product). Plain-C restatement of the reference's Crystal CPU attention for
 * the trie-attention path. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.
 *
 * Arithmetic follows the reference's types: Crystal Float32 products and sums
 * stay float (compiled with -ffp-contract=off, so no fused multiply-adds are
 * introduced), the softmax-backward dot is a Float64 accumulator of Float32
 * products (batched_depth_backward.cr:637-646), and the d_scores expression is
 * evaluated in double and rounded once (:648-651). µGPT's softmax_rows and
 * Mat#* are not available (shard.lock:15-17, not vendored); they are restated
 * as max-subtracted expf / float sum / divide and in-order float dot products.
 * Pinning: see tests/test_oracle.py (two-formulation agreement as in
 * spec/agpt_backward_attention_spec.cr, brute-force masked-dense attention and
 * autograd in torch, finite differences, closed forms and invariants).
 */
#include "trie_attn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* agpt_train.cu:2298-2321 */
void oracle_rope_table(int max_seq, int dim, float base, float* cos_t, float* sin_t) {
  int half = dim / 2;
  for (int pos = 0; pos < max_seq; pos++) {
    for (int i = 0; i < half; i++) {
      float theta = (float)pos / powf(base, 2.0f * (float)i / (float)dim);
      float c = cosf(theta), s = sinf(theta);
      cos_t[pos * dim + 2 * i] = c;
      cos_t[pos * dim + 2 * i + 1] = c;
      sin_t[pos * dim + 2 * i] = s;
      sin_t[pos * dim + 2 * i + 1] = s;
    }
  }
}

/* batched_depth_forward.cr:1051-1061 */
void oracle_rope_apply(float* x, int hd, const float* cos_t, const float* sin_t, int pos) {
  for (int i = 0; i < hd / 2; i++) {
    float c = cos_t[pos * hd + 2 * i], s = sin_t[pos * hd + 2 * i];
    float x0 = x[2 * i], x1 = x[2 * i + 1];
    x[2 * i] = x0 * c - x1 * s;
    x[2 * i + 1] = x0 * s + x1 * c;
  }
}

/* batched_depth_backward.cr:738-748 */
void oracle_rope_inverse(float* x, int hd, const float* cos_t, const float* sin_t, int pos) {
  for (int i = 0; i < hd / 2; i++) {
    float c = cos_t[pos * hd + 2 * i], s = sin_t[pos * hd + 2 * i];
    float x0 = x[2 * i], x1 = x[2 * i + 1];
    x[2 * i] = x0 * c + x1 * s;
    x[2 * i + 1] = -x0 * s + x1 * c;
  }
}

/* Ancestor rows of node n by depth: path[d-1] = ancestor at depth d. */
static int build_path(int64_t n, const int32_t* parent, const int32_t* depth, int32_t* path) {
  int p = depth[n];
  int64_t a = n;
  for (int d = p; d >= 1; d--) {
    path[d - 1] = (int32_t)a;
    a = parent[a];
  }
  return p;
}

static int max_depth_of(int64_t T, const int32_t* depth) {
  int m = 1;
  for (int64_t i = 0; i < T; i++)
    if (depth[i] > m) m = depth[i];
  return m;
}

/* µGPT softmax_rows restated: subtract the row max, expf, float sum, divide. */
static void softmax_row(float* x, int n) {
  float m = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > m) m = x[i];
  float sum = 0.0f;
  for (int i = 0; i < n; i++) {
    x[i] = expf(x[i] - m);
    sum += x[i];
  }
  for (int i = 0; i < n; i++) x[i] = x[i] / sum;
}

static double lse_of(const float* s, int n) {
  double m = s[0];
  for (int i = 1; i < n; i++)
    if (s[i] > m) m = s[i];
  double acc = 0.0;
  for (int i = 0; i < n; i++) acc += exp((double)s[i] - m);
  return m + log(acc);
}

/* batched_depth_forward.cr:836-971 */
void oracle_fwd_grouped(int64_t T, int H, int hd, const int32_t* parent,
                        const int32_t* depth, const float* Q, const float* K,
                        const float* V, float scale, float* O, float* W, int wstride,
                        float* lse) {
  const int D = H * hd;
  const int maxd = max_depth_of(T, depth);
  int32_t* path = (int32_t*)malloc(sizeof(int32_t) * (size_t)maxd);
  float* full = (float*)malloc(sizeof(float) * (size_t)maxd);
  for (int64_t n = 0; n < T; n++) {
    const int p = build_path(n, parent, depth, path);
    const int prefix_len = p - 1;
    for (int h = 0; h < H; h++) {
      const float* q = Q + n * D + h * hd;
      /* scores = q_group * k_prefix.t  (:889-894) */
      for (int pos = 0; pos < prefix_len; pos++) {
        const float* k = K + (int64_t)path[pos] * D + h * hd;
        float acc = 0.0f;
        for (int j = 0; j < hd; j++) acc += q[j] * k[j];
        full[pos] = acc * scale; /* :907-912 */
      }
      /* self score (:897-904) */
      {
        const float* k = K + n * D + h * hd;
        float dot = 0.0f;
        for (int j = 0; j < hd; j++) dot += q[j] * k[j];
        full[prefix_len] = dot * scale;
      }
      if (lse) lse[n * H + h] = (float)lse_of(full, p);
      softmax_row(full, p); /* :915 */
      const float* vself = V + n * D + h * hd;
      const float wself = full[prefix_len];
      for (int j = 0; j < hd; j++) {
        if (prefix_len > 0) { /* out_prefix = w_prefix * v_prefix (:919-937) */
          float acc = 0.0f;
          for (int pos = 0; pos < prefix_len; pos++)
            acc += full[pos] * V[(int64_t)path[pos] * D + h * hd + j];
          O[n * D + h * hd + j] = acc + wself * vself[j];
        } else { /* :938-944 */
          O[n * D + h * hd + j] = wself * vself[j];
        }
      }
      if (W)
        for (int pos = 0; pos < p; pos++) W[(n * H + h) * (int64_t)wstride + pos] = full[pos];
    }
  }
  free(path);
  free(full);
}

/* batched_depth_forward.cr:973-1023 */
void oracle_fwd_per_node(int64_t T, int H, int hd, const int32_t* parent,
                         const int32_t* depth, const float* Q, const float* K,
                         const float* V, float scale, float* O, float* W, int wstride) {
  const int D = H * hd;
  const int maxd = max_depth_of(T, depth);
  int32_t* path = (int32_t*)malloc(sizeof(int32_t) * (size_t)maxd);
  float* sc = (float*)malloc(sizeof(float) * (size_t)maxd);
  for (int64_t n = 0; n < T; n++) {
    const int p = build_path(n, parent, depth, path);
    for (int h = 0; h < H; h++) {
      const float* q = Q + n * D + h * hd;
      for (int pos = 0; pos < p; pos++) { /* scores = q_h * k_full.t */
        const float* k = K + (int64_t)path[pos] * D + h * hd;
        float acc = 0.0f;
        for (int j = 0; j < hd; j++) acc += q[j] * k[j];
        sc[pos] = acc;
      }
      for (int pos = 0; pos < p; pos++) sc[pos] = sc[pos] * scale; /* scale! */
      softmax_row(sc, p);
      for (int j = 0; j < hd; j++) { /* out = weights * v_full */
        float acc = 0.0f;
        for (int pos = 0; pos < p; pos++) acc += sc[pos] * V[(int64_t)path[pos] * D + h * hd + j];
        O[n * D + h * hd + j] = acc;
      }
      if (W)
        for (int pos = 0; pos < p; pos++) W[(n * H + h) * (int64_t)wstride + pos] = sc[pos];
    }
  }
  free(path);
  free(sc);
}

/* batched_depth_backward.cr:605-695 */
void oracle_bwd_head(int p, const int32_t* path, int h, int H, int hd, const float* w,
                     const float* q_row, const float* dO_row, const float* K,
                     const float* V, float* acc_k, float* acc_v, int pos,
                     const float* cos_t, const float* sin_t, float scale,
                     float* dq, float* dk_cur, float* dv_cur) {
  const int D = H * hd;
  float* dw = (float*)malloc(sizeof(float) * (size_t)p);
  float* ds = (float*)malloc(sizeof(float) * (size_t)p);
  double dot = 0.0;
  for (int i = 0; i < p; i++) { /* :637-646 */
    const float* v = V + (int64_t)path[i] * D + h * hd;
    float sum = 0.0f;
    for (int j = 0; j < hd; j++) sum += dO_row[j] * v[j];
    dw[i] = sum;
    dot += (double)(sum * w[i]);
  }
  for (int i = 0; i < p; i++) /* :648-651 */
    ds[i] = (float)((double)w[i] * ((double)dw[i] - dot) * (double)scale);
  for (int j = 0; j < hd; j++) { /* :653-660 */
    float sum = 0.0f;
    for (int i = 0; i < p; i++) sum += ds[i] * K[(int64_t)path[i] * D + h * hd + j];
    dq[j] = sum;
  }
  const int last = p - 1;
  const int64_t self = path[last];
  for (int i = 0; i < p; i++) { /* :667-690 */
    const float sg = ds[i], wt = w[i];
    if (i == last) {
      for (int j = 0; j < hd; j++) {
        dk_cur[j] = sg * q_row[j] + acc_k[self * D + h * hd + j];
        dv_cur[j] = wt * dO_row[j] + acc_v[self * D + h * hd + j];
      }
    } else {
      const int64_t a = path[i];
      for (int j = 0; j < hd; j++) {
        acc_k[a * D + h * hd + j] += sg * q_row[j];
        acc_v[a * D + h * hd + j] += wt * dO_row[j];
      }
    }
  }
  if (cos_t) { /* :693-694 */
    oracle_rope_inverse(dq, hd, cos_t, sin_t, pos);
    oracle_rope_inverse(dk_cur, hd, cos_t, sin_t, pos);
  }
  free(dw);
  free(ds);
}

/* spec/agpt_backward_attention_spec.cr:185-192, 212-276 */
void oracle_bwd_head_matrix(int p, const int32_t* path, int h, int H, int hd,
                            const float* w, const float* q_row, const float* dO_row,
                            const float* K, const float* V, float* acc_k, float* acc_v,
                            int pos, const float* cos_t, const float* sin_t, float scale,
                            float* dq, float* dk_cur, float* dv_cur) {
  const int D = H * hd;
  float* dwt = (float*)malloc(sizeof(float) * (size_t)p);
  float* ds = (float*)malloc(sizeof(float) * (size_t)p);
  float* dk_full = (float*)malloc(sizeof(float) * (size_t)p * (size_t)hd);
  float* dv_full = (float*)malloc(sizeof(float) * (size_t)p * (size_t)hd);
  for (int i = 0; i < p; i++) /* dv_full = attn_weights.t * d_out_h */
    for (int j = 0; j < hd; j++) dv_full[i * hd + j] = w[i] * dO_row[j];
  for (int i = 0; i < p; i++) { /* d_weights = d_out_h * v_h.t */
    const float* v = V + (int64_t)path[i] * D + h * hd;
    float acc = 0.0f;
    for (int j = 0; j < hd; j++) acc += dO_row[j] * v[j];
    dwt[i] = acc;
  }
  double dot = 0.0; /* softmax_backward_row_reference */
  for (int i = 0; i < p; i++) dot += (double)(dwt[i] * w[i]);
  for (int i = 0; i < p; i++) ds[i] = (float)((double)w[i] * ((double)dwt[i] - dot));
  for (int i = 0; i < p; i++) ds[i] = ds[i] * scale; /* d_scores.scale! */
  for (int j = 0; j < hd; j++) { /* dq_h = d_scores * k_h */
    float acc = 0.0f;
    for (int i = 0; i < p; i++) acc += ds[i] * K[(int64_t)path[i] * D + h * hd + j];
    dq[j] = acc;
  }
  for (int i = 0; i < p; i++) /* dk_full = d_scores.t * q_part */
    for (int j = 0; j < hd; j++) dk_full[i * hd + j] = ds[i] * q_row[j];
  const int last = p - 1;
  const int64_t self = path[last];
  for (int j = 0; j < hd; j++) {
    dk_full[last * hd + j] += acc_k[self * D + h * hd + j];
    dv_full[last * hd + j] += acc_v[self * D + h * hd + j];
    dk_cur[j] = dk_full[last * hd + j];
    dv_cur[j] = dv_full[last * hd + j];
  }
  for (int i = 0; i < last; i++) {
    const int64_t a = path[i];
    for (int j = 0; j < hd; j++) {
      acc_k[a * D + h * hd + j] += dk_full[i * hd + j];
      acc_v[a * D + h * hd + j] += dv_full[i * hd + j];
    }
  }
  if (cos_t) {
    oracle_rope_inverse(dq, hd, cos_t, sin_t, pos);
    oracle_rope_inverse(dk_cur, hd, cos_t, sin_t, pos);
  }
  free(dwt);
  free(ds);
  free(dk_full);
  free(dv_full);
}

/* batched_depth_backward.cr:236-291, levels deepest first
 * (trie_walk_trainer.cr:10-14: descendants before ancestors). */
void oracle_bwd_trie(int64_t T, int H, int hd, const int32_t* parent,
                     const int32_t* depth, const float* Q, const float* K,
                     const float* V, const float* W, int wstride, const float* dO,
                     const float* acc_dk_in, const float* acc_dv_in,
                     const float* cos_t, const float* sin_t, int rope_seq_len,
                     float scale, int matrix_form, float* dQ, float* dK, float* dV) {
  const int D = H * hd;
  const int maxd = max_depth_of(T, depth);
  float* acc_k = (float*)calloc((size_t)T * (size_t)D, sizeof(float));
  float* acc_v = (float*)calloc((size_t)T * (size_t)D, sizeof(float));
  if (acc_dk_in) memcpy(acc_k, acc_dk_in, sizeof(float) * (size_t)T * (size_t)D);
  if (acc_dv_in) memcpy(acc_v, acc_dv_in, sizeof(float) * (size_t)T * (size_t)D);
  int32_t* path = (int32_t*)malloc(sizeof(int32_t) * (size_t)maxd);
  /* bucket nodes by depth, keeping index order within a level */
  int64_t* cnt = (int64_t*)calloc((size_t)maxd + 2, sizeof(int64_t));
  for (int64_t i = 0; i < T; i++) cnt[depth[i]]++;
  int64_t* off = (int64_t*)calloc((size_t)maxd + 2, sizeof(int64_t));
  for (int d = 1; d <= maxd; d++) off[d + 1] = off[d] + cnt[d];
  int64_t* order = (int64_t*)malloc(sizeof(int64_t) * (size_t)(T > 0 ? T : 1));
  int64_t* fill = (int64_t*)calloc((size_t)maxd + 2, sizeof(int64_t));
  for (int64_t i = 0; i < T; i++) order[off[depth[i]] + fill[depth[i]]++] = i;
  for (int d = maxd; d >= 1; d--) {
    for (int64_t k = off[d]; k < off[d] + cnt[d]; k++) {
      const int64_t n = order[k];
      const int p = build_path(n, parent, depth, path);
      int pos = p - 1;
      if (cos_t && pos > rope_seq_len - 1) pos = rope_seq_len - 1;
      for (int h = 0; h < H; h++) {
        const float* w = W + (n * H + h) * (int64_t)wstride;
        if (matrix_form)
          oracle_bwd_head_matrix(p, path, h, H, hd, w, Q + n * D + h * hd, dO + n * D + h * hd,
                                 K, V, acc_k, acc_v, pos, cos_t, sin_t, scale,
                                 dQ + n * D + h * hd, dK + n * D + h * hd, dV + n * D + h * hd);
        else
          oracle_bwd_head(p, path, h, H, hd, w, Q + n * D + h * hd, dO + n * D + h * hd, K, V,
                          acc_k, acc_v, pos, cos_t, sin_t, scale, dQ + n * D + h * hd,
                          dK + n * D + h * hd, dV + n * D + h * hd);
      }
    }
  }
  free(acc_k);
  free(acc_v);
  free(path);
  free(cnt);
  free(off);
  free(order);
  free(fill);
}

/* ---- packed varlen (µGPT extern semantics from the call sites) ---------- */

static void varlen_fwd_one(int H, int hd, const float* q, const float* k, const float* v,
                           int64_t qi, int64_t off, int len, float* out, float* weights,
                           int max_len, float scale, float* sc) {
  for (int h = 0; h < H; h++) {
    const float* qq = q + (qi * H + h) * hd;
    for (int p = 0; p < len; p++) {
      const float* kk = k + ((off + p) * H + h) * (int64_t)hd;
      float acc = 0.0f;
      for (int j = 0; j < hd; j++) acc += qq[j] * kk[j];
      sc[p] = acc * scale;
    }
    softmax_row(sc, len);
    for (int j = 0; j < hd; j++) {
      float acc = 0.0f;
      for (int p = 0; p < len; p++) acc += sc[p] * v[((off + p) * H + h) * (int64_t)hd + j];
      out[(qi * H + h) * hd + j] = acc;
    }
    for (int p = 0; p < len; p++) weights[(qi * H + h) * (int64_t)max_len + p] = sc[p];
  }
}

static void varlen_bwd_one(int H, int hd, const float* q, const float* k, const float* v,
                           const float* weights, const float* d_out, int64_t qi, int64_t off,
                           int len, float* dq, float* dk, float* dv, int accumulate,
                           int max_len, float scale, float* dw, float* ds) {
  for (int h = 0; h < H; h++) {
    const float* w = weights + (qi * H + h) * (int64_t)max_len;
    const float* g = d_out + (qi * H + h) * hd;
    const float* qq = q + (qi * H + h) * hd;
    double dot = 0.0;
    for (int p = 0; p < len; p++) {
      const float* vv = v + ((off + p) * H + h) * (int64_t)hd;
      float sum = 0.0f;
      for (int j = 0; j < hd; j++) sum += g[j] * vv[j];
      dw[p] = sum;
      dot += (double)(sum * w[p]);
    }
    for (int p = 0; p < len; p++) ds[p] = (float)((double)w[p] * ((double)dw[p] - dot) * (double)scale);
    for (int j = 0; j < hd; j++) {
      float sum = 0.0f;
      for (int p = 0; p < len; p++) sum += ds[p] * k[((off + p) * H + h) * (int64_t)hd + j];
      dq[(qi * H + h) * hd + j] = sum;
    }
    for (int p = 0; p < len; p++) {
      float* dkr = dk + ((off + p) * H + h) * (int64_t)hd;
      float* dvr = dv + ((off + p) * H + h) * (int64_t)hd;
      for (int j = 0; j < hd; j++) {
        if (accumulate) {
          dkr[j] += ds[p] * qq[j];
          dvr[j] += w[p] * g[j];
        } else {
          dkr[j] = ds[p] * qq[j];
          dvr[j] = w[p] * g[j];
        }
      }
    }
  }
}

void oracle_varlen_fwd(int n_nodes, int H, int hd, const float* q, const float* k,
                       const float* v, const int* kv_offsets, const int* kv_lengths,
                       float* out, float* weights, int max_len, float scale) {
  float* sc = (float*)malloc(sizeof(float) * (size_t)(max_len > 0 ? max_len : 1));
  for (int i = 0; i < n_nodes; i++)
    varlen_fwd_one(H, hd, q, k, v, i, kv_offsets[i], kv_lengths[i], out, weights, max_len, scale, sc);
  free(sc);
}

void oracle_varlen_bwd(int n_nodes, int H, int hd, const float* q, const float* k,
                       const float* v, const float* weights, const float* d_out,
                       const int* kv_offsets, const int* kv_lengths, float* dq,
                       float* dk, float* dv, int max_len, float scale) {
  float* dw = (float*)malloc(sizeof(float) * (size_t)(max_len > 0 ? max_len : 1));
  float* ds = (float*)malloc(sizeof(float) * (size_t)(max_len > 0 ? max_len : 1));
  for (int i = 0; i < n_nodes; i++)
    varlen_bwd_one(H, hd, q, k, v, weights, d_out, i, kv_offsets[i], kv_lengths[i], dq, dk, dv, 0,
                   max_len, scale, dw, ds);
  free(dw);
  free(ds);
}

static int visible_len(int t, const int* query_to_node, const int* query_offsets,
                       const int* kv_lengths) {
  const int i = query_to_node[t];
  const int L = query_offsets[i + 1] - query_offsets[i];
  const int j = t - query_offsets[i];
  return kv_lengths[i] - L + j + 1;
}

void oracle_varlen_L_fwd(int T_q, int H, int hd, const float* q, const float* k,
                         const float* v, const int* query_to_node, const int* query_offsets,
                         const int* kv_offsets, const int* kv_lengths, float* out,
                         float* weights, int max_len, float scale) {
  float* sc = (float*)malloc(sizeof(float) * (size_t)(max_len > 0 ? max_len : 1));
  for (int t = 0; t < T_q; t++) {
    const int i = query_to_node[t];
    varlen_fwd_one(H, hd, q, k, v, t, kv_offsets[i],
                   visible_len(t, query_to_node, query_offsets, kv_lengths), out, weights, max_len,
                   scale, sc);
  }
  free(sc);
}

void oracle_varlen_L_bwd(int T_q, int H, int hd, const float* q, const float* k,
                         const float* v, const float* weights, const float* d_out,
                         const int* query_to_node, const int* query_offsets,
                         const int* kv_offsets, const int* kv_lengths, float* dq,
                         float* dk, float* dv, int max_len, float scale) {
  float* dw = (float*)malloc(sizeof(float) * (size_t)(max_len > 0 ? max_len : 1));
  float* ds = (float*)malloc(sizeof(float) * (size_t)(max_len > 0 ? max_len : 1));
  for (int t = 0; t < T_q; t++) {
    const int i = query_to_node[t];
    varlen_bwd_one(H, hd, q, k, v, weights, d_out, t, kv_offsets[i],
                   visible_len(t, query_to_node, query_offsets, kv_lengths), dq, dk, dv, 1,
                   max_len, scale, dw, ds);
  }
  free(dw);
  free(ds);
}
