/*
 * loss_oracle.c — TEST INFRASTRUCTURE ONLY (the checker, never the product).
 * Plain-C restatement of the reference's per-query AGPT loss and its
 * corpus-mass weights. Only tests/ and bench.py's cpu_baseline leg load it
 * (through oracle/liboracle.so).
 *
 * One query at a time, one thread's order: the softmax max and sum run over
 * the row left to right (the reference reduces them in a 2^k-thread tree,
 * agpt_train.cu:2096-2119, which changes the sum's rounding only), then the
 * endpoint / intermediate branch exactly as agpt_train.cu:2121-2193.
 * Compiled with -ffp-contract=off: every float operation rounds on its own.
 * Pinning: tests/test_loss_oracle.py (closed forms, a float64 formulation
 * by log-sum-exp, finite differences of the loss against the gradient, row
 * sums, the entropy weight of two equal counts, mass-weight invariants).
 */
#include "loss_oracle.h"

#include <float.h>
#include <math.h>

/* agpt_train.cu:2069-2194 agpt_loss_per_query_kernel, for every q. */
void oracle_loss_per_query(const float* logits, const int* query_to_node,
                           const int* query_offsets, const int* radix_ids,
                           const int* token_ids, const int* counts_offset,
                           const int* counts_tok, const int* counts_val,
                           const float* mass_weights, float* d_logits, float* loss_out,
                           int T_q, int V, float entropy_lambda, float intermediate_weight,
                           int ce_only) {
  for (int q = 0; q < T_q; q++) {
    const float* in = logits + (long long)q * V;
    float* g = d_logits + (long long)q * V;
    /* softmax: max, exp, sum, times 1/sum (:2096-2119) */
    float mx = -FLT_MAX;
    for (int j = 0; j < V; j++)
      if (in[j] > mx) mx = in[j];
    float sum = 0.0f;
    for (int j = 0; j < V; j++) {
      float e = expf(in[j] - mx);
      g[j] = e;
      sum += e;
    }
    float inv = 1.0f / sum;
    for (int j = 0; j < V; j++) g[j] *= inv;

    int n_idx = query_to_node[q];
    int node_end = query_offsets[n_idx + 1];
    int is_endpoint = (q + 1) == node_end;
    int ce_as_inter = ce_only && is_endpoint && (q + 1 < T_q); /* :2132 */
    if (is_endpoint && !ce_as_inter) {
      /* endpoint: stored counts (:2134-2179) */
      int rid = radix_ids[n_idx];
      int start = counts_offset[rid], end = counts_offset[rid + 1];
      if (start == end) {
        loss_out[q] = 0.0f;
        continue;
      }
      int total = 0;
      for (int e = start; e < end; e++) total += counts_val[e];
      float total_f = (float)total;
      float weight = 1.0f;
      if (entropy_lambda > 0.0f && (end - start) > 1) {
        float H = 0.0f;
        for (int e = start; e < end; e++) {
          float q_e = counts_val[e] / total_f;
          if (q_e > 0.0f) H -= q_e * logf(q_e);
        }
        float log_V = logf((float)V);
        weight = 1.0f + entropy_lambda * (H / log_V);
      }
      if (mass_weights) weight *= mass_weights[q];
      float loss = 0.0f;
      for (int e = start; e < end; e++) {
        int tok = counts_tok[e];
        int cnt = counts_val[e];
        float p = g[tok];
        loss -= (cnt / total_f) * logf(p + 1e-10f);
        g[tok] -= cnt / total_f;
      }
      if (weight != 1.0f) {
        loss *= weight;
        for (int j = 0; j < V; j++) g[j] *= weight;
      }
      loss_out[q] = loss;
    } else {
      /* intermediate: next token of the edge (:2180-2193) */
      int target = token_ids[q + 1];
      float p = g[target];
      float loss = -logf(p + 1e-10f);
      g[target] -= 1.0f;
      float w = intermediate_weight;
      if (mass_weights) w *= mass_weights[q];
      if (w != 1.0f) {
        loss *= w;
        for (int j = 0; j < V; j++) g[j] *= w;
      }
      loss_out[q] = loss;
    }
  }
}

/* agpt_train.cu:4608-4637: per-node weight, query-weighted mean, broadcast. */
void oracle_loss_mass_weights(const int* radix_ids, const int* edge_mass, const int* edge_lens,
                              const int* query_offsets, int n_nodes, int T_q, int mode,
                              float* out) {
  double total_w = 0.0;
  for (int i = 0; i < n_nodes; i++) {
    int r = radix_ids[i];
    float count = (float)edge_mass[r];
    float w = mode == 1 ? logf(1.0f + count) : mode == 2 ? sqrtf(count) : mode == 3 ? count : 1.0f;
    total_w += (double)w * edge_lens[r];
  }
  float mean_w = (T_q > 0) ? (float)(total_w / T_q) : 1.0f;
  if (mean_w <= 0.0f) mean_w = 1.0f;
  for (int i = 0; i < n_nodes; i++) {
    int r = radix_ids[i];
    float count = (float)edge_mass[r];
    float w = mode == 1 ? logf(1.0f + count) : mode == 2 ? sqrtf(count) : mode == 3 ? count : 1.0f;
    for (int q = query_offsets[i]; q < query_offsets[i + 1]; q++) out[q] = w / mean_w;
  }
}
