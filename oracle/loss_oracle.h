/*
 * loss_oracle.h — TEST INFRASTRUCTURE ONLY. Plain-C restatement of the
 * reference's per-query AGPT loss (agpt_train.cu:2069-2194) and corpus-mass
 * weights (agpt_train.cu:4608-4637), used by tests/ and bench.py's
 * cpu_baseline leg as the checker. Nothing in the product links or calls it.
 * Arguments as agpt_loss_per_query / agpt_loss_mass_weights, HOST arrays.
 */
#ifndef AGPT_LOSS_ORACLE_H
#define AGPT_LOSS_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

void oracle_loss_per_query(const float* logits, const int* query_to_node,
                           const int* query_offsets, const int* radix_ids,
                           const int* token_ids, const int* counts_offset,
                           const int* counts_tok, const int* counts_val,
                           const float* mass_weights, float* d_logits, float* loss_out,
                           int T_q, int V, float entropy_lambda, float intermediate_weight,
                           int ce_only);

/* mode: 0 off (weight 1), 1 log(1+m), 2 sqrt(m), 3 m (agpt_train.cu:141). */
void oracle_loss_mass_weights(const int* radix_ids, const int* edge_mass, const int* edge_lens,
                              const int* query_offsets, int n_nodes, int T_q, int mode,
                              float* out);

#ifdef __cplusplus
}
#endif

#endif
