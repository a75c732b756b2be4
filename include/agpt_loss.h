/*
 * agpt_loss.h — C ABI of the per-query AGPT loss (libagpt_attn.so, gfx950).
 *
 * Shares the conventions of agpt_attn.h: int status (AGPT_OK = 0) with the
 * message in agpt_last_error(), DEVICE pointers owned by the caller, work
 * ordered on the stream passed in (NULL = default stream), deterministic
 * results (no atomics; every sum in a fixed order).
 */
#ifndef AGPT_LOSS_H
#define AGPT_LOSS_H

#include "agpt_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Corpus-mass weighting modes (agpt_train.cu:141 MassWeightMode). */
#define AGPT_MASS_OFF     0
#define AGPT_MASS_LOG     1
#define AGPT_MASS_SQRT    2
#define AGPT_MASS_LINEAR  3

/* Replaces launch_agpt_loss_per_query (agpt_train.cu:2199-2216; kernel
 * agpt_loss_per_query_kernel :2069-2194), same arguments plus the trailing
 * stream. logits / d_logits [T_q, V] fp32 row-major; query q belongs to radix
 * node n = query_to_node[q], whose queries are query_offsets[n] ..
 * query_offsets[n+1]-1; q is that node's endpoint when q + 1 ==
 * query_offsets[n+1]. Endpoints read the next-token counts
 * counts_tok / counts_val [counts_offset[radix_ids[n]] .. counts_offset[radix_ids[n]+1]),
 * intermediates (and endpoints when ce_only != 0 and q + 1 < T_q) the
 * single target token_ids[q+1]. Writes d_logits (softmax minus target,
 * weighted) and loss_out [T_q]. mass_weights [T_q] or NULL.
 * Count entries or targets outside [0, V) are skipped (the reference
 * would index past the row). V up to 1024. */
int agpt_loss_per_query(const float* logits, const int* query_to_node,
                        const int* query_offsets, const int* radix_ids,
                        const int* token_ids, const int* counts_offset,
                        const int* counts_tok, const int* counts_val,
                        const float* mass_weights, float* d_logits, float* loss_out,
                        int T_q, int V, float entropy_lambda, float intermediate_weight,
                        int ce_only, void* stream);

/* Host-only: the per-query corpus-mass weights of agpt_train.cu:4608-4637.
 * HOST arrays: radix_ids [n_nodes] (radix id of chunk node i), edge_mass and
 * edge_lens indexed by radix id, query_offsets [n_nodes+1]; writes
 * out [T_q] = f(edge_mass) / mean, f = log(1+m) | sqrt(m) | m | 1 by mode,
 * mean = sum_i f_i * edge_len_i / T_q (1 if not positive). */
int agpt_loss_mass_weights(const int* radix_ids, const int* edge_mass, const int* edge_lens,
                           const int* query_offsets, int n_nodes, int T_q, int mode,
                           float* out);

#ifdef __cplusplus
}
#endif

#endif /* AGPT_LOSS_H */
