/*
 * trie_attn_oracle.h — TEST INFRASTRUCTURE ONLY. A plain-C restatement of the
 * reference's CPU trie attention, used by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker. Nothing in the product
 * (agpt_amd/, include/) links or calls it.
 *
 * Layouts: Q, K, V, O, dO, dQ, dK, dV are row-major [T, D], D = H*hd, head h
 * at columns h*hd..h*hd+hd-1. parent[i] < i or -1 (depth-1 node); depth[i] is
 * 1-based. Saved weights W are [T, H, wstride] (entries p < depth used).
 */
#ifndef AGPT_TRIE_ATTN_ORACLE_H
#define AGPT_TRIE_ATTN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* agpt_train.cu:2298-2321 build_rope_cache: theta = pos / base^(2i/dim),
 * cos/sin duplicated into lanes 2i and 2i+1; tables [max_seq, dim]. */
void oracle_rope_table(int max_seq, int dim, float base, float* cos_t, float* sin_t);

/* batched_depth_forward.cr:1051-1061 apply_rope_row! on one head slice. */
void oracle_rope_apply(float* x, int hd, const float* cos_t, const float* sin_t, int pos);

/* batched_depth_backward.cr:738-748 apply_inverse_rope_values!. */
void oracle_rope_inverse(float* x, int hd, const float* cos_t, const float* sin_t, int pos);

/* batched_depth_forward.cr:836-971 cpu_grouped_attention, per node:
 * prefix scores as q·K_prefixᵀ, separate self score, scale, softmax_rows,
 * W_prefix·V_prefix + w_self·v_self. Writes O, W and (extra, not in the
 * reference) lse[T, H] = log Σ exp(scaled scores), in double. */
void oracle_fwd_grouped(int64_t T, int H, int hd, const int32_t* parent,
                        const int32_t* depth, const float* Q, const float* K,
                        const float* V, float scale, float* O, float* W, int wstride,
                        float* lse);

/* batched_depth_forward.cr:973-1023 cpu_per_node_attention: scores over the
 * full path (self included) as one product, scale!, softmax, W·V_full. */
void oracle_fwd_per_node(int64_t T, int H, int hd, const int32_t* parent,
                         const int32_t* depth, const float* Q, const float* K,
                         const float* V, float scale, float* O, float* W, int wstride);

/* batched_depth_backward.cr:605-695 optimized_attention_backward_head for
 * one (node, head). path[0..p-1] = ancestor rows by depth (path[p-1] = node).
 * acc_k / acc_v: [T, D] accumulators (NodeGradAccum), read at the node's row
 * and scattered into the ancestors' rows. Writes dq / dk_cur / dv_cur (hd
 * floats each). Inverse RoPE is applied when cos_t != NULL. */
void oracle_bwd_head(int p, const int32_t* path, int h, int H, int hd, const float* w,
                     const float* q_row, const float* dO_row, const float* K,
                     const float* V, float* acc_k, float* acc_v, int pos,
                     const float* cos_t, const float* sin_t, float scale,
                     float* dq, float* dk_cur, float* dv_cur);

/* spec/agpt_backward_attention_spec.cr:212-276 reference_attention_backward_head,
 * the matrix-form twin (W^T·dO, dO·V^T, softmax_backward_row_reference,
 * d_scores·K, d_scoresᵀ·q); same arguments and outputs as oracle_bwd_head. */
void oracle_bwd_head_matrix(int p, const int32_t* path, int h, int H, int hd,
                            const float* w, const float* q_row, const float* dO_row,
                            const float* K, const float* V, float* acc_k, float* acc_v,
                            int pos, const float* cos_t, const float* sin_t, float scale,
                            float* dq, float* dk_cur, float* dv_cur);

/* Whole-trie backward: the per-node loop of batched_depth_backward.cr:236-291
 * run deepest level first over one shared accumulator map, so each node's
 * accumulator holds all of its descendants' contributions when it is
 * consumed. acc_dk_in / acc_dv_in ([T, D] or NULL) seed the accumulators.
 * matrix_form selects oracle_bwd_head_matrix instead of oracle_bwd_head. */
void oracle_bwd_trie(int64_t T, int H, int hd, const int32_t* parent,
                     const int32_t* depth, const float* Q, const float* K,
                     const float* V, const float* W, int wstride, const float* dO,
                     const float* acc_dk_in, const float* acc_dv_in,
                     const float* cos_t, const float* sin_t, int rope_seq_len,
                     float scale, int matrix_form, float* dQ, float* dK, float* dV);

/* Packed varlen semantics of the µGPT externs (agpt_train.cu:73-83,
 * 3106-3132), restated from their call sites: node/query i attends the
 * visible packed rows; weights [(i*H+h)*max_len + p]. */
void oracle_varlen_fwd(int n_nodes, int H, int hd, const float* q, const float* k,
                       const float* v, const int* kv_offsets, const int* kv_lengths,
                       float* out, float* weights, int max_len, float scale);
void oracle_varlen_bwd(int n_nodes, int H, int hd, const float* q, const float* k,
                       const float* v, const float* weights, const float* d_out,
                       const int* kv_offsets, const int* kv_lengths, float* dq,
                       float* dk, float* dv, int max_len, float scale);
void oracle_varlen_L_fwd(int T_q, int H, int hd, const float* q, const float* k,
                         const float* v, const int* query_to_node, const int* query_offsets,
                         const int* kv_offsets, const int* kv_lengths, float* out,
                         float* weights, int max_len, float scale);
/* accumulates into dk / dv */
void oracle_varlen_L_bwd(int T_q, int H, int hd, const float* q, const float* k,
                         const float* v, const float* weights, const float* d_out,
                         const int* query_to_node, const int* query_offsets,
                         const int* kv_offsets, const int* kv_lengths, float* dq,
                         float* dk, float* dv, int max_len, float scale);

#ifdef __cplusplus
}
#endif

#endif
