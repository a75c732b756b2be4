/*
 * agpt_attn.h — C ABI of the MI355X (gfx950) trie-scoped attention library
 * (libagpt_attn.so).
 *
 * The path: every trie node n (one node-token = one query position) attends
 * over the K/V rows of its root->n ancestor path a_1..a_p (a_p = n,
 * p = depth(n)), per head:
 *     s_j = (q_n . k_{a_j}) * scale,  w = softmax(s),  o_n = sum_j w_j v_{a_j}
 * and the backward pass returns dQ, and dK/dV reduced over each key's whole
 * subtree:
 *     dK[a] = R(pos_a)^T ( sum_{n in subtree(a)} ds_{n,depth(a)} q_n + ACC_k[a] )
 *     dV[a] =              sum_{n in subtree(a)} w_{n,depth(a)} dO_n + ACC_v[a]
 * where ds_j = w_j (dO.v_j - sum_i w_i dO.v_i) * scale, and R is the RoPE
 * rotation at the owner's position pos = min(depth-1, rope_seq_len-1).
 *
 * Reference semantics followed:
 *   forward   src/agpt/batched_depth_forward.cr:836-971 (cpu_grouped_attention)
 *   backward  src/agpt/batched_depth_backward.cr:605-695
 *             (optimized_attention_backward_head), accumulators
 *             src/agpt/node_state.cr:58-74, inverse RoPE :738-748.
 *
 * Conventions shared by every entry point:
 *   - Every function returns an int status (AGPT_OK = 0); none exits or
 *     aborts. agpt_last_error() returns a message for the last failure on
 *     the calling thread.
 *   - Tensor pointers are DEVICE pointers owned by the caller, row-major
 *     [T, D] with D = n_heads * head_dim and head h at columns
 *     h*head_dim .. h*head_dim+head_dim-1 (the [N, d_model] layout of
 *     batched_depth_forward.cr:658-664 / agpt_train.cu:4746-4749).
 *   - Work is ordered on the stream passed in (NULL = default stream); no
 *     entry point synchronises the device except agpt_sync().
 *   - Results are deterministic: no floating-point atomics anywhere, every
 *     reduction runs in a fixed order, so two calls give identical bytes.
 */
#ifndef AGPT_ATTN_H
#define AGPT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define AGPT_OK               0
#define AGPT_ERR_INVALID_ARG  1  /* null pointer, bad size, misaligned buffer */
#define AGPT_ERR_NOT_DFS      2  /* parent table is not a DFS preorder forest */
#define AGPT_ERR_NO_PLAN      3  /* fwd/bwd called before a successful plan   */
#define AGPT_ERR_UNSUPPORTED  4  /* head_dim / dtype / depth not built         */
#define AGPT_ERR_DEVICE       5  /* a HIP runtime call failed                  */
#define AGPT_ERR_TOO_DEEP     6  /* a node is deeper than config.max_depth     */

/* ---- input element types (Q, K, V, O, dO); gradients are always fp32 --- */
#define AGPT_DTYPE_F32   0
#define AGPT_DTYPE_BF16  1

typedef struct agpt_attn_s* agpt_attn_handle;

typedef struct {
    int n_heads;    /* H, uniform heads (batched_depth_forward.cr:646)        */
    int head_dim;   /* hd: 4, 8, 16, 32 or 64                                 */
    int max_depth;  /* upper bound on node depth = keys per query, 1..256     */
    int dtype;      /* AGPT_DTYPE_F32 or AGPT_DTYPE_BF16                      */
} agpt_attn_config;

typedef struct {
    float scale;              /* 0 => 1/sqrt(head_dim), as batched_depth_forward.cr:878 */
    const float* rope_cos;    /* device [rope_seq_len, head_dim] or NULL = no RoPE      */
    const float* rope_sin;    /* same layout; entry [pos, 2i] is used for pair (2i,2i+1) */
    int rope_seq_len;         /* positions are clamped to rope_seq_len-1 (agpt_train.cu:4471-4473) */
    void* stream;             /* hipStream_t, NULL = default stream                      */
    /* Optional profiling hook: when prof_events != NULL, the library records
     * prof_events[0] on the stream before its first kernel and
     * prof_events[i+1] after its i-th kernel, for i < n_prof_events-1.
     * The events (hipEvent_t) are created and owned by the caller. */
    void** prof_events;
    int n_prof_events;
    /* Backward of a range plan (agpt_attn_plan_range) only: an event
     * (hipEvent_t, or NULL) that the reduction of the context rows' dK/dV
     * waits for on the stream before it starts. The batches of one trie may
     * then run on several streams: each batch passes the event its caller
     * recorded after the previous batch's backward, so the context rows
     * (rows that an earlier batch wrote) get their additions in batch order
     * while the batches' other kernels overlap. */
    void* ctx_wait;
} agpt_attn_opts;

/* Message describing the last failure on this thread ("" if none). */
const char* agpt_last_error(void);

/* Library / kernel build identification string. */
const char* agpt_version(void);

/* ---- handle-based trie attention ---------------------------------------- */

/* Creates a handle holding the plan and the device workspace.
 * Replaces the per-call cudaMalloc/cudaFree of batched_depth_forward.cr:747-755,
 * 820-823 and the static lazily-grown buffers of agpt_train.cu:4543-4572. */
int agpt_attn_create(const agpt_attn_config* cfg, agpt_attn_handle* out);

/* Frees the handle and its device workspace. NULL is accepted. */
int agpt_attn_destroy(agpt_attn_handle h);

/* Validates and uploads the tree of one batch (a subtree, a bigram partition
 * or a whole trie). parent is a HOST array of n_nodes entries in DFS preorder:
 * parent[i] is the row index of i's parent (parent[i] < i) or -1 for a
 * depth-1 node (a child of the trie root, which has no K/V row). Every
 * subtree must be a contiguous range of rows. Allocates the device tables and
 * the reduction workspace (the only allocating call besides create).
 * Replaces the per-chunk host packing + 13 H2D copies of
 * agpt_train.cu:4444-4590 and the ancestor lists of
 * batched_depth_forward.cr:342-361. */
int agpt_attn_plan(agpt_attn_handle h, const int32_t* parent, int64_t n_nodes);

/* Batches of one trie: a contiguous range of its DFS rows, e.g. a run of
 * bigram partitions (the reference's --partition-depth batching,
 * agpt_train.cu:3808-3890; subtree keys streaming_radix_builder.cr:212-240).
 * The reference truncates the ancestor chain of a partition whose root
 * child lives in another file (its known approximation,
 * streaming_radix_builder.cr:46-55); here every row of the range attends
 * its whole path: the ancestors of row_begin that lie before the range (the
 * range's context, at most max_depth-1 rows) are read as keys, and the
 * range's share of their dK/dV is returned to them:
 *   AGPT_CTX_GLOBAL: fwd/bwd take the whole trie's tensors ([n_total, D]);
 *     the range's rows are read and written in place, and bwd ADDS the
 *     range's share of dK/dV of each context row into that row of dK/dV
 *     (seeds and inverse RoPE as usual: the sum of the parts is the whole).
 *     The batch holding a row as a query writes it, so the ranges of a trie
 *     run in ascending row order, on one stream (or ordered by the caller).
 *   AGPT_CTX_PACKED: fwd/bwd take tensors holding the range alone, after its
 *     n_ctx context rows: rows 0..n_ctx-1 are the ancestors of row_begin,
 *     root first (the reference's suggested context-only duplicate,
 *     streaming_radix_builder.cr:53-55), then the range's rows. bwd WRITES
 *     the range's share of dK/dV of the context rows into rows 0..n_ctx-1
 *     (no seeds there; inverse RoPE applied) for the caller to add to their
 *     owners; O, lse and dQ of those rows are not written.
 * Context rows are keys only: they are not queries of the range. */
#define AGPT_CTX_GLOBAL 0
#define AGPT_CTX_PACKED 1

/* Plans rows [row_begin, row_end) of a trie whose whole DFS parent table
 * (n_total rows, host memory) is `parent`, as described above. n_ctx =
 * depth(row_begin) - 1 (agpt_attn_plan_info's max_depth and n_nodes refer to
 * the range). agpt_attn_plan(h, parent, n) is this with the whole trie. */
int agpt_attn_plan_range(agpt_attn_handle h, const int32_t* parent, int64_t n_total,
                         int64_t row_begin, int64_t row_end, int ctx_mode);

/* Size of the static scratch array agpt_attn_plan_static places a plan in,
 * per device. */
#define AGPT_STATIC_SCRATCH_BYTES (64u << 20)

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc, code that
 * captures fwd/bwd into a HIP graph: plan before the capture, since the
 * uploads here are synchronous hipMemcpy calls, which a capture does not
 * allow; fwd/bwd of the plan may then be captured). Same contract and results as agpt_attn_plan, but every
 * device table and workspace of the plan is placed in a static array of the
 * library (AGPT_STATIC_SCRATCH_BYTES = 64 MiB per device, held until the
 * process ends) instead of being allocated: the call makes no hipMalloc or
 * hipFree (its only device calls are hipMemcpy uploads of the tables and,
 * once per device, hipGetSymbolAddress). A batch needing more returns
 * AGPT_ERR_INVALID_ARG with the bytes it needs (an fp32 batch with 8 heads
 * x 16 at depth 32 fits up to ~60K node-tokens). fwd/bwd then run unchanged.
 * Every static plan on a device shares that device's array: each call takes
 * it over, and fwd/bwd of a handle whose plan an earlier static plan made
 * return AGPT_ERR_NO_PLAN. Work of the previous static plan still running on
 * a stream races with this call's uploads: the caller orders them. Rejects a
 * handle that holds an allocated plan (releasing it would call hipFree). */
int agpt_attn_plan_static(agpt_attn_handle h, const int32_t* parent, int64_t n_nodes);

/* agpt_attn_plan, but the tree arrives as radix nodes (agpt_train.cu:892-940): radix
 * node r (DFS preorder, radix_parent[r] < r or -1) owns edge_len[r] >= 1
 * consecutive node-token rows; row j of the edge has the edge's previous row
 * as parent. Row order: radix nodes in order, edge rows in order. */
int agpt_attn_plan_radix(agpt_attn_handle h, const int32_t* radix_parent,
                         const int32_t* edge_len, int64_t n_radix);

/* Host-only: the node-token rows of a radix tree, as agpt_attn_plan_radix
 * plans them (the ancestor chains of agpt_train.cu:892-940 expanded into one
 * parent per row). Writes *n_rows = Σ edge_len and, if parent_out is
 * non-NULL, the rows' parent table (cap entries at most: a smaller cap
 * returns AGPT_ERR_INVALID_ARG after setting *n_rows). Errors: AGPT_ERR_NOT_DFS
 * for a radix_parent that is not an earlier node or -1, AGPT_ERR_INVALID_ARG
 * for edge_len < 1 or more than 2^31 rows. No device calls. */
int agpt_attn_radix_rows(const int32_t* radix_parent, const int32_t* edge_len, int64_t n_radix,
                         int32_t* parent_out, int64_t cap, int64_t* n_rows);

/* Planned batch statistics (host values): node-tokens T, number of tiles,
 * sum of depths (keys attended, Σp), maximum depth. Any pointer may be NULL. */
int agpt_attn_plan_info(agpt_attn_handle h, int64_t* n_nodes, int64_t* n_tiles,
                        int64_t* sum_depth, int32_t* max_depth);

/* Describes the kernel variant chosen for the planned batch (e.g. LDS-staged,
 * heads per workgroup, LDS bytes); valid until the next plan or destroy. */
const char* agpt_attn_describe(agpt_attn_handle h);

/* Forward. Q (post-RoPE), K (post-RoPE), V: [T, D] of cfg.dtype.
 * Writes O [T, D] (cfg.dtype) and lse [T, H] fp32, the natural-log
 * log-sum-exp of each query's scaled scores (it replaces the saved weights
 * [T, H, p] of node_state.cr:10: w_j = exp(s_j - lse)). */
int agpt_attn_fwd(agpt_attn_handle h, const void* q, const void* k, const void* v,
                  void* o, float* lse, const agpt_attn_opts* opts);

/* Backward. Reads Q, K, V, O, dO (cfg.dtype) and lse from agpt_attn_fwd.
 * Writes dQ, dK, dV [T, D] fp32 (pre-RoPE space for dQ and dK when RoPE is
 * on). acc_dk / acc_dv (fp32 [T, D], or NULL) are external descendant
 * contributions added to each node's own dK/dV before inverse RoPE, the
 * seeded NodeGradAccum of batched_depth_backward.cr:671-675. */
int agpt_attn_bwd(agpt_attn_handle h, const void* q, const void* k, const void* v,
                  const void* o, const float* lse, const void* d_o,
                  float* dq, float* dk, float* dv,
                  const float* acc_dk, const float* acc_dv,
                  const agpt_attn_opts* opts);

/* Host-only plan check (no device call): validates a DFS-preorder parent
 * table and fills depth[i] (1-based) and subtree_end[i] (exclusive) when
 * the pointers are non-NULL. Returns AGPT_ERR_NOT_DFS with a message if the
 * order is not a preorder with contiguous subtrees. */
int agpt_attn_check_tree(const int32_t* parent, int64_t n_nodes,
                         int32_t* depth, int32_t* subtree_end);

/* Host-only: a DFS-preorder permutation of an arbitrary forest.
 * perm[k] = original row placed at position k; children keep their
 * relative order. parent uses original indices (-1 for depth 1). */
int agpt_attn_dfs_order(const int32_t* parent, int64_t n_nodes, int32_t* perm);

/* ---- drop-ins for the reference's packed varlen calls --------------------
 * Same argument meaning as the µGPT externs the reference binds
 * (agpt_train.cu:73-86, 3120-3132; Crystal call sites
 * batched_depth_forward.cr:767-778, batched_depth_backward.cr:471-476,
 * agpt_train.cu:4740-4744, 4988-4992), fp32 device buffers, packed layouts:
 *   q / output / dq      [(i*H + h)*hd + j]           (i = node or query)
 *   k / v / dk / dv      [((kv_off + p)*H + h)*hd + j]
 *   weights              [(i*H + h)*max_len + p]       (p < visible length)
 * The extra trailing `stream` argument (NULL = default stream) is the only
 * signature change; every function returns a status instead of void. */

/* batched_depth_forward.cr:767 / agpt_train.cu:73-77: node i attends the
 * kv_lengths[i] packed rows starting at kv_offsets[i]. */
int agpt_varlen_attention(const float* q_packed, const float* k_packed,
                          const float* v_packed, const int* kv_offsets,
                          const int* kv_lengths, float* output, float* weights_out,
                          int n_nodes, int n_heads, int head_dim, int max_len,
                          float scale, void* stream);

/* batched_depth_backward.cr:471 / agpt_train.cu:78-83: from the saved
 * weights; writes dq and the packed dk_full / dv_full rows of every node
 * (each packed row belongs to one node, so the rows are overwritten). */
int agpt_varlen_attention_backward(const float* q_packed, const float* k_packed,
                                   const float* v_packed, const float* attn_weights,
                                   const float* d_out, const int* kv_offsets,
                                   const int* kv_lengths, float* dq, float* dk_full,
                                   float* dv_full, int n_nodes, int n_heads,
                                   int head_dim, int max_len, float scale,
                                   void* stream);

/* agpt_train.cu:84-86: packed [(i*H+h)*hd + j] -> [N, D]. Both layouts are
 * the same bytes (agpt_train.cu:4746-4749), so this is a device copy. */
int agpt_unpack_batched_attn_output(const float* packed_output, float* unpacked_output,
                                    int n_nodes, int n_heads, int head_dim,
                                    void* stream);

/* agpt_train.cu:3120-3125: query t belongs to radix node i =
 * query_to_node[t], j = t - query_offsets[i]; it attends the first
 * kv_lengths[i] - L_i + j + 1 rows of node i's packed prefix
 * (L_i = query_offsets[i+1] - query_offsets[i]: ancestors + edge[0..j]). */
int agpt_varlen_attention_L_queries(const float* q_packed, const float* k_packed,
                                    const float* v_packed, const int* query_to_node,
                                    const int* query_offsets, const int* kv_offsets,
                                    const int* kv_lengths, float* output,
                                    float* weights_out, int T_q, int n_heads,
                                    int head_dim, int max_kv_len, float scale,
                                    void* stream);

/* agpt_train.cu:3126-3132: ACCUMULATES into dk_full / dv_full (the caller
 * zeroes them first, agpt_train.cu:4982-4984); writes dq. The queries of one
 * radix node must be consecutive (query_offsets ascending), as the chunk
 * packer of agpt_train.cu:4456-4479 lays them out. */
int agpt_varlen_attention_L_queries_backward(const float* q_packed, const float* k_packed,
                                             const float* v_packed,
                                             const float* attn_weights,
                                             const float* d_out,
                                             const int* query_to_node,
                                             const int* query_offsets,
                                             const int* kv_offsets,
                                             const int* kv_lengths, float* dq,
                                             float* dk_full, float* dv_full, int T_q,
                                             int n_heads, int head_dim, int max_kv_len,
                                             float scale, void* stream);

/* agpt_train.cu:87 cuda_sync(): waits for the device. */
int agpt_sync(void);

#ifdef __cplusplus
}
#endif

#endif /* AGPT_ATTN_H */
