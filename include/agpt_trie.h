/*
 * agpt_trie.h — host-only C ABI of libagpt_trie.so: the seeded synthetic
 * corpus generator and the trie builder that produce the inputs of the
 * trie-attention path (node-token parent tables in DFS preorder).
 *
 * The reference builds its tries offline with Crystal tools
 * (src/agpt/trie_corpus.cr:200-228 ingest, src/agpt/streaming_radix_builder.cr
 * radix compression and subtree keys); these functions restate only the parts
 * that define the attention inputs: which prefixes become nodes, their
 * parent/child structure and depth, radix-chain heads, and the unigram /
 * bigram partition key. No device code; safe to call without a GPU.
 */
#ifndef AGPT_TRIE_H
#define AGPT_TRIE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct agpt_trie_s* agpt_trie_handle;

/* Seeded order-k Markov corpus over `vocab` symbols. Symbol r has marginal
 * rank r with Zipf weight (r+1)^-zipf_s; the conditional law given the last
 * `order` symbols is p(x|ctx) ∝ (x+1)^-zipf_s * exp(sigma * xi(ctx, x)),
 * xi ~ N(0,1) drawn from a counter-based generator keyed by (seed, ctx, x).
 * Writes n tokens. Returns 0 on success. */
int agpt_markov_corpus(uint64_t seed, int order, int vocab, double zipf_s,
                       double sigma, int64_t n, int32_t* out_tokens);

/* Uniform i.i.d. tokens in [0, vocab) from seed (the chain-control corpus). */
int agpt_uniform_tokens(uint64_t seed, int vocab, int64_t n, int32_t* out_tokens);

/* Leveled trie of a token stream with TrieCorpus#ingest semantics
 * (trie_corpus.cr:200-228): starts are 0..n-2 (or max_starts of them spread
 * evenly, trie_corpus.cr:897-913, when max_starts > 0); each start inserts the
 * path tokens[start .. start+len) with len = min(max_depth, n-1-start).
 * Nodes come out in DFS preorder with children in ascending token order. */
int agpt_trie_build(const int32_t* tokens, int64_t n, int max_depth,
                    int64_t max_starts, agpt_trie_handle* out);

/* The trie the reference's on-disk radix pipeline trains on
 * (src/tools/build_index.cr + build_radix.cr): StreamingLeveledBuilder#build
 * (streaming_leveled_builder.cr:48-108) inserts every start 0..n-2 with a
 * path that runs while the next position is inside the corpus, so paths
 * near the end reach the corpus' last token (a node with no next-token
 * observation); StreamingRadixBuilder#build (streaming_radix_builder.cr:
 * 149-180) then runs an edge on through nodes with exactly one next-token
 * entry and drops every edge whose endpoint has none (the end-of-corpus
 * leaf). The result holds the node-tokens of the kept radix edges, DFS
 * preorder, children by ascending token; its counts are the leveled
 * nodes' own (a parent keeps the entry of a dropped child). */
int agpt_trie_build_radix(const int32_t* tokens, int64_t n, int max_depth,
                          agpt_trie_handle* out);

/* One root child's subtree of agpt_trie_build_radix's trie: the same
 * pipeline over the starts whose first token is first_token only, so a
 * corpus whose whole trie does not fit is built (and batched) one root
 * child at a time; the subtrees in token order are the whole trie's rows
 * in order (the reference's per-subtree files, streaming_radix_builder.cr:
 * 388-426, hold the same subtrees). */
int agpt_trie_build_radix_part(const int32_t* tokens, int64_t n, int max_depth,
                               int32_t first_token, agpt_trie_handle* out);

/* `n_chains` independent unary chains of `chain_len` nodes each (never
 * merged); chain c takes tokens[c*chain_len ...]. The dense-causal control. */
int agpt_trie_build_chains(const int32_t* tokens, int64_t n_chains, int chain_len,
                           agpt_trie_handle* out);

/* Node-token count T, radix-node count (edge heads: a root child, or a node
 * whose parent has not exactly one next-token entry, streaming_radix_builder.cr:
 * 155-170; a chain trie: a parent without exactly one child),
 * Σ depth, max depth, number of root children, number of bigram partitions. */
int agpt_trie_stats(agpt_trie_handle t, int64_t* n_nodes, int64_t* n_radix,
                    int64_t* sum_depth, int32_t* max_depth, int64_t* n_root_children,
                    int64_t* n_bigram_parts);

/* Copies the per-node tables (any pointer may be NULL), each of T entries:
 * parent (-1 for depth 1), depth (1-based), token, subtree_end (exclusive),
 * radix_head (1 if the node starts a radix edge), partition (bigram subtree
 * key (first_token << 8) | second_token, second_token = 255 for depth-1
 * nodes, the sentinel of streaming_radix_builder.cr:219-224). */
int agpt_trie_export(agpt_trie_handle t, int32_t* parent, int32_t* depth,
                     int32_t* token, int32_t* subtree_end, int32_t* radix_head,
                     int32_t* partition);

/* Radix view: number of radix nodes R, then per radix node (DFS preorder)
 * its radix parent (-1 for root children) and edge length. */
int agpt_trie_export_radix(agpt_trie_handle t, int32_t* radix_parent,
                           int32_t* edge_len);

/* Corpus observations of a trie built by agpt_trie_build (TrieCorpus#ingest
 * + #observe, trie_corpus.cr:200-228) or agpt_trie_build_radix:
 * visits[i] = starts whose path passes node i; node i's next-token counts
 * (every visit observes the token after its prefix, also where the path
 * stops at the depth limit, except a visit ending on the corpus' last
 * token) as CSR over the T nodes: entries offsets[i] .. offsets[i+1]-1 of
 * tok / val, tokens ascending. Call first with tok = val = offsets = NULL
 * to get n_entries. Returns 2 for a chain trie (no corpus). */
int agpt_trie_next_counts(agpt_trie_handle t, int32_t* visits, int64_t* n_entries,
                          int32_t* offsets, int32_t* tok, int32_t* val);

/* ---- radix subtree files ---------------------------------------------------
 * The reference's on-disk radix trie, format v2 (streaming_radix_builder.cr:
 * 10-32, 388-470): out_dir/subtrees/radix_subtree_%06d.bin (one per root
 * child, keyed by its radix id), out_dir/manifest.bin, out_dir/meta.bin.
 * Record: radix_id, parent_radix_id (0 = virtual root), first_char_depth,
 * edge_len, edge tokens, edge_mass (count of the edge's first node),
 * entry_count, (token, count) entries of the endpoint's next-token counts. */
typedef struct agpt_radix_s* agpt_radix_handle;

/* Writes the radix files of a trie built with agpt_trie_build or
 * agpt_trie_build_radix (needs its corpus counts) as the reference's builder does (streaming_radix_builder.cr:
 * 100-330): edge starts breadth first from the root, radix ids in that order
 * from 1, an edge extended while its end has exactly one next-token entry
 * and that child exists, edge_mass = the sum of the head's counts, meta's
 * corpus_token_count = the corpus length. out_dir and out_dir/subtrees must
 * exist. */
int agpt_radix_write_subtrees(agpt_trie_handle t, const char* out_dir, int32_t vocab_size);

/* Reads one radix_subtree_%06d.bin (agpt_train.cu:495-669 load_subtree):
 * global ids mapped to local ones, radix nodes reordered to DFS preorder with
 * children by ascending first token (what agpt_attn_plan_radix takes).
 * Returns 2 (cannot open), 3 (bad magic), 4 (bad version), 5 (malformed). */
int agpt_radix_read_subtree(const char* path, agpt_radix_handle* out);

/* Sizes of a read subtree: radix nodes R, edge chars (node-tokens), count
 * entries, the root child's radix id, the deepest endpoint. */
int agpt_radix_info(agpt_radix_handle r, int64_t* n_radix, int64_t* n_chars, int64_t* n_entries,
                    int32_t* root_child_id, int32_t* max_endpoint_depth);

/* Copies the DFS-ordered tables (any pointer may be NULL): per radix node
 * [R] its global radix id, local parent (-1 for the root child),
 * first_char_depth, edge_len, edge_mass; edge_tokens [chars] in row order;
 * the endpoint counts as CSR counts_offset [R+1], counts_tok, counts_val. */
int agpt_radix_export(agpt_radix_handle r, int32_t* radix_id, int32_t* radix_parent,
                      int32_t* first_char_depth, int32_t* edge_len, int32_t* edge_mass,
                      int32_t* edge_tokens, int32_t* counts_offset, int32_t* counts_tok,
                      int32_t* counts_val);

void agpt_radix_free(agpt_radix_handle r);

void agpt_trie_free(agpt_trie_handle t);

#ifdef __cplusplus
}
#endif

#endif /* AGPT_TRIE_H */
