// trie_build.cpp — host-only synthetic corpus generator and leveled-trie
// builder (libagpt_trie.so). See include/agpt_trie.h for the contract.
//
// The trie is built by sorting the start positions by their path strings:
// in sorted order every prefix first appears right where a DFS preorder with
// ascending child tokens visits it, so one linear pass over the sorted starts
// emits the nodes directly in the row order the attention kernels need
// (subtrees are contiguous row ranges). This replaces the hash-map child
// insertion of TrieCorpus#insert_prefix_step (trie_corpus.cr:893-896) with an
// order-producing build; the node set is the same (trie_corpus.cr:200-228).

#include "../../include/agpt_trie.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

inline uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline double unit_open(uint64_t h) {  // (0, 1)
  return (static_cast<double>(h >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

inline double std_normal(uint64_t key) {  // Box-Muller on two hashed uniforms
  const double u1 = unit_open(splitmix64(key ^ 0x5151515151515151ull));
  const double u2 = unit_open(splitmix64(key ^ 0xA3A3A3A3A3A3A3A3ull));
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

struct Trie {
  std::vector<int32_t> parent, depth, token, end, radix_head, partition;
  // Corpus observations (trie_corpus.cr:210-219): visits[n] = starts whose
  // path passes n; a visit that ends at n (depth limit or corpus end) still
  // observes the next token, kept in (end_node, end_tok) pairs.
  std::vector<int32_t> visits, end_node, end_tok;
  int64_t n_radix = 0, sum_depth = 0, n_root_children = 0, n_parts = 0;
  int32_t max_depth = 0;
};

void finish(Trie* t) {
  const int64_t n = static_cast<int64_t>(t->parent.size());
  t->end.resize(n);
  for (int64_t i = 0; i < n; ++i) t->end[i] = static_cast<int32_t>(i + 1);
  for (int64_t i = n - 1; i >= 0; --i) {
    const int32_t p = t->parent[i];
    if (p >= 0 && t->end[p] < t->end[i]) t->end[p] = t->end[i];
  }
  std::vector<int32_t> nchild(n, 0);
  t->n_root_children = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (t->parent[i] >= 0) nchild[t->parent[i]]++;
    else t->n_root_children++;
  }
  t->radix_head.resize(n);
  t->partition.resize(n);
  t->n_radix = 0;
  t->sum_depth = 0;
  t->max_depth = 0;
  std::vector<int32_t> first_tok(n), second_tok(n);
  for (int64_t i = 0; i < n; ++i) {
    const int32_t p = t->parent[i];
    // A chain continues through a parent with exactly one child
    // (streaming_radix_builder.cr:159-170); root children always start one.
    const int head = (p < 0 || nchild[p] != 1) ? 1 : 0;
    t->radix_head[i] = head;
    t->n_radix += head;
    t->sum_depth += t->depth[i];
    t->max_depth = std::max(t->max_depth, t->depth[i]);
    if (p < 0) {
      first_tok[i] = t->token[i];
      second_tok[i] = 255;
    } else {
      first_tok[i] = first_tok[p];
      second_tok[i] = (t->depth[i] == 2) ? t->token[i] : second_tok[p];
    }
    // Bigram subtree key (streaming_radix_builder.cr:212-240).
    t->partition[i] = ((first_tok[i] & 0xff) << 8) | (second_tok[i] & 0xff);
  }
  std::unordered_set<int32_t> keys(t->partition.begin(), t->partition.end());
  t->n_parts = static_cast<int64_t>(keys.size());
}

}  // namespace

struct agpt_trie_s {
  Trie t;
};

extern "C" int agpt_markov_corpus(uint64_t seed, int order, int vocab, double zipf_s,
                                  double sigma, int64_t n, int32_t* out) {
  if (!out || n < 0 || vocab < 2 || vocab > 65536 || order < 0 || order > 16) return 1;
  std::vector<double> zipf(vocab);
  for (int r = 0; r < vocab; ++r) zipf[r] = std::pow(static_cast<double>(r + 1), -zipf_s);
  std::vector<double> zcdf(vocab);
  std::partial_sum(zipf.begin(), zipf.end(), zcdf.begin());
  auto sample = [&](const double* cdf, uint64_t step) -> int32_t {
    const double u = unit_open(splitmix64(seed ^ 0xC0FFEE1234567ull ^ (step * 0x9E3779B97F4A7C15ull))) *
                     cdf[vocab - 1];
    const int64_t idx = std::upper_bound(cdf, cdf + vocab, u) - cdf;
    return static_cast<int32_t>(idx < vocab ? idx : vocab - 1);
  };
  // Conditional CDFs are cached per context: contexts of a Markov stream repeat.
  std::unordered_map<uint64_t, uint32_t> cache;
  std::vector<double> pool;
  std::vector<double> cdf(vocab);
  for (int64_t i = 0; i < n; ++i) {
    if (i < order) {
      out[i] = sample(zcdf.data(), static_cast<uint64_t>(i));
      continue;
    }
    uint64_t ctx = splitmix64(seed ^ 0x1D872B41ull);
    for (int k = order; k >= 1; --k) ctx = splitmix64(ctx ^ static_cast<uint64_t>(out[i - k] + 1));
    const double* c;
    auto it = cache.find(ctx);
    if (it != cache.end()) {
      c = pool.data() + static_cast<size_t>(it->second) * vocab;
    } else {
      double acc = 0.0;
      for (int x = 0; x < vocab; ++x) {
        const double xi = std_normal(splitmix64(ctx ^ (static_cast<uint64_t>(x) * 0xD6E8FEB86659FD93ull)));
        acc += zipf[x] * std::exp(sigma * xi);
        cdf[x] = acc;
      }
      if (pool.size() < (size_t{1} << 27)) {  // cap the cache at 1 GiB of doubles
        const uint32_t slot = static_cast<uint32_t>(pool.size() / vocab);
        pool.insert(pool.end(), cdf.begin(), cdf.end());
        cache.emplace(ctx, slot);
        c = pool.data() + static_cast<size_t>(slot) * vocab;
      } else {
        c = cdf.data();
      }
    }
    out[i] = sample(c, static_cast<uint64_t>(i));
  }
  return 0;
}

extern "C" int agpt_uniform_tokens(uint64_t seed, int vocab, int64_t n, int32_t* out) {
  if (!out || n < 0 || vocab < 1) return 1;
  for (int64_t i = 0; i < n; ++i)
    out[i] = static_cast<int32_t>(splitmix64(seed * 0x2545F4914F6CDD1Dull + static_cast<uint64_t>(i)) %
                                  static_cast<uint64_t>(vocab));
  return 0;
}

extern "C" int agpt_trie_build(const int32_t* tokens, int64_t n, int max_depth,
                               int64_t max_starts, agpt_trie_handle* out) {
  if (!out || (!tokens && n > 0) || max_depth < 1) return 1;
  *out = nullptr;
  auto* h = new agpt_trie_s();
  Trie& t = h->t;
  const int64_t total_starts = n - 1;  // trie_corpus.cr:203
  std::vector<int64_t> starts;
  if (total_starts > 0) {
    const int64_t count = (max_starts > 0) ? std::min(total_starts, max_starts) : total_starts;
    starts.resize(count);
    if (count == total_starts) {
      std::iota(starts.begin(), starts.end(), int64_t{0});
    } else {  // distributed_starts, trie_corpus.cr:897-913 (start_offset 0)
      for (int64_t i = 0; i < count; ++i) starts[i] = (i * total_starts / count) % total_starts;
    }
  }
  auto len_of = [&](int64_t s) -> int64_t { return std::min<int64_t>(max_depth, total_starts - s); };
  std::sort(starts.begin(), starts.end(), [&](int64_t a, int64_t b) {
    const int64_t la = len_of(a), lb = len_of(b), m = std::min(la, lb);
    for (int64_t i = 0; i < m; ++i) {
      const int32_t x = tokens[a + i], y = tokens[b + i];
      if (x != y) return x < y;
    }
    if (la != lb) return la < lb;
    return a < b;
  });
  std::vector<int32_t> stack(static_cast<size_t>(max_depth) + 1, -1);  // stack[d] = node at depth d
  int64_t prev = -1;
  for (int64_t s : starts) {
    const int64_t len = len_of(s);
    int64_t lcp = 0;
    if (prev >= 0) {
      const int64_t m = std::min(len, len_of(prev));
      while (lcp < m && tokens[s + lcp] == tokens[prev + lcp]) ++lcp;
    }
    for (int64_t d = lcp + 1; d <= len; ++d) {
      const int32_t id = static_cast<int32_t>(t.parent.size());
      t.parent.push_back(stack[d - 1]);
      t.depth.push_back(static_cast<int32_t>(d));
      t.token.push_back(tokens[s + d - 1]);
      t.visits.push_back(0);
      stack[d] = id;
    }
    for (int64_t d = 1; d <= len; ++d) ++t.visits[stack[d]];
    if (len > 0) {  // the last step observes tokens[s + len] (index < total_starts)
      t.end_node.push_back(stack[len]);
      t.end_tok.push_back(tokens[s + len]);
    }
    prev = s;
  }
  finish(&t);
  *out = h;
  return 0;
}

extern "C" int agpt_trie_build_chains(const int32_t* tokens, int64_t n_chains, int chain_len,
                                      agpt_trie_handle* out) {
  if (!out || !tokens || n_chains < 0 || chain_len < 1) return 1;
  auto* h = new agpt_trie_s();
  Trie& t = h->t;
  const int64_t n = n_chains * chain_len;
  t.parent.resize(n);
  t.depth.resize(n);
  t.token.resize(n);
  for (int64_t c = 0; c < n_chains; ++c)
    for (int j = 0; j < chain_len; ++j) {
      const int64_t i = c * chain_len + j;
      t.parent[i] = j == 0 ? -1 : static_cast<int32_t>(i - 1);
      t.depth[i] = j + 1;
      t.token[i] = tokens[i];
    }
  finish(&t);
  *out = h;
  return 0;
}

extern "C" int agpt_trie_stats(agpt_trie_handle h, int64_t* n_nodes, int64_t* n_radix,
                               int64_t* sum_depth, int32_t* max_depth, int64_t* n_root_children,
                               int64_t* n_bigram_parts) {
  if (!h) return 1;
  const Trie& t = h->t;
  if (n_nodes) *n_nodes = static_cast<int64_t>(t.parent.size());
  if (n_radix) *n_radix = t.n_radix;
  if (sum_depth) *sum_depth = t.sum_depth;
  if (max_depth) *max_depth = t.max_depth;
  if (n_root_children) *n_root_children = t.n_root_children;
  if (n_bigram_parts) *n_bigram_parts = t.n_parts;
  return 0;
}

extern "C" int agpt_trie_export(agpt_trie_handle h, int32_t* parent, int32_t* depth,
                                int32_t* token, int32_t* subtree_end, int32_t* radix_head,
                                int32_t* partition) {
  if (!h) return 1;
  const Trie& t = h->t;
  const size_t bytes = t.parent.size() * sizeof(int32_t);
  if (parent) std::memcpy(parent, t.parent.data(), bytes);
  if (depth) std::memcpy(depth, t.depth.data(), bytes);
  if (token) std::memcpy(token, t.token.data(), bytes);
  if (subtree_end) std::memcpy(subtree_end, t.end.data(), bytes);
  if (radix_head) std::memcpy(radix_head, t.radix_head.data(), bytes);
  if (partition) std::memcpy(partition, t.partition.data(), bytes);
  return 0;
}

extern "C" int agpt_trie_export_radix(agpt_trie_handle h, int32_t* radix_parent,
                                      int32_t* edge_len) {
  if (!h) return 1;
  const Trie& t = h->t;
  const int64_t n = static_cast<int64_t>(t.parent.size());
  std::vector<int32_t> radix_of(n, -1);
  int32_t r = -1;
  for (int64_t i = 0; i < n; ++i) {
    if (t.radix_head[i]) {
      ++r;
      const int32_t p = t.parent[i];
      if (radix_parent) radix_parent[r] = p < 0 ? -1 : radix_of[p];
      if (edge_len) edge_len[r] = 0;
    }
    radix_of[i] = r;
    if (edge_len) edge_len[r]++;
  }
  return 0;
}

extern "C" int agpt_trie_next_counts(agpt_trie_handle h, int32_t* visits, int64_t* n_entries,
                                     int32_t* offsets, int32_t* tok, int32_t* val) {
  if (!h || !n_entries) return 1;
  const Trie& t = h->t;
  const int64_t n = static_cast<int64_t>(t.parent.size());
  if (t.visits.size() != static_cast<size_t>(n)) return 2;  // a chain trie has no corpus
  if (visits) std::memcpy(visits, t.visits.data(), n * sizeof(int32_t));
  // Per node: children (DFS order = ascending token) with their visits, then
  // the ending observations merged by token, all in ascending token order.
  std::vector<int32_t> end_first(n, -1), end_next(t.end_node.size(), -1);
  for (int64_t i = static_cast<int64_t>(t.end_node.size()) - 1; i >= 0; --i) {
    end_next[i] = end_first[t.end_node[i]];
    end_first[t.end_node[i]] = static_cast<int32_t>(i);
  }
  std::vector<int32_t> first_child(n, -1), next_sib(n, -1);
  for (int64_t i = n - 1; i >= 0; --i) {
    const int32_t p = t.parent[i];
    if (p >= 0) {
      next_sib[i] = first_child[p];
      first_child[p] = static_cast<int32_t>(i);
    }
  }
  int64_t k = 0;
  std::vector<std::pair<int32_t, int32_t>> hist;
  for (int64_t i = 0; i < n; ++i) {
    if (offsets) offsets[i] = static_cast<int32_t>(k);
    hist.clear();
    for (int32_t c = first_child[i]; c >= 0; c = next_sib[c]) hist.emplace_back(t.token[c], t.visits[c]);
    for (int32_t e = end_first[i]; e >= 0; e = end_next[e]) hist.emplace_back(t.end_tok[e], 1);
    std::sort(hist.begin(), hist.end());
    for (size_t j = 0; j < hist.size(); ++j) {
      if (j > 0 && hist[j].first == hist[j - 1].first) {  // same token: merge into the last entry
        if (val) val[k - 1] += hist[j].second;
        continue;
      }
      if (tok) tok[k] = hist[j].first;
      if (val) val[k] = hist[j].second;
      ++k;
    }
  }
  if (offsets) offsets[n] = static_cast<int32_t>(k);
  *n_entries = k;
  return 0;
}

extern "C" void agpt_trie_free(agpt_trie_handle h) { delete h; }
