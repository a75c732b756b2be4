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
#include <array>
#include <cstdio>
#include <map>
#include <string>
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
  // Corpus observations: visits[n] = starts whose path passes n; the
  // next-token counts of n as CSR (coff [T+1], ctok, cval; tokens
  // ascending). Empty for a chain trie (no corpus).
  std::vector<int32_t> visits, coff, ctok, cval;
  int64_t n_corpus = 0;
  int64_t n_radix = 0, sum_depth = 0, n_root_children = 0, n_parts = 0;
  int32_t max_depth = 0;
};

// Tables derived from parent / depth / token (and radix_head when
// `heads_set`: a corpus trie decides its radix heads from counts).
void finish(Trie* t, bool heads_set) {
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
  if (!heads_set) {
    // No corpus: a chain continues through a parent with exactly one child.
    t->radix_head.resize(n);
    for (int64_t i = 0; i < n; ++i) {
      const int32_t p = t->parent[i];
      t->radix_head[i] = (p < 0 || nchild[p] != 1) ? 1 : 0;
    }
  }
  t->partition.resize(n);
  t->n_radix = 0;
  t->sum_depth = 0;
  t->max_depth = 0;
  std::vector<int32_t> first_tok(n), second_tok(n);
  for (int64_t i = 0; i < n; ++i) {
    const int32_t p = t->parent[i];
    t->n_radix += t->radix_head[i];
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

// Path length of a start: how many tokens from `s` become nodes.
//   ingest (TrieCorpus#ingest, trie_corpus.cr:200-228): every inserted token
//     has a next token, so the path stops before the corpus' last token;
//   streaming (StreamingLeveledBuilder#build, streaming_leveled_builder.cr:
//     48-108): a cursor advances while cursor + 1 < n, so a path runs onto
//     the corpus' last token, whose node observes no next token.
enum class Paths { kIngest, kStreaming };

// Builds the nodes of the given starts in DFS preorder (children by
// ascending token) with their visits and next-token counts.
void build_nodes(Trie& t, const int32_t* tokens, int64_t n, int max_depth, std::vector<int64_t>& starts,
                 Paths mode) {
  auto len_of = [&](int64_t s) -> int64_t {
    const int64_t room = mode == Paths::kIngest ? n - 1 - s : n - s;
    return std::min<int64_t>(max_depth, room);
  };
  // Sorted by path string, every prefix first appears where a DFS preorder
  // with ascending child tokens visits it.
  std::sort(starts.begin(), starts.end(), [&](int64_t a, int64_t b) {
    const int64_t la = len_of(a), lb = len_of(b), m = std::min(la, lb);
    for (int64_t i = 0; i < m; ++i) {
      const int32_t x = tokens[a + i], y = tokens[b + i];
      if (x != y) return x < y;
    }
    if (la != lb) return la < lb;
    return a < b;
  });
  // A visit that ends at a node (depth limit) still observes the token
  // after its prefix, when there is one: (node, token) pairs.
  std::vector<int32_t> end_node, end_tok;
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
    if (len > 0 && s + len < n) {
      end_node.push_back(stack[len]);
      end_tok.push_back(tokens[s + len]);
    }
    prev = s;
  }
  // Next-token counts: the children (each child's visits observed its
  // token) merged with the ending observations, ascending by token.
  const int64_t T = static_cast<int64_t>(t.parent.size());
  std::vector<int32_t> end_first(T, -1), end_next(end_node.size(), -1);
  for (int64_t i = static_cast<int64_t>(end_node.size()) - 1; i >= 0; --i) {
    end_next[i] = end_first[end_node[i]];
    end_first[end_node[i]] = static_cast<int32_t>(i);
  }
  std::vector<int32_t> first_child(T, -1), next_sib(T, -1);
  for (int64_t i = T - 1; i >= 0; --i) {
    const int32_t p = t.parent[i];
    if (p >= 0) {
      next_sib[i] = first_child[p];
      first_child[p] = static_cast<int32_t>(i);
    }
  }
  t.coff.assign(static_cast<size_t>(T) + 1, 0);
  std::vector<std::pair<int32_t, int32_t>> hist;
  for (int64_t i = 0; i < T; ++i) {
    t.coff[i] = static_cast<int32_t>(t.ctok.size());
    hist.clear();
    for (int32_t c = first_child[i]; c >= 0; c = next_sib[c]) hist.emplace_back(t.token[c], t.visits[c]);
    for (int32_t e = end_first[i]; e >= 0; e = end_next[e]) hist.emplace_back(end_tok[e], 1);
    std::sort(hist.begin(), hist.end());
    for (size_t j = 0; j < hist.size(); ++j) {
      if (j > 0 && hist[j].first == hist[j - 1].first) {  // same token: merge into the last entry
        t.cval.back() += hist[j].second;
        continue;
      }
      t.ctok.push_back(hist[j].first);
      t.cval.push_back(hist[j].second);
    }
  }
  t.coff[T] = static_cast<int32_t>(t.ctok.size());
  t.n_corpus = n;
}

// Radix heads by the reference's rule (streaming_radix_builder.cr:155-170):
// an edge runs on through a node with exactly one next-token entry, so a
// node starts an edge when it is a root child or its parent's count list
// does not have exactly one entry.
void count_heads(Trie& t) {
  const int64_t T = static_cast<int64_t>(t.parent.size());
  t.radix_head.resize(T);
  for (int64_t i = 0; i < T; ++i) {
    const int32_t p = t.parent[i];
    t.radix_head[i] = (p < 0 || t.coff[p + 1] - t.coff[p] != 1) ? 1 : 0;
  }
}

// Drops every radix edge whose endpoint has no next-token entry (the
// end-of-corpus leaf, streaming_radix_builder.cr:177-180): the edge's rows
// form the head's whole subtree (each inner node has one child, the
// endpoint none), so removing them keeps a DFS-preorder forest. The counts
// of the remaining nodes are kept as they are (a parent still lists the
// dropped child's token, as the reference's endpoint records do).
void drop_dead_edges(Trie& t) {
  const int64_t T = static_cast<int64_t>(t.parent.size());
  std::vector<uint8_t> keep(T, 1);
  for (int64_t h = 0; h < T;) {
    int64_t e = h;  // last row of the edge that starts at h
    while (e + 1 < T && !t.radix_head[e + 1] && t.parent[e + 1] == e) ++e;
    if (t.coff[e + 1] == t.coff[e])
      for (int64_t i = h; i <= e; ++i) keep[i] = 0;
    h = e + 1;
  }
  std::vector<int32_t> nid(T, -1);
  int64_t m = 0;
  for (int64_t i = 0; i < T; ++i)
    if (keep[i]) nid[i] = static_cast<int32_t>(m++);
  if (m == T) return;
  Trie u;
  u.n_corpus = t.n_corpus;
  u.coff.push_back(0);
  for (int64_t i = 0; i < T; ++i) {
    if (!keep[i]) continue;
    const int32_t p = t.parent[i];
    u.parent.push_back(p < 0 ? -1 : nid[p]);
    u.depth.push_back(t.depth[i]);
    u.token.push_back(t.token[i]);
    u.visits.push_back(t.visits[i]);
    u.radix_head.push_back(t.radix_head[i]);
    u.ctok.insert(u.ctok.end(), t.ctok.begin() + t.coff[i], t.ctok.begin() + t.coff[i + 1]);
    u.cval.insert(u.cval.end(), t.cval.begin() + t.coff[i], t.cval.begin() + t.coff[i + 1]);
    u.coff.push_back(static_cast<int32_t>(u.ctok.size()));
  }
  t = std::move(u);
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

namespace {

std::vector<int64_t> starts_of(int64_t n, int64_t max_starts) {
  const int64_t total_starts = n - 1;  // trie_corpus.cr:203, streaming_leveled_builder.cr:43
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
  return starts;
}

}  // namespace

extern "C" int agpt_trie_build(const int32_t* tokens, int64_t n, int max_depth,
                               int64_t max_starts, agpt_trie_handle* out) {
  if (!out || (!tokens && n > 0) || max_depth < 1) return 1;
  *out = nullptr;
  auto* h = new agpt_trie_s();
  Trie& t = h->t;
  std::vector<int64_t> starts = starts_of(n, max_starts);
  build_nodes(t, tokens, n, max_depth, starts, Paths::kIngest);
  count_heads(t);
  finish(&t, true);
  *out = h;
  return 0;
}

extern "C" int agpt_trie_build_radix(const int32_t* tokens, int64_t n, int max_depth,
                                     agpt_trie_handle* out) {
  if (!out || (!tokens && n > 0) || max_depth < 1) return 1;
  *out = nullptr;
  auto* h = new agpt_trie_s();
  Trie& t = h->t;
  std::vector<int64_t> starts = starts_of(n, 0);
  build_nodes(t, tokens, n, max_depth, starts, Paths::kStreaming);
  count_heads(t);
  drop_dead_edges(t);
  finish(&t, true);
  *out = h;
  return 0;
}

extern "C" int agpt_trie_build_radix_part(const int32_t* tokens, int64_t n, int max_depth,
                                          int32_t first_token, agpt_trie_handle* out) {
  if (!out || (!tokens && n > 0) || max_depth < 1) return 1;
  *out = nullptr;
  auto* h = new agpt_trie_s();
  Trie& t = h->t;
  std::vector<int64_t> starts;
  for (const int64_t s : starts_of(n, 0))
    if (tokens[s] == first_token) starts.push_back(s);
  build_nodes(t, tokens, n, max_depth, starts, Paths::kStreaming);
  count_heads(t);
  drop_dead_edges(t);
  finish(&t, true);
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
  finish(&t, false);
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
  if (offsets) std::memcpy(offsets, t.coff.data(), (n + 1) * sizeof(int32_t));
  if (tok && !t.ctok.empty()) std::memcpy(tok, t.ctok.data(), t.ctok.size() * sizeof(int32_t));
  if (val && !t.cval.empty()) std::memcpy(val, t.cval.data(), t.cval.size() * sizeof(int32_t));
  *n_entries = static_cast<int64_t>(t.ctok.size());
  return 0;
}

// ---- radix subtree files (streaming_radix_builder.cr:27-32, 100-330, 388-470;
// read side agpt_train.cu:495-669) ---------------------------------------------

namespace {

constexpr uint32_t kRadixMagic = 0x52445841u;  // 'RDXA'
constexpr int32_t kRadixVersion = 2;

void put_i32(std::vector<uint8_t>& b, int32_t v) {
  const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
  b.insert(b.end(), p, p + 4);
}
void put_i64(std::vector<uint8_t>& b, int64_t v) {
  const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
  b.insert(b.end(), p, p + 8);
}
bool write_file(const std::string& path, const std::vector<uint8_t>& b) {
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) return false;
  const bool ok = std::fwrite(b.data(), 1, b.size(), f) == b.size();
  return std::fclose(f) == 0 && ok;
}

}  // namespace

struct agpt_radix_s {
  int32_t root_child_id = 0, max_endpoint_depth = 0;
  // radix nodes in DFS preorder (children by ascending first token)
  std::vector<int32_t> radix_id, parent, first_char_depth, edge_len, edge_mass, edge_off;
  std::vector<int32_t> tokens;  // edge tokens, DFS order
  std::vector<int32_t> coff, ctok, cval;
};

extern "C" int agpt_radix_write_subtrees(agpt_trie_handle h, const char* out_dir, int32_t vocab_size) {
  if (!h || !out_dir) return 1;
  const Trie& t = h->t;
  const int64_t n = static_cast<int64_t>(t.parent.size());
  if (t.visits.size() != static_cast<size_t>(n)) return 2;  // no corpus counts
  const std::vector<int32_t>& off = t.coff;
  const std::vector<int32_t>& tok = t.ctok;
  const std::vector<int32_t>& val = t.cval;
  std::vector<int32_t> first_child(n, -1), next_sib(n, -1), roots;
  for (int64_t i = n - 1; i >= 0; --i) {
    const int32_t p = t.parent[i];
    if (p >= 0) {
      next_sib[i] = first_child[p];
      first_child[p] = static_cast<int32_t>(i);
    }
  }
  for (int64_t i = 0; i < n; ++i)
    if (t.parent[i] < 0) roots.push_back(static_cast<int32_t>(i));
  struct Start {
    int32_t parent_radix, node, depth;  // node = leveled parent (-1: root)
  };
  std::vector<Start> frontier{{0, -1, 1}};
  std::map<int32_t, std::vector<uint8_t>> files;  // subtree key -> body
  std::map<int32_t, std::array<int64_t, 3>> stats;  // key -> records, chars, max endpoint depth
  std::vector<int32_t> subtree_of{0};
  int32_t next_id = 1;
  int64_t total_chars = 0;
  int32_t max_ep = 0;
  for (size_t fi = 0; fi < frontier.size(); ++fi) {  // FIFO: breadth first
    const Start st = frontier[fi];
    std::vector<int32_t> kids;
    if (st.node < 0) kids = roots;
    else
      for (int32_t c = first_child[st.node]; c >= 0; c = next_sib[c]) kids.push_back(c);
    for (int32_t c : kids) {
      std::vector<int32_t> edge{t.token[c]};
      int32_t cur = c;
      // extend while the node has one next-token entry and its child
      // exists (the child then continues the edge: it is no radix head)
      while (first_child[cur] >= 0 && !t.radix_head[first_child[cur]]) {
        cur = first_child[cur];
        edge.push_back(t.token[cur]);
      }
      const int32_t rid = next_id++;
      const int32_t key = st.parent_radix == 0 ? rid : subtree_of[st.parent_radix];
      subtree_of.push_back(key);
      const int32_t ep = t.depth[cur];
      std::vector<uint8_t>& b = files[key];
      put_i32(b, rid);
      put_i32(b, st.parent_radix);
      put_i32(b, st.depth);
      put_i32(b, static_cast<int32_t>(edge.size()));
      for (int32_t x : edge) put_i32(b, x);
      int32_t mass = 0;  // v2 edge mass: the sum of the head's counts
      for (int32_t e = off[c]; e < off[c + 1]; ++e) mass += val[e];
      put_i32(b, mass);
      put_i32(b, off[cur + 1] - off[cur]);
      for (int32_t e = off[cur]; e < off[cur + 1]; ++e) {
        put_i32(b, tok[e]);
        put_i32(b, val[e]);
      }
      auto& sv = stats[key];
      sv[0] += 1;
      sv[1] += static_cast<int64_t>(edge.size());
      sv[2] = std::max<int64_t>(sv[2], ep);
      total_chars += static_cast<int64_t>(edge.size());
      max_ep = std::max(max_ep, ep);
      if (off[cur + 1] - off[cur] >= 2) frontier.push_back({rid, cur, ep + 1});
    }
  }
  const std::string dir(out_dir);
  std::vector<uint8_t> manifest;
  put_i32(manifest, static_cast<int32_t>(kRadixMagic));
  put_i32(manifest, kRadixVersion);
  put_i32(manifest, static_cast<int32_t>(files.size()));
  for (const auto& kv : files) {  // std::map: ascending root-child id
    const auto& sv = stats[kv.first];
    std::vector<uint8_t> b;
    put_i32(b, static_cast<int32_t>(kRadixMagic));
    put_i32(b, kRadixVersion);
    put_i32(b, kv.first);
    put_i32(b, static_cast<int32_t>(sv[0]));
    put_i64(b, sv[1]);
    put_i32(b, static_cast<int32_t>(sv[2]));
    b.insert(b.end(), kv.second.begin(), kv.second.end());
    char name[64];
    std::snprintf(name, sizeof(name), "/subtrees/radix_subtree_%06d.bin", kv.first);
    if (!write_file(dir + name, b)) return 4;
    put_i32(manifest, kv.first);
    put_i32(manifest, static_cast<int32_t>(sv[0]));
    put_i64(manifest, sv[1]);
    put_i32(manifest, static_cast<int32_t>(sv[2]));
  }
  if (!write_file(dir + "/manifest.bin", manifest)) return 4;
  std::vector<uint8_t> meta;
  put_i32(meta, static_cast<int32_t>(kRadixMagic));
  put_i32(meta, kRadixVersion);
  put_i32(meta, next_id);  // radix nodes + the virtual root
  put_i32(meta, max_ep + 1);
  put_i64(meta, total_chars);
  put_i32(meta, static_cast<int32_t>(t.n_corpus));
  put_i32(meta, vocab_size);
  put_i64(meta, 0);  // corpus hash
  put_i32(meta, 4);
  for (char ch : std::string("char")) meta.push_back(static_cast<uint8_t>(ch));
  if (!write_file(dir + "/meta.bin", meta)) return 4;
  return 0;
}

extern "C" int agpt_radix_read_subtree(const char* path, agpt_radix_handle* out) {
  if (!path || !out) return 1;
  *out = nullptr;
  FILE* f = std::fopen(path, "rb");
  if (!f) return 2;
  std::vector<uint8_t> b;
  uint8_t buf[1 << 16];
  size_t got;
  while ((got = std::fread(buf, 1, sizeof(buf), f)) > 0) b.insert(b.end(), buf, buf + got);
  std::fclose(f);
  size_t pos = 0;
  bool ok = true;
  auto i32 = [&]() -> int32_t {
    if (pos + 4 > b.size()) { ok = false; return 0; }
    int32_t v;
    std::memcpy(&v, b.data() + pos, 4);
    pos += 4;
    return v;
  };
  auto i64 = [&]() -> int64_t {
    if (pos + 8 > b.size()) { ok = false; return 0; }
    int64_t v;
    std::memcpy(&v, b.data() + pos, 8);
    pos += 8;
    return v;
  };
  if (static_cast<uint32_t>(i32()) != kRadixMagic || !ok) return 3;
  if (i32() != kRadixVersion || !ok) return 4;
  auto* r = new agpt_radix_s();
  r->root_child_id = i32();
  const int32_t count = i32();
  const int64_t chars = i64();
  r->max_endpoint_depth = i32();
  if (!ok || count < 0 || chars < 0) { delete r; return 5; }
  // records in file order (breadth first)
  std::vector<int32_t> rid(count), gpar(count), fcd(count), elen(count), mass(count), eoff(count), cstart(count),
      ccount(count);
  std::vector<int32_t> toks, ct, cv;
  for (int32_t i = 0; i < count && ok; ++i) {
    rid[i] = i32();
    gpar[i] = i32();
    fcd[i] = i32();
    elen[i] = i32();
    if (elen[i] < 1 || pos + 4 * static_cast<size_t>(elen[i]) > b.size()) { ok = false; break; }
    eoff[i] = static_cast<int32_t>(toks.size());
    for (int32_t e = 0; e < elen[i]; ++e) toks.push_back(i32());
    mass[i] = i32();
    ccount[i] = i32();
    if (ccount[i] < 0 || pos + 8 * static_cast<size_t>(ccount[i]) > b.size()) { ok = false; break; }
    cstart[i] = static_cast<int32_t>(ct.size());
    for (int32_t e = 0; e < ccount[i]; ++e) {
      ct.push_back(i32());
      cv.push_back(i32());
    }
  }
  if (!ok || pos != b.size() || static_cast<int64_t>(toks.size()) != chars) { delete r; return 5; }
  // global -> local ids; the subtree's root child has global parent 0
  std::unordered_map<int32_t, int32_t> local;
  local.reserve(static_cast<size_t>(count) * 2);
  for (int32_t i = 0; i < count; ++i) local[rid[i]] = i;
  std::vector<int32_t> lpar(count, -1);
  std::vector<std::vector<int32_t>> kids(count);
  std::vector<int32_t> tops;
  for (int32_t i = 0; i < count; ++i) {
    const auto it = gpar[i] == 0 ? local.end() : local.find(gpar[i]);
    if (it == local.end()) tops.push_back(i);
    else {
      lpar[i] = it->second;
      kids[it->second].push_back(i);
    }
  }
  auto by_tok = [&](int32_t a, int32_t c) { return toks[eoff[a]] < toks[eoff[c]] || (toks[eoff[a]] == toks[eoff[c]] && a < c); };
  std::sort(tops.begin(), tops.end(), by_tok);
  for (auto& k : kids) std::sort(k.begin(), k.end(), by_tok);
  // DFS preorder
  std::vector<int32_t> order, newid(count, -1), stack(tops.rbegin(), tops.rend());
  while (!stack.empty()) {
    const int32_t i = stack.back();
    stack.pop_back();
    newid[i] = static_cast<int32_t>(order.size());
    order.push_back(i);
    for (auto it = kids[i].rbegin(); it != kids[i].rend(); ++it) stack.push_back(*it);
  }
  r->coff.push_back(0);
  for (int32_t i : order) {
    r->radix_id.push_back(rid[i]);
    r->parent.push_back(lpar[i] < 0 ? -1 : newid[lpar[i]]);
    r->first_char_depth.push_back(fcd[i]);
    r->edge_len.push_back(elen[i]);
    r->edge_mass.push_back(mass[i]);
    r->edge_off.push_back(static_cast<int32_t>(r->tokens.size()));
    r->tokens.insert(r->tokens.end(), toks.begin() + eoff[i], toks.begin() + eoff[i] + elen[i]);
    r->ctok.insert(r->ctok.end(), ct.begin() + cstart[i], ct.begin() + cstart[i] + ccount[i]);
    r->cval.insert(r->cval.end(), cv.begin() + cstart[i], cv.begin() + cstart[i] + ccount[i]);
    r->coff.push_back(static_cast<int32_t>(r->ctok.size()));
  }
  *out = r;
  return 0;
}

extern "C" int agpt_radix_info(agpt_radix_handle r, int64_t* n_radix, int64_t* n_chars, int64_t* n_entries,
                               int32_t* root_child_id, int32_t* max_endpoint_depth) {
  if (!r) return 1;
  if (n_radix) *n_radix = static_cast<int64_t>(r->radix_id.size());
  if (n_chars) *n_chars = static_cast<int64_t>(r->tokens.size());
  if (n_entries) *n_entries = static_cast<int64_t>(r->ctok.size());
  if (root_child_id) *root_child_id = r->root_child_id;
  if (max_endpoint_depth) *max_endpoint_depth = r->max_endpoint_depth;
  return 0;
}

extern "C" int agpt_radix_export(agpt_radix_handle r, int32_t* radix_id, int32_t* radix_parent,
                                 int32_t* first_char_depth, int32_t* edge_len, int32_t* edge_mass,
                                 int32_t* edge_tokens, int32_t* counts_offset, int32_t* counts_tok,
                                 int32_t* counts_val) {
  if (!r) return 1;
  auto cp = [](int32_t* dst, const std::vector<int32_t>& src) {
    if (dst && !src.empty()) std::memcpy(dst, src.data(), src.size() * sizeof(int32_t));
  };
  cp(radix_id, r->radix_id);
  cp(radix_parent, r->parent);
  cp(first_char_depth, r->first_char_depth);
  cp(edge_len, r->edge_len);
  cp(edge_mass, r->edge_mass);
  cp(edge_tokens, r->tokens);
  cp(counts_offset, r->coff);
  cp(counts_tok, r->ctok);
  cp(counts_val, r->cval);
  return 0;
}

extern "C" void agpt_radix_free(agpt_radix_handle r) { delete r; }

extern "C" void agpt_trie_free(agpt_trie_handle h) { delete h; }
