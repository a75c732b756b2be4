// trie_fast.h — the fast trie-attention kernels (included by trie_attn.hip).
//
// Persistent streaming workgroups. The tiles are kTile consecutive DFS rows;
// a unit of work is (tile, head group of HG heads). Each workgroup (256
// threads, 4 waves) owns one head group and a contiguous range of tiles and
// walks it in order, keeping the tile context in LDS:
//   key set   K, V [P + kTile][WS]: slots 0..P-1 hold the prefix rows (the
//             ancestors of the tile's first row s, slot d = depth d+1),
//             slots P.. the tile rows (P = max_depth - 1);
//   tile rows Q (and dO for the backward) [kTile][WS];
//   anc       [kTile][ldd] int16: key-set slot of each row's ancestor at
//             every depth;
//   tables    depths, subtree ends, work items, lse and δ of the tile rows.
// While a tile computes, the next tile's rows and tables are already in
// flight into registers; the switch then costs two barriers. The next
// tile's prefix never needs HBM: every ancestor of its first row is either
// an ancestor of the current first row (the same slot, left in place) or a
// row of the current tile (copied LDS to LDS). Only the first tile of a
// range loads its prefix rows from memory.
//
// Work items are chain groups built by the plan: up to four consecutive rows
// (queries) or key-set entries (keys) where each is the previous one's child
// — the interior of a radix edge. One item-head pair runs on a quad of
// adjacent lanes, one block of the fp32 matrix instruction
// v_mfma_f32_4x4x1_16b (16 independent 4x4 blocks per wave: D[i][j] +=
// A[lane 4b+i] * B[lane 4b+j], row i in register i, column j in lane j of
// the block). Lane x owns member x of the group: its head vector and its
// softmax state.
//
//  query side (forward; dQ): item = query chain group r0..r0+n-1. Member x
//    sees the keys at depth <= depth(r0+x), all on the last member's path,
//    so one walk over that path serves the group, four keys per step. Lane
//    j brings key j's row as the A operand and lane x its query as B, so the
//    score block S^T[key][member] lands with member x's four scores in lane x
//    (softmax needs no lane exchange); P then is the A operand of P·V, whose
//    B operand in lane j' is dims [j'*HD/4, (j'+1)*HD/4) of each key's V row;
//    the output block holds member i's dims of lane j' in register i.
//  key side (dK/dV): item = key chain group; the subtrees are nested, so one
//    pass over the first member's query range serves the group, four queries
//    per step (member x takes query j iff a_x <= j < end(a_x)).
//
// Rounds: the plan sorts each tile's items by cost (walk length, resp.
// query-range length), longest first; a round is 16/HG consecutive items,
// one per quad, and runs as many steps as its first item needs (a uniform
// trip count: the matrix instructions never see a partial execution mask;
// steps past an item's end are masked). Wave w takes rounds w, w+4, ...
//
// The running softmax max starts at the member's self score and moves only
// when a score exceeds it by more than 2^8 (then the sums are rescaled).
//
// Workgroups are dealt to the 8 XCDs round-robin; workgroup b takes slot
// (b % 8) * (G / 8) + b / 8, so the workgroups of one XCD hold neighbouring
// tile ranges.
#pragma once

namespace agpt_fast {

using namespace agpt;

constexpr int kXcds = 8;
constexpr int kTile = 64;             // rows per tile
constexpr int kThreads = 256;         // 4 waves per workgroup
constexpr int kWaves = kThreads / 64;
constexpr int kGroup = 4;             // chain-group members = lanes per block
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)
constexpr int kCopyPer = 2;           // prefix-copy jobs per thread (else reload)

// A work item (int32) packs: first entry (bits 0-8), member count (9-11),
// first step b0 (12-17), last step b1 - 1 (18-23), scratch slot (24-26),
// part (27-28), part count - 1 (29-30). An item walks 4-row steps [b0, b1)
// of its group's walk (the path of a query group, the query range of a key
// group). A long walk is cut into parts of whole steps: part k of n covers
// steps [k*nb/n, (k+1)*nb/n) of its nb steps; the parts of one group write
// partial results to scratch slot `slot`, merged in fixed part order after
// the rounds. n = 1 is a group that is not cut.
__host__ __device__ constexpr int item_first(int v) { return v & 511; }
__host__ __device__ constexpr int item_count(int v) { return (v >> 9) & 7; }
__host__ __device__ constexpr int item_b0(int v) { return (v >> 12) & 63; }
__host__ __device__ constexpr int item_b1(int v) { return ((v >> 18) & 63) + 1; }
__host__ __device__ constexpr int item_slot(int v) { return (v >> 24) & 7; }
__host__ __device__ constexpr int item_part(int v) { return (v >> 27) & 3; }
__host__ __device__ constexpr int item_nparts(int v) { return ((v >> 29) & 3) + 1; }
__host__ __device__ constexpr int make_item(int first, int count, int b0, int b1, int part = 0, int nparts = 1,
                                            int slot = 0) {
  return first | (count << 9) | (b0 << 12) | ((b1 - 1) << 18) | (slot << 24) | (part << 27) |
         ((nparts - 1) << 29);
}
// First step of part `part` of `nparts` over nb steps.
__host__ __device__ constexpr int part_begin(int nb, int part, int nparts) { return part * nb / nparts; }

// Cutting: items longer than kCutSteps steps are cut into ceil(nb /
// kCutSteps) parts, longest items first, while scratch slots last: the
// query side has kQSlots slots of up to 2 parts, the key side kKSlots slots
// of up to 4 parts.
constexpr int kCutSteps = 4;
constexpr int kQSlots = 8, kQParts = 2;
constexpr int kKSlots = 8, kKParts = 4;
// Scratch floats per (slot, part, head, member): the forward keeps the P·V
// partial (HD), the running max and sum (padded to 16 B); dQ keeps HD;
// dK|dV keep 2*HD.
__host__ __device__ constexpr int fwd_part_floats(int HD) { return HD + 4; }
inline size_t q_scratch_bytes(int HG, int HD, bool fwd) {
  return static_cast<size_t>(kQSlots) * kQParts * HG * 4 * (fwd ? fwd_part_floats(HD) : HD) * sizeof(float);
}
inline size_t k_scratch_bytes(int HG, int HD) {
  return static_cast<size_t>(kKSlots) * kKParts * HG * 4 * 2 * HD * sizeof(float);
}

// anc row length: max depth rounded up to whole 4-key steps, plus 4 so that
// rows written by consecutive lanes spread over the banks.
__host__ __device__ constexpr int anc_stride(int max_depth) { return ((max_depth + 3) & ~3) + 4; }

// Row stride (elements) of a staged slice: one extra 16-byte chunk, so four
// consecutive rows read at one column fall on distinct banks.
template <typename Tin>
__host__ __device__ constexpr int lds_stride(int width) {
  return width + static_cast<int>(16 / sizeof(Tin));
}

// Stream modes (bit flags): the query side walks paths (anc table, query
// items); the key side walks query ranges (subtree ends, key items); lse and
// δ of the tile rows go to LDS tables when the backward needs them.
constexpr int kQSide = 1, kKSide = 2, kLse = 4, kDl = 8;

// Dynamic LDS of a stream (see Stream): key set K, V [P + kTile][WS], ns
// staged tile tensors [kTile][WS], anc [kTile][ldd] int16 (query side), and
// with pdl the δ partials [kTile][HG][HD/EPC] fp32.
__host__ __device__ inline size_t stream_lds_bytes(int max_depth, int HG, int HD, int elem, int ns, bool pdl, bool anc) {
  const int ws = HG * HD + 16 / elem;
  size_t b = static_cast<size_t>(2 * (max_depth - 1 + kTile) + ns * kTile) * ws * elem;
  if (anc) b += static_cast<size_t>(kTile) * anc_stride(max_depth) * sizeof(int16_t);
  b = (b + 15) & ~static_cast<size_t>(15);
  if (pdl) b += static_cast<size_t>(kTile) * HG * (HD / (16 / elem)) * sizeof(float);
  return b;
}

typedef float f4 __attribute__((ext_vector_type(4)));
// 16-byte chunk as a native vector (the HIP uint4 struct blocks register
// promotion of arrays of chunks).
typedef unsigned u4 __attribute__((ext_vector_type(4)));

// One 4x4x1 fp32 matrix step on every quad of the wave (see the header).
__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

// S[r] (register r, lane x of a quad) = Σ_i A_r[i] * B_x[i] over HD dims,
// with lane j supplying row a = A_j and lane x column b = B_x. Two
// accumulator chains keep the dependent matrix steps apart.
template <int HD>
__device__ __forceinline__ f4 mfma_dot(const float (&a)[HD], const float (&b)[HD]) {
  f4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
#pragma unroll
  for (int i = 0; i < HD; i += 2) {
    s0 = mfma4(a[i], b[i], s0);
    s1 = mfma4(a[i + 1], b[i + 1], s1);
  }
  return s0 + s1;
}

// acc[t] (register i, lane j') += Σ_k P_i[k] * C_{j'}[k][t]: lane i supplies
// p[k] (row i of the A operand at step k), lane j' the DPL-slice of row k.
template <int DPL>
__device__ __forceinline__ void mfma_accum(f4 (&acc)[DPL], const float (&p)[kGroup],
                                           const float (&c)[kGroup][DPL]) {
#pragma unroll
  for (int k = 0; k < kGroup; ++k)
#pragma unroll
    for (int t = 0; t < DPL; ++t) acc[t] = mfma4(p[k], c[k][t], acc[t]);
}

// Broadcast of lane i's value to its whole quad (quad_perm [i,i,i,i]).
template <int I>
__device__ __forceinline__ float qbcast(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), I * 0x55, 0xF, 0xF, true));
}
__device__ __forceinline__ void quad_bcast_all(float x, float (&out)[kGroup]) {
  out[0] = qbcast<0>(x);
  out[1] = qbcast<1>(x);
  out[2] = qbcast<2>(x);
  out[3] = qbcast<3>(x);
}

template <int N>
__device__ __forceinline__ float dot(const float (&a)[N], const float (&b)[N]) {
  float r = a[0] * b[0];
#pragma unroll
  for (int i = 1; i < N; ++i) r += a[i] * b[i];
  return r;
}

// Inverse RoPE on dims [d0, d0 + N) of a head (N even, d0 even); the tables
// are [seq, HD] with entry [pos, 2i] used for the pair (2i, 2i+1).
template <int N, int HD>
__device__ __forceinline__ void rope_inverse_part(float (&x)[N], const float* __restrict__ cos_t,
                                                  const float* __restrict__ sin_t, int pos, int d0) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float c = cos_t[pos * HD + d0 + 2 * i];
    const float s = sin_t[pos * HD + d0 + 2 * i];
    const float x0 = x[2 * i], x1 = x[2 * i + 1];
    x[2 * i] = x0 * c + x1 * s;
    x[2 * i + 1] = -x0 * s + x1 * c;
  }
}

// Makes a value wave-uniform (it already is by construction; this lets the
// compiler keep loop counts in scalar registers).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Lane coordinates: quad q = lane / 4 holds item slot q / HG, head q % HG;
// x = lane % 4 is the member (and the row of the matrix block) it owns.
template <int HG>
struct Lane {
  int wave, lane, x, slot, hl;
  __device__ __forceinline__ Lane() {
    wave = threadIdx.x >> 6;
    lane = threadIdx.x & 63;
    x = lane & 3;
    const int quad = lane >> 2;
    slot = quad / HG;
    hl = quad - slot * HG;
  }
};

// Tile tables in LDS.
template <int HG>
struct StreamTables {
  int32_t depth[kTile];
  int32_t tend[kTile];        // absolute subtree end of the tile rows
  int32_t pend[kMaxDepth];    // absolute subtree end of the prefix slots
  int32_t qitem[kTile + kQSlots * (kQParts - 1)];
  int32_t kitem[kTile + kMaxDepth + kKSlots * kKParts];
  float l2[HG][kTile];        // lse * log2(e) of the tile rows (backward)
  float dl[HG][kTile];        // δ of the tile rows (backward)
  int32_t cut[kWaves];        // per wave: some item it loaded is cut
};

// Item counts per tile: one query item per row at most, one key item per
// key-set entry (prefix + rows), plus the extra parts of cut items; the item
// fields hold the slot and part numbers.
static_assert(kQSlots <= 8 && kKSlots <= 8 && kQParts <= 4 && kKParts <= 4, "item fields");
static_assert(kMaxDepth <= 4 * 64 && kTile <= 4 * 64 && kMaxDepth + kTile <= 512, "item fields");

// The workgroup's head group and tile range [t0, t1).
__device__ __forceinline__ void assign_range(int n_tiles, int n_hg, int& hg, int& t0, int& t1) {
  const int G = gridDim.x;  // a multiple of 8 and of n_hg
  const int b = blockIdx.x;
  const int L = (b % kXcds) * (G / kXcds) + b / kXcds;
  hg = L % n_hg;
  const int r = L / n_hg;
  const int R = G / n_hg;
  t0 = static_cast<int>(static_cast<int64_t>(r) * n_tiles / R);
  t1 = static_cast<int>(static_cast<int64_t>(r + 1) * n_tiles / R);
}

// ---------------------------------------------------------------------------
// Tile context stream. NT = tile-row tensors fetched: 1 = Q (forward);
// 2 = Q, dO; 3 = Q, dO, O (O is reduced to δ partials, not staged).
// kMode: the kQSide / kKSide / kLse / kDl flags above.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, int NT, int kMode, typename PlanT>
struct Stream {
  static constexpr bool kQ = kMode & kQSide;
  static constexpr bool kK = kMode & kKSide;
  static constexpr int W = HG * HD;
  static constexpr int WS = lds_stride<Tin>(W);
  static constexpr int EPC = 16 / static_cast<int>(sizeof(Tin));  // elements per 16-B chunk
  static constexpr int CPR = W / EPC;                              // chunks per row slice
  static constexpr int CPH = HD / EPC;                             // chunks per head
  static constexpr int ROWJ = kTile * CPR;                         // chunk jobs per row tensor
  static constexpr int KV_PER = (2 * ROWJ + kThreads - 1) / kThreads;
  static constexpr int T_PER = (ROWJ + kThreads - 1) / kThreads;
  static constexpr int NS = NT < 2 ? NT : 2;  // staged tile tensors
  static constexpr int PJ = 2 * CPR;          // copy jobs per prefix slot (K and V)

  const PlanT pl;
  const Tin* K;
  const Tin* V;
  const Tin* TT[NT];
  const float* lse;
  const float* Dl;
  int D, H, hg, P, ldd;
  // LDS
  Tin* Ks;
  Tin* Vs;
  Tin* Ts;       // [NS][kTile][WS]
  int16_t* anc;  // [kTile][ldd]
  float* pdl;    // [kTile][HG][CPH] δ partials (NT == 3)
  StreamTables<HG>& tb;
  // current tile
  int t, s, ntile, A, poff, nq, nk;
  bool cut;  // the tile has cut items (a merge pass follows its rounds)
  // next tile (prefetched)
  int n_t, n_s, n_ntile, n_A, n_poff, n_qoff, n_nq, n_koff, n_nk;
  u4 kv[KV_PER];
  u4 tt[NT][T_PER];
  int dep, tend_r, qit, kit0, kit1;
  float lse_r, dl_r;
  int cp_id[kCopyPer];

  __device__ __forceinline__ Stream(const PlanT& pl_, const Tin* K_, const Tin* V_, const Tin* T0,
                                    const Tin* T1, const Tin* T2, const float* lse_, const float* Dl_,
                                    int H_, int hg_, unsigned char* dyn, StreamTables<HG>& tb_)
      : pl(pl_), K(K_), V(V_), lse(lse_), Dl(Dl_), H(H_), hg(hg_), tb(tb_) {
    TT[0] = T0;
    if constexpr (NT > 1) TT[1] = T1;
    if constexpr (NT > 2) TT[2] = T2;
    D = H * HD;
    P = pl.max_depth - 1;
    ldd = anc_stride(pl.max_depth);
    Ks = reinterpret_cast<Tin*>(dyn);
    Vs = Ks + (P + kTile) * WS;
    Ts = Vs + (P + kTile) * WS;
    anc = reinterpret_cast<int16_t*>(Ts + NS * kTile * WS);
    // Offsets from the LDS base (integer casts of the pointer would lose its
    // address space and turn the accesses into flat ones).
    const int abytes = (2 * (P + kTile) + NS * kTile) * WS * static_cast<int>(sizeof(Tin)) +
                       (kQ ? kTile * ldd * static_cast<int>(sizeof(int16_t)) : 0);
    pdl = reinterpret_cast<float*>(dyn + ((abytes + 15) & ~15));
  }

  __host__ __device__ static size_t lds_bytes(int max_depth) {
    return stream_lds_bytes(max_depth, HG, HD, sizeof(Tin), NS, NT == 3, kQ);
  }

  __device__ __forceinline__ const Tin* gsrc(const Tin* base, int64_t row, int c) const {
    return base + row * D + hg * W + c * EPC;
  }

  // Issues the loads of tile nt into registers (consumed by commit()).
  __device__ __forceinline__ void prefetch(int nt) {
    const int tid = threadIdx.x;
    n_t = nt;
    n_s = nt * kTile;
    n_ntile = min(kTile, static_cast<int>(pl.T - n_s));
    n_poff = pl.pref_off[nt];
    n_A = pl.pref_off[nt + 1] - n_poff;
    if constexpr (kQ) {
      n_qoff = pl.q_item_off[nt];
      n_nq = pl.q_item_off[nt + 1] - n_qoff;
    }
    if constexpr (kK) {
      n_koff = pl.k_item_off[nt];
      n_nk = pl.k_item_off[nt + 1] - n_koff;
    }
    // Every load is unconditional, from an in-range address (indices past
    // the tile are clamped; commit() ignores those values), so the values
    // stay in registers and the loads stay in flight until commit().
    const int last = n_ntile - 1;
#pragma unroll
    for (int k = 0; k < KV_PER; ++k) {
      const int j = min(tid + k * kThreads, 2 * ROWJ - 1);
      const int ten = j / ROWJ;
      const int r = min((j - ten * ROWJ) / CPR, last);
      kv[k] = *reinterpret_cast<const u4*>(gsrc(ten ? V : K, n_s + r, j % CPR));
    }
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int k = 0; k < T_PER; ++k) {
        const int j = min(tid + k * kThreads, ROWJ - 1);
        const int r = min(j / CPR, last);
        tt[i][k] = *reinterpret_cast<const u4*>(gsrc(TT[i], n_s + r, j % CPR));
      }
    const int lane = tid & 63;
    dep = pl.depth[n_s + min(lane, last)];
    if constexpr (kQ) qit = pl.q_items[n_qoff + min(tid, max(n_nq - 1, 0))];
    if constexpr (kK) {
      tend_r = pl.end[n_s + min(tid, last)];
      kit0 = pl.k_items[n_koff + min(tid, max(n_nk - 1, 0))];
      kit1 = pl.k_items[n_koff + min(tid + kThreads, max(n_nk - 1, 0))];
    }
    if constexpr ((kMode & (kLse | kDl)) != 0) {
      const int i = min(tid, n_ntile * HG - 1);
      const int r = i / HG;
      const int64_t o = (static_cast<int64_t>(n_s) + r) * H + hg * HG + (i - r * HG);
      if constexpr ((kMode & kLse) != 0) lse_r = lse[o];
      if constexpr ((kMode & kDl) != 0) dl_r = Dl[o];
    }
#pragma unroll
    for (int k = 0; k < kCopyPer; ++k) {
      const int d = (tid + k * kThreads) / PJ;
      // Entries past the prefix load a valid one; commit() ignores them (no
      // value is used here, so the loads stay in flight until commit()).
      cp_id[k] = pl.prefix[n_A > 0 ? n_poff + min(d, n_A - 1) : max(n_poff - 1, 0)];
    }
  }

  // Installs the prefetched tile in LDS. cold: the prefix rows are loaded
  // from memory (first tile of a range, or a prefix too long to copy).
  __device__ __forceinline__ void commit(bool cold) {
    const int tid = threadIdx.x;
    cold = cold || n_A * PJ > kCopyPer * kThreads;
    u4 cpv[kCopyPer];
    int cpe[kCopyPer];
#pragma unroll
    for (int k = 0; k < kCopyPer; ++k) {
      // A row of the current tile that moves into the prefix (id >= s);
      // other jobs read row 0 and discard it.
      const int j = tid + k * kThreads;
      const int rem = j % PJ;
      const int row = (!cold && cp_id[k] >= s) ? cp_id[k] - s : 0;
      cpv[k] = *reinterpret_cast<const u4*>((rem < CPR ? Ks : Vs) + (P + row) * WS + (rem % CPR) * EPC);
      cpe[k] = tb.tend[row];
    }
    __syncthreads();  // the current tile's context is no longer read
#pragma unroll
    for (int k = 0; k < KV_PER; ++k) {
      const int j = tid + k * kThreads;
      const int ten = j / ROWJ;
      const int r = (j - ten * ROWJ) / CPR;
      const int c = j % CPR;
      if (j < 2 * ROWJ && r < n_ntile)
        *reinterpret_cast<u4*>((ten ? Vs : Ks) + (P + r) * WS + c * EPC) = kv[k];
    }
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int k = 0; k < T_PER; ++k) {
        const int j = tid + k * kThreads;
        const int r = j / CPR;
        if (j < ROWJ && r < n_ntile)
          *reinterpret_cast<u4*>(Ts + (i * kTile + r) * WS + (j % CPR) * EPC) = tt[i][k];
      }
    if constexpr (NT == 3) {  // δ partials: dO·O over each 16-byte chunk
#pragma unroll
      for (int k = 0; k < T_PER; ++k) {
        const int j = tid + k * kThreads;
        const int r = j / CPR;
        if (j < ROWJ && r < n_ntile) {
          const float* g = reinterpret_cast<const float*>(&tt[1][k]);
          const float* o = reinterpret_cast<const float*>(&tt[2][k]);
          pdl[r * (HG * CPH) + j % CPR] = (g[0] * o[0] + g[1] * o[1]) + (g[2] * o[2] + g[3] * o[3]);
        }
      }
    }
    if (!cold) {
#pragma unroll
      for (int k = 0; k < kCopyPer; ++k) {
        const int j = tid + k * kThreads;
        const int d = j / PJ;
        const int rem = j % PJ;
        if (cp_id[k] >= s && d < n_A) {
          *reinterpret_cast<u4*>((rem < CPR ? Ks : Vs) + d * WS + (rem % CPR) * EPC) = cpv[k];
          if (kK && rem == 0) tb.pend[d] = cpe[k];
        }
      }
    } else {
      for (int j = tid; j < n_A * PJ; j += kThreads) {
        const int d = j / PJ;
        const int rem = j % PJ;
        const int id = pl.prefix[n_poff + d];
        *reinterpret_cast<u4*>((rem < CPR ? Ks : Vs) + d * WS + (rem % CPR) * EPC) =
            *reinterpret_cast<const u4*>(gsrc(rem < CPR ? K : V, id, rem % CPR));
        if (kK && rem == 0) tb.pend[d] = pl.pref_end[n_poff + d];
      }
    }
    const int lane = tid & 63;
    const int wave = tid >> 6;
    if (tid < 64) tb.depth[tid] = dep;
    bool cut_here = false;
    if constexpr (kQ) {
      if (tid < n_nq) tb.qitem[tid] = qit;
      cut_here = tid < n_nq && item_nparts(qit) > 1;
    }
    if constexpr (kK) {
      if (tid < n_ntile) tb.tend[tid] = tend_r;
      if (tid < n_nk) tb.kitem[tid] = kit0;
      if (tid + kThreads < n_nk) tb.kitem[tid + kThreads] = kit1;
      cut_here = (tid < n_nk && item_nparts(kit0) > 1) || (tid + kThreads < n_nk && item_nparts(kit1) > 1);
    }
    {
      const bool any_cut = __any(cut_here);
      if (lane == 0) tb.cut[wave] = any_cut;
    }
    if (tid < n_ntile * HG) {
      const int r = tid / HG;
      if constexpr ((kMode & kLse) != 0) tb.l2[tid - r * HG][r] = lse_r * kLog2e;
      if constexpr ((kMode & kDl) != 0) tb.dl[tid - r * HG][r] = dl_r;
    }
    // anc: in preorder the ancestor of row r at depth d+1 is the last row
    // i <= r of that depth (a tile row: slot P + i), or else prefix slot d.
    const uint64_t upto = lane == 63 ? ~0ull : ((2ull << lane) - 1);
    for (int d = wave; kQ && d < ldd; d += kWaves) {
      const uint64_t m = __ballot(dep == d + 1);
      if (lane < n_ntile) {
        int v = P + lane;  // padding past the row's depth: a valid slot
        if (d < dep) {
          const uint64_t mm = m & upto;
          v = mm ? P + 63 - __clzll(mm) : d;
        }
        anc[lane * ldd + d] = static_cast<int16_t>(v);
      }
    }
    t = n_t;
    s = n_s;
    ntile = n_ntile;
    A = n_A;
    poff = n_poff;
    if constexpr (kQ) nq = n_nq;
    if constexpr (kK) nk = n_nk;
    __syncthreads();
    cut = (tb.cut[0] | tb.cut[1] | tb.cut[2] | tb.cut[3]) != 0;
  }

  // Slot of tile row r, and of key-set entry k (prefix entries first).
  __device__ __forceinline__ int row_slot(int r) const { return P + r; }
  __device__ __forceinline__ int entry_slot(int k) const { return k < A ? k : P + (k - A); }
  // The four key-set slots of step b on the path of tile row r.
  __device__ __forceinline__ void slots(int r, int b, int (&sl)[kGroup]) const {
    const uint2 w = *reinterpret_cast<const uint2*>(anc + r * ldd + 4 * b);
    sl[0] = static_cast<int>(w.x & 0xffffu);
    sl[1] = static_cast<int>(w.x >> 16);
    sl[2] = static_cast<int>(w.y & 0xffffu);
    sl[3] = static_cast<int>(w.y >> 16);
  }
};

// Slot x of four (x = the lane's member index), without branches.
__device__ __forceinline__ int pick(const int (&sl)[kGroup], int x) {
  const int lo = x & 1 ? sl[1] : sl[0];
  const int hi = x & 1 ? sl[3] : sl[2];
  return x & 2 ? hi : lo;
}

// Walk steps of a round: those of its first (longest) item.
__device__ __forceinline__ int round_steps(int it) { return uniform(item_b1(it) - item_b0(it)); }

// Query chain group of one quad: rows, depths, the member this lane owns and
// the item's part: steps [b0, b1) of the path walk; member x takes the keys
// at path index < lim.
struct QueryItem {
  int it, r0, cnt, rl, p_last, pm, rx, b0, b1, lim;
  bool live;
  // Step index of walk step b (clamped into the part: past-the-end steps are
  // masked by lim).
  __device__ __forceinline__ int step(int b) const { return min(b0 + b, b1 - 1); }
  __device__ __forceinline__ bool key_live(int b, int r) const { return 4 * (b0 + b) + r < lim; }
};

template <int HG>
__device__ __forceinline__ QueryItem query_item(const StreamTables<HG>& tb, int n_items, int pos,
                                                int first, int x) {
  QueryItem q;
  q.live = pos < n_items;
  const int it = tb.qitem[q.live ? pos : first];
  q.it = it;
  q.r0 = item_first(it);
  q.cnt = item_count(it);
  q.rl = q.r0 + q.cnt - 1;
  q.p_last = tb.depth[q.rl];
  q.pm = (q.live && x < q.cnt) ? q.p_last - (q.cnt - 1 - x) : 0;  // member x sees depths d < pm
  q.rx = q.r0 + min(x, q.cnt - 1);
  q.b0 = item_b0(it);
  q.b1 = item_b1(it);
  q.lim = min(q.pm, 4 * q.b1);
  return q;
}

// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, typename PlanT>
__global__ __launch_bounds__(kThreads) void fwd_kernel(PlanT pl, const Tin* __restrict__ Q,
                                                       const Tin* __restrict__ K,
                                                       const Tin* __restrict__ V,
                                                       Tin* __restrict__ O,
                                                       float* __restrict__ lse, int H, float scale) {
  constexpr int DPL = HD / kGroup;
  constexpr int ITEMS = 64 / (kGroup * HG);
  using ST = Stream<HD, Tin, HG, 1, kQSide, PlanT>;
  constexpr int WS = ST::WS;
  __shared__ StreamTables<HG> tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  int hg, t0, t1;
  assign_range(pl.n_tiles, H / HG, hg, t0, t1);
  if (t0 >= t1) return;
  ST st(pl, K, V, Q, nullptr, nullptr, nullptr, nullptr, H, hg, dyn, tb);
  // Scratch of cut items: [slot][part][head][member][P·V (HD) | m, l, pad].
  constexpr int FP = fwd_part_floats(HD);
  float* scr = reinterpret_cast<float*>(dyn + ST::lds_bytes(pl.max_depth));
  auto scr_at = [&](int slot, int part, int hh, int m) {
    return scr + (((slot * kQParts + part) * HG + hh) * kGroup + m) * FP;
  };
  const int D = H * HD;
  const Lane<HG> ln;
  const int x = ln.x;
  const int h = hg * HG + ln.hl;
  const int hoff = ln.hl * HD;
  const float qscale = scale * kLog2e;
  st.s = 0;
  st.prefetch(t0);
  st.commit(true);
  for (int t = t0; t < t1; ++t) {
    if (t + 1 < t1) st.prefetch(t + 1);
    for (int round = ln.wave; round * ITEMS < st.nq; round += kWaves) {
      const int first = round * ITEMS;
      const int nblk = round_steps(tb.qitem[first]);
      const QueryItem qi = query_item<HG>(tb, st.nq, first + ln.slot, first, x);
      float q[HD], ks[HD];
      load_vec<HD>(st.Ts + qi.rx * WS + hoff, q);
      load_vec<HD>(st.Ks + st.row_slot(qi.rx) * WS + hoff, ks);
#pragma unroll
      for (int i = 0; i < HD; ++i) q[i] *= qscale;
      float m = dot<HD>(q, ks);  // self score: the running max starts here
      float l = 0.0f;
      f4 acc[DPL];
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int b = 0; b < nblk; ++b) {
        int sl[kGroup];
        st.slots(qi.rl, qi.step(b), sl);
        float kr[HD], vc[kGroup][DPL];
        load_vec<HD>(st.Ks + pick(sl, x) * WS + hoff, kr);
#pragma unroll
        for (int k = 0; k < kGroup; ++k) load_vec<DPL>(st.Vs + sl[k] * WS + hoff + x * DPL, vc[k]);
        const f4 sv = mfma_dot<HD>(kr, q);  // sv[r]: key 4b+r against member x
        float sc[kGroup], mx = m;
#pragma unroll
        for (int r = 0; r < kGroup; ++r) {
          sc[r] = qi.key_live(b, r) ? sv[r] : -__builtin_inff();
          mx = fmaxf(mx, sc[r]);
        }
        const bool resc = mx > m + kRescaleLog2;
        if (__any(resc)) {
          const float alpha = resc ? fast_exp2(m - mx) : 1.0f;
          m = resc ? mx : m;
          l *= alpha;
          float al[kGroup];
          quad_bcast_all(alpha, al);
#pragma unroll
          for (int i = 0; i < DPL; ++i)
#pragma unroll
            for (int g = 0; g < kGroup; ++g) acc[i][g] *= al[g];
        }
        float p[kGroup];
#pragma unroll
        for (int r = 0; r < kGroup; ++r) {
          p[r] = fast_exp2(sc[r] - m);  // exp2(-inf) = 0 for masked keys
          l += p[r];
        }
        mfma_accum<DPL>(acc, p, vc);
      }
      if (item_nparts(qi.it) > 1) {
        // One part of a cut item: its softmax state to the scratch slot.
        if (qi.live) {
          const int sl = item_slot(qi.it), pt = item_part(qi.it);
#pragma unroll
          for (int g = 0; g < kGroup; ++g) {
            if (g < qi.cnt) {
              float o[DPL];
#pragma unroll
              for (int i = 0; i < DPL; ++i) o[i] = acc[i][g];
              store_vec<DPL>(scr_at(sl, pt, ln.hl, g) + x * DPL, o);
            }
          }
          if (x < qi.cnt) {
            scr_at(sl, pt, ln.hl, x)[HD] = m;
            scr_at(sl, pt, ln.hl, x)[HD + 1] = l;
          }
        }
        continue;
      }
      const float inv = qi.pm > 0 ? 1.0f / l : 0.0f;
      float il[kGroup];
      quad_bcast_all(inv, il);
      if (qi.live) {
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
          if (g < qi.cnt) {
            float o[DPL];
#pragma unroll
            for (int i = 0; i < DPL; ++i) o[i] = acc[i][g] * il[g];
            store_vec<DPL>(O + (static_cast<int64_t>(st.s) + qi.r0 + g) * D + h * HD + x * DPL, o);
          }
        }
        if (x < qi.cnt) lse[(static_cast<int64_t>(st.s) + qi.rx) * H + h] = (m + fast_log2(l)) * kLn2;
      }
    }
    // Cut items: combine the parts' softmax states in part order. One thread
    // per (member, head, DPL-slice) of an item.
    if (st.cut) {
      __syncthreads();
      constexpr int kJobs = kGroup * HG * kGroup;
      for (int j = threadIdx.x; j < st.nq * kJobs; j += kThreads) {
        const int it = tb.qitem[j / kJobs];
        if (item_nparts(it) == 1 || item_part(it) != 0) continue;
        const int r = j % kJobs;
        const int g = r / (HG * kGroup);
        const int hh = (r / kGroup) % HG;
        const int d0 = (r % kGroup) * DPL;
        if (g >= item_count(it)) continue;
        const int sl = item_slot(it), np = item_nparts(it);
        float mp[kQParts], mx = -__builtin_inff();
#pragma unroll
        for (int p = 0; p < kQParts; ++p) {
          mp[p] = p < np ? scr_at(sl, p, hh, g)[HD] : -__builtin_inff();
          mx = fmaxf(mx, mp[p]);
        }
        float l = 0.0f, o[DPL];
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[i] = 0.0f;
#pragma unroll
        for (int p = 0; p < kQParts; ++p) {
          if (p < np) {
            const float a = fast_exp2(mp[p] - mx);
            float y[DPL];
            load_vec<DPL>(scr_at(sl, p, hh, g) + d0, y);
            l += a * scr_at(sl, p, hh, g)[HD + 1];
#pragma unroll
            for (int i = 0; i < DPL; ++i) o[i] += a * y[i];
          }
        }
        const float inv = 1.0f / l;
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[i] *= inv;
        const int64_t row = static_cast<int64_t>(st.s) + item_first(it) + g;
        const int hd = hg * HG + hh;
        store_vec<DPL>(O + row * D + hd * HD + d0, o);
        if (d0 == 0) lse[row * H + hd] = (mx + fast_log2(l)) * kLn2;
      }
    }
    if (t + 1 < t1) st.commit(false);
  }
}

// ---------------------------------------------------------------------------
// Backward, query side: δ and dQ. δ = dO·O for fp32 inputs (from the chunk
// partials); for bf16 inputs O is a rounded output, so δ = Σ_j w_j dO·v_j is
// recomputed over the path in fp32 (batched_depth_backward.cr:637-646). δ is
// written to Dl [T, H] for the key side.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) void bwd_q_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const Tin* __restrict__ O, const float* __restrict__ lse, const Tin* __restrict__ dO,
    float* __restrict__ dQ, float* __restrict__ Dl, RopeT rope, int H, float scale) {
  constexpr int DPL = HD / kGroup;
  constexpr int ITEMS = 64 / (kGroup * HG);
  constexpr bool kDeltaFromO = sizeof(Tin) == sizeof(float);
  constexpr int NT = kDeltaFromO ? 3 : 2;
  using ST = Stream<HD, Tin, HG, NT, kQSide | kLse, PlanT>;
  constexpr int WS = ST::WS;
  __shared__ StreamTables<HG> tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  int hg, t0, t1;
  assign_range(pl.n_tiles, H / HG, hg, t0, t1);
  if (t0 >= t1) return;
  ST st(pl, K, V, Q, dO, O, lse, nullptr, H, hg, dyn, tb);
  // Scratch of cut items (fp32 only: the bf16 δ walk needs the whole path):
  // [slot][part][head][member][HD] dQ partials.
  float* scr = reinterpret_cast<float*>(dyn + ST::lds_bytes(pl.max_depth));
  auto scr_at = [&](int slot, int part, int hh, int m) {
    return scr + (((slot * kQParts + part) * HG + hh) * kGroup + m) * HD;
  };
  const int D = H * HD;
  const Lane<HG> ln;
  const int x = ln.x;
  const int h = hg * HG + ln.hl;
  const int hoff = ln.hl * HD;
  const float qscale = scale * kLog2e;
  const Tin* Qs = st.Ts;
  const Tin* Gs = st.Ts + kTile * WS;
  st.s = 0;
  st.prefetch(t0);
  st.commit(true);
  for (int t = t0; t < t1; ++t) {
    if (t + 1 < t1) st.prefetch(t + 1);
    const int64_t s = st.s;
    for (int round = ln.wave; round * ITEMS < st.nq; round += kWaves) {
      const int first = round * ITEMS;
      const int nblk = round_steps(tb.qitem[first]);
      const QueryItem qi = query_item<HG>(tb, st.nq, first + ln.slot, first, x);
      const float l2 = tb.l2[ln.hl][qi.rx];
      float q[HD], go[HD];
      load_vec<HD>(Qs + qi.rx * WS + hoff, q);
      load_vec<HD>(Gs + qi.rx * WS + hoff, go);
#pragma unroll
      for (int i = 0; i < HD; ++i) q[i] *= qscale;
      // Scores and dO·v of step b: lane x gets member x against the 4 keys.
      auto step = [&](int b, int (&sl)[kGroup], f4& sv, f4& tv) {
        st.slots(qi.rl, qi.step(b), sl);
        const int mine = pick(sl, x);
        float kr[HD], vr[HD];
        load_vec<HD>(st.Ks + mine * WS + hoff, kr);
        load_vec<HD>(st.Vs + mine * WS + hoff, vr);
        sv = mfma_dot<HD>(kr, q);
        tv = mfma_dot<HD>(vr, go);
      };
      float dl = 0.0f;
      if constexpr (kDeltaFromO) {
        const float* pp = st.pdl + (qi.rx * HG + ln.hl) * ST::CPH;
#pragma unroll
        for (int c = 0; c < ST::CPH; ++c) dl += pp[c];
      } else {
        for (int b = 0; b < nblk; ++b) {
          int sl[kGroup];
          f4 sv, tv;
          step(b, sl, sv, tv);
#pragma unroll
          for (int r = 0; r < kGroup; ++r) {
            const float w = qi.key_live(b, r) ? fast_exp2(sv[r] - l2) : 0.0f;
            dl += w * tv[r];
          }
        }
      }
      f4 dq[DPL];
#pragma unroll
      for (int i = 0; i < DPL; ++i) dq[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int b = 0; b < nblk; ++b) {
        int sl[kGroup];
        f4 sv, tv;
        step(b, sl, sv, tv);
        float ds[kGroup];
#pragma unroll
        for (int r = 0; r < kGroup; ++r) {
          const float w = qi.key_live(b, r) ? fast_exp2(sv[r] - l2) : 0.0f;
          ds[r] = w * (tv[r] - dl) * scale;
        }
        // The key rows are dead here; keep the chunk loads below this point
        // so both never hold registers at once.
        __builtin_amdgcn_sched_barrier(0);
        float kc[kGroup][DPL];
#pragma unroll
        for (int k = 0; k < kGroup; ++k) load_vec<DPL>(st.Ks + sl[k] * WS + hoff + x * DPL, kc[k]);
        mfma_accum<DPL>(dq, ds, kc);
      }
      if (qi.live && item_nparts(qi.it) > 1) {
        // One part of a cut item: its dQ partial to the scratch slot.
        const int sl = item_slot(qi.it), pt = item_part(qi.it);
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
          if (g < qi.cnt) {
            float v[DPL];
#pragma unroll
            for (int i = 0; i < DPL; ++i) v[i] = dq[i][g];
            store_vec<DPL>(scr_at(sl, pt, ln.hl, g) + x * DPL, v);
          }
        }
        if (pt == 0 && x < qi.cnt) Dl[(s + qi.rx) * H + h] = dl;
      } else if (qi.live) {
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
          if (g < qi.cnt) {
            float v[DPL];
#pragma unroll
            for (int i = 0; i < DPL; ++i) v[i] = dq[i][g];
            if (rope.cos_t)
              rope_inverse_part<DPL, HD>(v, rope.cos_t, rope.sin_t,
                                         rope_pos(qi.p_last - (qi.cnt - 1 - g), rope.seq_len), x * DPL);
            store_vec<DPL>(dQ + (s + qi.r0 + g) * D + h * HD + x * DPL, v);
          }
        }
        if (x < qi.cnt) Dl[(s + qi.rx) * H + h] = dl;
      }
    }
    // Cut items: sum the dQ partials in part order, then inverse RoPE. One
    // thread per (member, head, DPL-slice) of an item.
    if (st.cut) {
      __syncthreads();
      constexpr int kJobs = kGroup * HG * kGroup;
      for (int j = threadIdx.x; j < st.nq * kJobs; j += kThreads) {
        const int it = tb.qitem[j / kJobs];
        if (item_nparts(it) == 1 || item_part(it) != 0) continue;
        const int r = j % kJobs;
        const int g = r / (HG * kGroup);
        const int hh = (r / kGroup) % HG;
        const int d0 = (r % kGroup) * DPL;
        const int cnt = item_count(it);
        if (g >= cnt) continue;
        const int sl = item_slot(it), np = item_nparts(it);
        float v[DPL];
        load_vec<DPL>(scr_at(sl, 0, hh, g) + d0, v);
#pragma unroll
        for (int p = 1; p < kQParts; ++p) {
          if (p < np) {
            float y[DPL];
            load_vec<DPL>(scr_at(sl, p, hh, g) + d0, y);
#pragma unroll
            for (int i = 0; i < DPL; ++i) v[i] += y[i];
          }
        }
        const int r0 = item_first(it);
        if (rope.cos_t)
          rope_inverse_part<DPL, HD>(v, rope.cos_t, rope.sin_t,
                                     rope_pos(tb.depth[r0 + cnt - 1] - (cnt - 1 - g), rope.seq_len), d0);
        store_vec<DPL>(dQ + (s + r0 + g) * D + (hg * HG + hh) * HD + d0, v);
      }
    }
    if (t + 1 < t1) st.commit(false);
  }
}

// ---------------------------------------------------------------------------
// Backward, key side: dK / dV of the tile's key set. Prefix keys leave their
// partial over this tile in Pk/Pv (row pref_off[t] + depth-1); tile rows
// whose subtree ends inside the tile are finished here (seed, inverse RoPE);
// open tile rows leave their partial in dK/dV for the reduction kernels.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) void bwd_kv_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const float* __restrict__ lse, const float* __restrict__ Dl, const Tin* __restrict__ dO,
    float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ Pk, float* __restrict__ Pv,
    const float* __restrict__ acc_dk, const float* __restrict__ acc_dv, RopeT rope, int H,
    float scale) {
  constexpr int DPL = HD / kGroup;
  constexpr int ITEMS = 64 / (kGroup * HG);
  using ST = Stream<HD, Tin, HG, 2, kKSide | kLse | kDl, PlanT>;
  constexpr int WS = ST::WS;
  __shared__ StreamTables<HG> tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  int hg, t0, t1;
  assign_range(pl.n_tiles, H / HG, hg, t0, t1);
  if (t0 >= t1) return;
  ST st(pl, K, V, Q, dO, nullptr, lse, Dl, H, hg, dyn, tb);
  // Scratch of cut items: [slot][part][head][member][dK|dV][HD].
  float* scr = reinterpret_cast<float*>(dyn + ST::lds_bytes(pl.max_depth));
  auto scr_at = [&](int slot, int part, int hh, int m, int kv) {
    return scr + ((((slot * kKParts + part) * HG + hh) * kGroup + m) * 2 + kv) * HD;
  };
  const int D = H * HD;
  const Lane<HG> ln;
  const int x = ln.x;
  const int hoff = ln.hl * HD;
  const float qscale = scale * kLog2e;
  const Tin* Qs = st.Ts;
  const Tin* Gs = st.Ts + kTile * WS;
  const float* l2h = tb.l2[ln.hl];
  const float* dlh = tb.dl[ln.hl];
  st.s = 0;
  st.prefetch(t0);
  st.commit(true);
  for (int t = t0; t < t1; ++t) {
    if (t + 1 < t1) st.prefetch(t + 1);
    const int64_t s = st.s;
    const int A = st.A, ntile = st.ntile;
    auto range_lo = [&](int k) { return k < A ? 0 : k - A; };
    auto range_hi = [&](int k) {
      return k < A ? min(tb.pend[k] - st.s, ntile) : min(tb.tend[k - A] - st.s, ntile);
    };
    // Query range of item `it`: its steps of the group's range (the first
    // member's range contains the others').
    auto part_range = [&](int it, int& lo, int& hi) {
      const int k0 = item_first(it);
      const int glo = range_lo(k0);
      lo = glo + 4 * item_b0(it);
      hi = min(glo + 4 * item_b1(it), range_hi(k0));
    };
    // Final dK/dV of key-set entry ki (dims x*DPL.. of head h): prefix keys
    // leave the tile's partial in Pk/Pv; tile rows whose subtree ends inside
    // the tile are finished (seed, inverse RoPE), open ones leave a partial.
    auto emit = [&](int ki, int hh, int d0, float (&gk)[DPL], float (&gv)[DPL]) {
      const int hd = hg * HG + hh;
      if (ki < A) {
        const int64_t row = static_cast<int64_t>(st.poff) + ki;
        store_vec<DPL>(Pk + row * D + hd * HD + d0, gk);
        store_vec<DPL>(Pv + row * D + hd * HD + d0, gv);
      } else {
        const int c = ki - A;
        const int64_t a = s + c;
        if (tb.tend[c] <= s + ntile) {
          if (acc_dk) {
            float y[DPL];
            load_vec<DPL>(acc_dk + a * D + hd * HD + d0, y);
#pragma unroll
            for (int i = 0; i < DPL; ++i) gk[i] += y[i];
          }
          if (acc_dv) {
            float y[DPL];
            load_vec<DPL>(acc_dv + a * D + hd * HD + d0, y);
#pragma unroll
            for (int i = 0; i < DPL; ++i) gv[i] += y[i];
          }
          if (rope.cos_t)
            rope_inverse_part<DPL, HD>(gk, rope.cos_t, rope.sin_t, rope_pos(tb.depth[c], rope.seq_len), d0);
        }
        store_vec<DPL>(dK + a * D + hd * HD + d0, gk);
        store_vec<DPL>(dV + a * D + hd * HD + d0, gv);
      }
    };
    for (int round = ln.wave; round * ITEMS < st.nk; round += kWaves) {
      const int first = round * ITEMS;
      const int nblk = round_steps(tb.kitem[first]);
      const int pos = first + ln.slot;
      const bool live = pos < st.nk;
      const int it = tb.kitem[live ? pos : first];
      const int k0 = item_first(it);
      const int cnt = item_count(it);
      const int kx = k0 + min(x, cnt - 1);  // entry of the member this lane owns
      float kk[HD], vv[HD];
      load_vec<HD>(st.Ks + st.entry_slot(kx) * WS + hoff, kk);
      load_vec<HD>(st.Vs + st.entry_slot(kx) * WS + hoff, vv);
#pragma unroll
      for (int i = 0; i < HD; ++i) kk[i] *= qscale;
      int lo, hi;
      part_range(it, lo, hi);
      // Member x takes the queries of its range inside this item's part (the
      // round may run past the part); padding members take none.
      const int klo = max(range_lo(kx), lo);
      const int khi = (live && x < cnt) ? min(range_hi(kx), hi) : klo;
      f4 dk[DPL], dv[DPL];
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        dk[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        dv[i] = dk[i];
      }
      for (int b = 0; b < nblk; ++b) {
        const int j0 = lo + 4 * b;
        const int jr = min(j0 + x, hi - 1);  // query row this lane supplies
        float qr[HD], gr[HD], l2[kGroup], dl[kGroup];
        load_vec<HD>(Qs + jr * WS + hoff, qr);
        load_vec<HD>(Gs + jr * WS + hoff, gr);
#pragma unroll
        for (int k = 0; k < kGroup; ++k) {
          const int j = min(j0 + k, hi - 1);
          l2[k] = l2h[j];
          dl[k] = dlh[j];
        }
        const f4 sv = mfma_dot<HD>(qr, kk);  // sv[r]: query j0+r against key member x
        const f4 tv = mfma_dot<HD>(gr, vv);
        float w[kGroup], ds[kGroup];
#pragma unroll
        for (int r = 0; r < kGroup; ++r) {
          const int j = j0 + r;
          w[r] = (j >= klo && j < khi) ? fast_exp2(sv[r] - l2[r]) : 0.0f;
          ds[r] = w[r] * (tv[r] - dl[r]) * scale;
        }
        // The query rows are dead here; keep the chunk loads below this point
        // so both never hold registers at once.
        __builtin_amdgcn_sched_barrier(0);
        float qc[kGroup][DPL], gc[kGroup][DPL];
#pragma unroll
        for (int k = 0; k < kGroup; ++k) {
          const int j = min(j0 + k, hi - 1);
          load_vec<DPL>(Qs + j * WS + hoff + x * DPL, qc[k]);
          load_vec<DPL>(Gs + j * WS + hoff + x * DPL, gc[k]);
        }
        mfma_accum<DPL>(dk, ds, qc);
        mfma_accum<DPL>(dv, w, gc);
      }
      if (!live) continue;
      const bool cut = item_nparts(it) > 1;
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        if (g >= cnt) continue;
        float gk[DPL], gv[DPL];
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          gk[i] = dk[i][g];
          gv[i] = dv[i][g];
        }
        if (cut) {  // one part of a cut item: to the scratch slot
          store_vec<DPL>(scr_at(item_slot(it), item_part(it), ln.hl, g, 0) + x * DPL, gk);
          store_vec<DPL>(scr_at(item_slot(it), item_part(it), ln.hl, g, 1) + x * DPL, gv);
        } else {
          emit(k0 + g, ln.hl, x * DPL, gk, gv);
        }
      }
    }
    // Cut items: sum the parts in part order and emit. One thread per
    // (member, head, DPL-slice) of an item.
    if (st.cut) {
      __syncthreads();
      constexpr int kJobs = kGroup * HG * kGroup;  // member, head, slice
      for (int j = threadIdx.x; j < st.nk * kJobs; j += kThreads) {
        const int it = tb.kitem[j / kJobs];
        if (item_nparts(it) == 1 || item_part(it) != 0) continue;
        const int r = j % kJobs;
        const int g = r / (HG * kGroup);
        const int hh = (r / kGroup) % HG;
        const int d0 = (r % kGroup) * DPL;
        if (g >= item_count(it)) continue;
        const int sl = item_slot(it), np = item_nparts(it);
        float a[DPL], b[DPL];
        load_vec<DPL>(scr_at(sl, 0, hh, g, 0) + d0, a);
        load_vec<DPL>(scr_at(sl, 0, hh, g, 1) + d0, b);
#pragma unroll
        for (int p = 1; p < kKParts; ++p) {
          if (p < np) {
            float y[DPL], z[DPL];
            load_vec<DPL>(scr_at(sl, p, hh, g, 0) + d0, y);
            load_vec<DPL>(scr_at(sl, p, hh, g, 1) + d0, z);
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
              a[i] += y[i];
              b[i] += z[i];
            }
          }
        }
        emit(item_first(it) + g, hh, d0, a, b);
      }
    }
    if (t + 1 < t1) st.commit(false);
  }
}

}  // namespace agpt_fast
