// trie_fast.h — the fast trie-attention kernels (included by trie_attn.hip).
//
// Workgroup = (tile, head group): a tile is pl.tile consecutive DFS rows
// [s, e), the head group HG heads; blockDim.x / 64 waves.
//
// Work items are chain groups built by the plan: up to four consecutive rows
// (queries) or key-set entries (keys) where each is the previous one's child
// — the interior of a radix edge. Nearly every row of a chain-dominated trie
// sits in a full group.
//
// One item-head pair runs on a quad of adjacent lanes. Lane c of the quad
// holds head dims [c*HD/4, (c+1)*HD/4) of all four members and owns the
// scalar softmax state of member c; its register slot j holds member j ^ c.
// A member's full dot product is the sum of four lane partials: the
// transpose-reduce (two DPP exchanges) leaves member c's sum in lane c, and
// per-member scalars are broadcast back over the quad with quad_perm DPP.
// With that layout the 4*HG lanes of an item read one contiguous row slice
// of HG*HD elements per staged vector, so LDS reads carry no bank conflicts,
// and each K/V (resp. Q/dO) read serves four members.
//
//  fwd_kernel, bwd_q_kernel: item = query chain group r0..r0+n-1. Member i
//    sees the keys at depth <= depth(r0+i), all on the last member's path, so
//    one walk over that path serves the group. The head-group slice of the
//    tile's key set — the A prefix rows (ancestors of s by depth), then the
//    tile rows — is staged in LDS, and every row's path is an LDS table
//    anc[depth][row] of key-set slots.
//  bwd_kv_kernel: item = key chain group; its subtrees are nested, so one
//    pass over the first member's query range serves all of them (member i
//    takes query j iff a_i <= j < end(a_i)). The tile's Q and dO slices are
//    staged in LDS.
//
// Balance: the plan stores each tile's items sorted by cost (walk length,
// resp. query-range length), longest first; a round is 16/HG consecutive
// sorted items, so the lanes of a wave do similar work. Wave w of the
// workgroup takes rounds w, w+nw, ...
//
// The running softmax max starts at the member's self score and moves only
// when a score exceeds it by more than 2^8 (then the sums are rescaled).
//
// Blocks are dealt to the 8 XCDs round-robin; block b runs work item
// (b % 8) * per + b / 8 so each XCD sweeps a contiguous stretch of tiles,
// whose shared prefix rows then stay in that XCD's L2.
#pragma once

namespace agpt_fast {

using namespace agpt;

constexpr int kXcds = 8;
constexpr int kMaxTile = 128;
constexpr int kGroup = 4;             // chain-group members = lanes per item-head quad
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)

// A work item packs (first entry, member count): first | (count << 10).
__host__ __device__ constexpr int item_first(int v) { return v & 1023; }
__host__ __device__ constexpr int item_count(int v) { return v >> 10; }
__host__ __device__ constexpr int make_item(int first, int count) { return first | (count << 10); }

struct Tables {
  int32_t parent[kMaxTile];  // tile-local parent, or -1 when outside the tile
  int32_t depth[kMaxTile];
  int32_t end[kMaxTile];     // tile-local subtree end, clamped to ntile
  int32_t prefix[kMaxDepth];
  int32_t prefix_end[kMaxDepth];  // tile-local, clamped to [0, ntile]
  int16_t item[kMaxTile + kMaxDepth];
};

__device__ __forceinline__ bool map_block(int n_tiles, int n_hg, int& t, int& hg) {
  const int nb = n_tiles * n_hg;
  const int per = (nb + kXcds - 1) / kXcds;
  const int b = blockIdx.x;
  const int L = (b % kXcds) * per + b / kXcds;
  if (L >= nb) return false;
  t = L / n_hg;
  hg = L - t * n_hg;
  return true;
}

template <typename PlanT>
struct Tile {
  int t, hg, ntile, A;
  int32_t s, poff;
  __device__ __forceinline__ bool init(const PlanT& pl, int n_hg) {
    if (!map_block(pl.n_tiles, n_hg, t, hg)) return false;
    s = t * pl.tile;
    ntile = min(pl.tile, static_cast<int>(pl.T - s));
    poff = pl.pref_off[t];
    A = pl.pref_off[t + 1] - poff;
    return true;
  }
};

template <typename PlanT>
__device__ __forceinline__ void load_tables(const PlanT& pl, const Tile<PlanT>& tl, Tables& sh,
                                            const int16_t* __restrict__ item_src, int n_items) {
  const int32_t s = tl.s;
  for (int i = threadIdx.x; i < tl.ntile; i += blockDim.x) {
    const int32_t p = pl.parent[s + i];
    sh.parent[i] = p >= s ? p - s : -1;
    sh.depth[i] = pl.depth[s + i];
    sh.end[i] = min(pl.end[s + i] - s, tl.ntile);
  }
  for (int i = threadIdx.x; i < tl.A; i += blockDim.x) {
    const int32_t a = pl.prefix[tl.poff + i];
    sh.prefix[i] = a;
    sh.prefix_end[i] = min(pl.end[a] - s, tl.ntile);
  }
  for (int i = threadIdx.x; i < n_items; i += blockDim.x) sh.item[i] = item_src[i];
}

// Copies the width-element slice (column col0) of n_rows rows — row i is
// prefix[i] for i < A, else s + i - A — into dst (row stride width).
template <typename Tin>
__device__ __forceinline__ void stage_rows(Tin* __restrict__ dst, const Tin* __restrict__ src,
                                           int D, int col0, int width, int n_rows,
                                           const int32_t* __restrict__ prefix, int A, int32_t s) {
  constexpr int kPer16 = 16 / sizeof(Tin);
  const int chunks = width / kPer16;
  for (int i = threadIdx.x; i < n_rows * chunks; i += blockDim.x) {
    const int slot = i / chunks;
    const int c = i - slot * chunks;
    const int64_t row = slot < A ? static_cast<int64_t>(prefix[slot]) : static_cast<int64_t>(s) + (slot - A);
    *reinterpret_cast<uint4*>(dst + slot * width + c * kPer16) =
        *reinterpret_cast<const uint4*>(src + row * D + col0 + c * kPer16);
  }
}

// anc[d * ldr + r] = key-set slot of row r's ancestor at depth d+1: tile rows
// map to A + row, rows outside the tile (the prefix) to d.
__device__ __forceinline__ void build_anc(const Tables& sh, int A, int ntile, int16_t* __restrict__ anc,
                                          int ldr) {
  for (int r = threadIdx.x; r < ntile; r += blockDim.x) {
    int cur = r;
    int d = sh.depth[r] - 1;
    for (;;) {
      anc[d * ldr + r] = static_cast<int16_t>(A + cur);
      --d;
      cur = sh.parent[cur];
      if (cur < 0) break;
    }
    for (; d >= 0; --d) anc[d * ldr + r] = static_cast<int16_t>(d);
  }
}

// ---- quad exchanges (quad_perm DPP: lane c reads lane c ^ k of its quad) ---
template <int CTRL>
__device__ __forceinline__ float qperm(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
constexpr int kXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kXor3 = 0x1B;  // quad_perm [3,2,1,0]

// p[j] = this lane's partial for member j ^ c; returns member c's full sum.
__device__ __forceinline__ float quad_reduce(const float (&p)[kGroup]) {
  const float a0 = p[0] + qperm<kXor2>(p[2]);  // members c, c^1 over lanes {c, c^2}
  const float a1 = p[1] + qperm<kXor2>(p[3]);
  return a0 + qperm<kXor1>(a1);
}

// x = member c's scalar in lane c; out[j] = member (j ^ c)'s scalar.
__device__ __forceinline__ void quad_bcast(float x, float (&out)[kGroup]) {
  out[0] = x;
  out[1] = qperm<kXor1>(x);
  out[2] = qperm<kXor2>(x);
  out[3] = qperm<kXor3>(x);
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

// Lane coordinates: quad q = lane / 4 holds item slot q / HG, head q % HG.
template <int HG>
struct Lane {
  int wave, nw, c, slot, hl;
  __device__ __forceinline__ Lane() {
    wave = threadIdx.x >> 6;
    nw = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    c = lane & 3;
    const int quad = lane >> 2;
    slot = quad / HG;
    hl = quad - slot * HG;
  }
};

// Shared set-up of the query-side kernels: tables, key-set staging, anc.
template <int HD, typename Tin, int HG, typename PlanT>
struct QuerySide {
  static constexpr int W = HG * HD;
  Tin* Ks;
  Tin* Vs;
  int16_t* anc;
  int ldr;
  __device__ __forceinline__ void setup(const PlanT& pl, const Tile<PlanT>& tl, Tables& sh,
                                        unsigned char* dyn, const Tin* K, const Tin* V, int D,
                                        int n_items) {
    const int key_rows = pl.max_depth - 1 + pl.tile;
    Ks = reinterpret_cast<Tin*>(dyn);
    Vs = Ks + key_rows * W;
    anc = reinterpret_cast<int16_t*>(Vs + key_rows * W);
    ldr = pl.tile;
    load_tables(pl, tl, sh, pl.q_items + pl.q_item_off[tl.t], n_items);
    __syncthreads();
    stage_rows(Ks, K, D, tl.hg * W, W, tl.A + tl.ntile, sh.prefix, tl.A, tl.s);
    stage_rows(Vs, V, D, tl.hg * W, W, tl.A + tl.ntile, sh.prefix, tl.A, tl.s);
    build_anc(sh, tl.A, tl.ntile, anc, ldr);
    __syncthreads();
  }
};

// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, typename PlanT>
__global__ __launch_bounds__(256) void fwd_kernel(PlanT pl, const Tin* __restrict__ Q,
                                                  const Tin* __restrict__ K,
                                                  const Tin* __restrict__ V, Tin* __restrict__ O,
                                                  float* __restrict__ lse, int H, float scale) {
  constexpr int DPL = HD / kGroup;
  constexpr int ITEMS = 64 / (kGroup * HG);
  using QS = QuerySide<HD, Tin, HG, PlanT>;
  constexpr int W = QS::W;
  __shared__ Tables sh;
  extern __shared__ __align__(16) unsigned char dyn[];
  Tile<PlanT> tl;
  if (!tl.init(pl, H / HG)) return;
  const int D = H * HD;
  const int n_items = pl.q_item_off[tl.t + 1] - pl.q_item_off[tl.t];
  QS qs;
  qs.setup(pl, tl, sh, dyn, K, V, D, n_items);

  const Lane<HG> ln;
  const int c = ln.c;
  const int h = tl.hg * HG + ln.hl;
  const int col = ln.hl * HD + c * DPL;  // this lane's dims inside a staged row
  const float qscale = scale * kLog2e;
  for (int round = ln.wave; round * ITEMS < n_items; round += ln.nw) {
    const int pos = round * ITEMS + ln.slot;
    if (pos >= n_items) continue;  // uniform over the quad
    const int it = sh.item[pos];
    const int r0 = item_first(it);
    const int cnt = item_count(it);
    const int rl = r0 + cnt - 1;
    const int p_last = sh.depth[rl];
    const int pm = c < cnt ? p_last - (cnt - 1 - c) : 0;  // member c sees depths d < pm
    float q[kGroup][DPL], acc[kGroup][DPL], part[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const int r = r0 + min(j ^ c, cnt - 1);
      load_vec<DPL>(Q + (static_cast<int64_t>(tl.s) + r) * D + h * HD + c * DPL, q[j]);
      float k0[DPL];
      load_vec<DPL>(qs.Ks + (tl.A + r) * W + col, k0);
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        q[j][i] *= qscale;
        acc[j][i] = 0.0f;
      }
      part[j] = dot<DPL>(q[j], k0);
    }
    float m = quad_reduce(part);  // self score: the running max starts here
    float l = 0.0f;
    for (int d = p_last - 1; d >= 0; --d) {
      const int sl = qs.anc[d * qs.ldr + rl];
      float kk[DPL], vv[DPL];
      load_vec<DPL>(qs.Ks + sl * W + col, kk);
      load_vec<DPL>(qs.Vs + sl * W + col, vv);
#pragma unroll
      for (int j = 0; j < kGroup; ++j) part[j] = dot<DPL>(q[j], kk);
      const float sc = quad_reduce(part);
      const bool vis = d < pm;
      const bool resc = vis && sc > m + kRescaleLog2;
      if (__any(resc)) {
        const float alpha = resc ? fast_exp2(m - sc) : 1.0f;
        m = resc ? sc : m;
        l *= alpha;
        float al[kGroup];
        quad_bcast(alpha, al);
#pragma unroll
        for (int j = 0; j < kGroup; ++j)
#pragma unroll
          for (int i = 0; i < DPL; ++i) acc[j][i] *= al[j];
      }
      const float pr = vis ? fast_exp2(sc - m) : 0.0f;
      l += pr;
      float pj[kGroup];
      quad_bcast(pr, pj);
#pragma unroll
      for (int j = 0; j < kGroup; ++j)
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[j][i] += pj[j] * vv[i];
    }
    const float inv = c < cnt ? 1.0f / l : 0.0f;
    float il[kGroup];
    quad_bcast(inv, il);
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const int mem = j ^ c;
      if (mem < cnt) {
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[j][i] *= il[j];
        store_vec<DPL>(O + (static_cast<int64_t>(tl.s) + r0 + mem) * D + h * HD + c * DPL, acc[j]);
      }
    }
    if (c < cnt) lse[(static_cast<int64_t>(tl.s) + r0 + c) * H + h] = (m + fast_log2(l)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Backward, query side: δ and dQ. δ = dO·O for fp32 inputs; for bf16 inputs
// O is a rounded output, so δ = Σ_j w_j (dO·v_j) is recomputed over the path
// in fp32 (batched_depth_backward.cr:637-646). δ is written to Dl [T, H].
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, typename PlanT, typename RopeT>
__global__ __launch_bounds__(256) void bwd_q_kernel(PlanT pl, const Tin* __restrict__ Q,
                                                    const Tin* __restrict__ K,
                                                    const Tin* __restrict__ V,
                                                    const Tin* __restrict__ O,
                                                    const float* __restrict__ lse,
                                                    const Tin* __restrict__ dO,
                                                    float* __restrict__ dQ, float* __restrict__ Dl,
                                                    RopeT rope, int H, float scale) {
  constexpr int DPL = HD / kGroup;
  constexpr int ITEMS = 64 / (kGroup * HG);
  using QS = QuerySide<HD, Tin, HG, PlanT>;
  constexpr int W = QS::W;
  __shared__ Tables sh;
  extern __shared__ __align__(16) unsigned char dyn[];
  Tile<PlanT> tl;
  if (!tl.init(pl, H / HG)) return;
  const int D = H * HD;
  const int n_items = pl.q_item_off[tl.t + 1] - pl.q_item_off[tl.t];
  QS qs;
  qs.setup(pl, tl, sh, dyn, K, V, D, n_items);

  constexpr bool kDeltaFromO = sizeof(Tin) == sizeof(float);
  const Lane<HG> ln;
  const int c = ln.c;
  const int h = tl.hg * HG + ln.hl;
  const int col = ln.hl * HD + c * DPL;
  const float qscale = scale * kLog2e;
  for (int round = ln.wave; round * ITEMS < n_items; round += ln.nw) {
    const int pos = round * ITEMS + ln.slot;
    if (pos >= n_items) continue;
    const int it = sh.item[pos];
    const int r0 = item_first(it);
    const int cnt = item_count(it);
    const int rl = r0 + cnt - 1;
    const int p_last = sh.depth[rl];
    const int pm = c < cnt ? p_last - (cnt - 1 - c) : 0;
    const int64_t own = static_cast<int64_t>(tl.s) + r0 + min(c, cnt - 1);
    const float l2 = lse[own * H + h] * kLog2e;
    float q[kGroup][DPL], go[kGroup][DPL], dq[kGroup][DPL], part[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const int64_t n = static_cast<int64_t>(tl.s) + r0 + min(j ^ c, cnt - 1);
      load_vec<DPL>(Q + n * D + h * HD + c * DPL, q[j]);
      load_vec<DPL>(dO + n * D + h * HD + c * DPL, go[j]);
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        q[j][i] *= qscale;
        dq[j][i] = 0.0f;
      }
      if constexpr (kDeltaFromO) {
        float o[DPL];
        load_vec<DPL>(O + n * D + h * HD + c * DPL, o);
        part[j] = dot<DPL>(o, go[j]);
      }
    }
    float dl = 0.0f;
    if constexpr (kDeltaFromO) {
      dl = quad_reduce(part);
    } else {
      for (int d = p_last - 1; d >= 0; --d) {
        const int sl = qs.anc[d * qs.ldr + rl];
        float kk[DPL], vv[DPL], pt[kGroup];
        load_vec<DPL>(qs.Ks + sl * W + col, kk);
        load_vec<DPL>(qs.Vs + sl * W + col, vv);
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
          part[j] = dot<DPL>(q[j], kk);
          pt[j] = dot<DPL>(go[j], vv);
        }
        const float sc = quad_reduce(part);
        const float tv = quad_reduce(pt);
        const float w = d < pm ? fast_exp2(sc - l2) : 0.0f;
        dl += w * tv;
      }
    }
    for (int d = p_last - 1; d >= 0; --d) {
      const int sl = qs.anc[d * qs.ldr + rl];
      float kk[DPL], vv[DPL], pt[kGroup];
      load_vec<DPL>(qs.Ks + sl * W + col, kk);
      load_vec<DPL>(qs.Vs + sl * W + col, vv);
#pragma unroll
      for (int j = 0; j < kGroup; ++j) {
        part[j] = dot<DPL>(q[j], kk);
        pt[j] = dot<DPL>(go[j], vv);
      }
      const float sc = quad_reduce(part);
      const float tv = quad_reduce(pt);
      const float w = d < pm ? fast_exp2(sc - l2) : 0.0f;
      const float ds = w * (tv - dl) * scale;
      float dsj[kGroup];
      quad_bcast(ds, dsj);
#pragma unroll
      for (int j = 0; j < kGroup; ++j)
#pragma unroll
        for (int i = 0; i < DPL; ++i) dq[j][i] += dsj[j] * kk[i];
    }
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const int mem = j ^ c;
      if (mem < cnt) {
        const int64_t n = static_cast<int64_t>(tl.s) + r0 + mem;
        if (rope.cos_t)
          rope_inverse_part<DPL, HD>(dq[j], rope.cos_t, rope.sin_t,
                                     rope_pos(p_last - (cnt - 1 - mem), rope.seq_len), c * DPL);
        store_vec<DPL>(dQ + n * D + h * HD + c * DPL, dq[j]);
      }
    }
    if (c < cnt) Dl[own * H + h] = dl;
  }
}

// ---------------------------------------------------------------------------
// Backward, key side: dK / dV of the tile's key set. Prefix keys leave their
// partial over this tile in Pk/Pv (row pref_off[t] + depth-1); tile rows
// whose subtree ends inside the tile are finished here (seed, inverse RoPE);
// open tile rows leave their partial in dK/dV for the reduction kernels.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, typename PlanT, typename RopeT>
__global__ __launch_bounds__(256) void bwd_kv_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const float* __restrict__ lse, const float* __restrict__ Dl, const Tin* __restrict__ dO,
    float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ Pk, float* __restrict__ Pv,
    const float* __restrict__ acc_dk, const float* __restrict__ acc_dv, RopeT rope, int H,
    float scale) {
  constexpr int DPL = HD / kGroup;
  constexpr int ITEMS = 64 / (kGroup * HG);
  constexpr int W = HG * HD;
  __shared__ Tables sh;
  __shared__ float ql2[kMaxTile * HG];
  __shared__ float qdl[kMaxTile * HG];
  extern __shared__ __align__(16) unsigned char dyn[];
  Tile<PlanT> tl;
  if (!tl.init(pl, H / HG)) return;
  const int ntile = tl.ntile, A = tl.A;
  const int D = H * HD;
  const int n_items = pl.k_item_off[tl.t + 1] - pl.k_item_off[tl.t];
  Tin* Qs = reinterpret_cast<Tin*>(dyn);
  Tin* Gs = Qs + pl.tile * W;
  load_tables(pl, tl, sh, pl.k_items + pl.k_item_off[tl.t], n_items);
  stage_rows(Qs, Q, D, tl.hg * W, W, ntile, sh.prefix, 0, tl.s);
  stage_rows(Gs, dO, D, tl.hg * W, W, ntile, sh.prefix, 0, tl.s);
  for (int i = threadIdx.x; i < ntile * HG; i += blockDim.x) {
    const int r = i / HG;
    const int h = tl.hg * HG + (i - r * HG);
    ql2[i] = lse[(static_cast<int64_t>(tl.s) + r) * H + h] * kLog2e;
    qdl[i] = Dl[(static_cast<int64_t>(tl.s) + r) * H + h];
  }
  __syncthreads();

  const Lane<HG> ln;
  const int c = ln.c;
  const int h = tl.hg * HG + ln.hl;
  const int col = ln.hl * HD + c * DPL;
  const float qscale = scale * kLog2e;
  for (int round = ln.wave; round * ITEMS < n_items; round += ln.nw) {
    const int pos = round * ITEMS + ln.slot;
    if (pos >= n_items) continue;
    const int it = sh.item[pos];
    const int k0 = item_first(it);
    const int cnt = item_count(it);
    // Entry k of the key set: prefix[k] for k < A, else tile row k - A.
    auto key_row = [&](int k) -> int64_t {
      return k < A ? static_cast<int64_t>(sh.prefix[k]) : static_cast<int64_t>(tl.s) + (k - A);
    };
    float kk[kGroup][DPL], vv[kGroup][DPL], dk[kGroup][DPL], dv[kGroup][DPL];
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const int64_t a = key_row(k0 + min(j ^ c, cnt - 1));
      load_vec<DPL>(K + a * D + h * HD + c * DPL, kk[j]);
      load_vec<DPL>(V + a * D + h * HD + c * DPL, vv[j]);
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        kk[j][i] *= qscale;
        dk[j][i] = 0.0f;
        dv[j][i] = 0.0f;
      }
    }
    // Query range of member c (empty for a padding member) and of the group
    // (the first member's range contains the others').
    const int kc = k0 + c;
    int klo = 0, khi = 0;
    if (c < cnt) {
      klo = kc < A ? 0 : kc - A;
      khi = kc < A ? sh.prefix_end[kc] : sh.end[kc - A];
    }
    const int lo = k0 < A ? 0 : k0 - A;
    const int hi = k0 < A ? sh.prefix_end[k0] : sh.end[k0 - A];
    for (int j = lo; j < hi; ++j) {
      float qv[DPL], gv[DPL], ps[kGroup], pt[kGroup];
      load_vec<DPL>(Qs + j * W + col, qv);
      load_vec<DPL>(Gs + j * W + col, gv);
      const float l2 = ql2[j * HG + ln.hl];
      const float dl = qdl[j * HG + ln.hl];
#pragma unroll
      for (int b = 0; b < kGroup; ++b) {
        ps[b] = dot<DPL>(qv, kk[b]);
        pt[b] = dot<DPL>(gv, vv[b]);
      }
      const float sc = quad_reduce(ps);
      const float tv = quad_reduce(pt);
      const bool in = j >= klo && j < khi;
      const float w = in ? fast_exp2(sc - l2) : 0.0f;
      const float ds = w * (tv - dl) * scale;
      float wj[kGroup], dsj[kGroup];
      quad_bcast(w, wj);
      quad_bcast(ds, dsj);
#pragma unroll
      for (int b = 0; b < kGroup; ++b)
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          dk[b][i] += dsj[b] * qv[i];
          dv[b][i] += wj[b] * gv[i];
        }
    }
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const int mem = j ^ c;
      if (mem >= cnt) continue;
      const int ki = k0 + mem;
      if (ki < A) {
        const int64_t row = static_cast<int64_t>(tl.poff) + ki;
        store_vec<DPL>(Pk + row * D + h * HD + c * DPL, dk[j]);
        store_vec<DPL>(Pv + row * D + h * HD + c * DPL, dv[j]);
      } else {
        const int64_t a = static_cast<int64_t>(tl.s) + (ki - A);
        if (pl.end[a] <= tl.s + ntile) {  // subtree ends inside the tile: final
          if (acc_dk) {
            float x[DPL];
            load_vec<DPL>(acc_dk + a * D + h * HD + c * DPL, x);
#pragma unroll
            for (int i = 0; i < DPL; ++i) dk[j][i] += x[i];
          }
          if (acc_dv) {
            float x[DPL];
            load_vec<DPL>(acc_dv + a * D + h * HD + c * DPL, x);
#pragma unroll
            for (int i = 0; i < DPL; ++i) dv[j][i] += x[i];
          }
          if (rope.cos_t)
            rope_inverse_part<DPL, HD>(dk[j], rope.cos_t, rope.sin_t,
                                       rope_pos(sh.depth[ki - A], rope.seq_len), c * DPL);
        }
        store_vec<DPL>(dK + a * D + h * HD + c * DPL, dk[j]);
        store_vec<DPL>(dV + a * D + h * HD + c * DPL, dv[j]);
      }
    }
  }
}

inline size_t query_lds_bytes(int max_depth, int tile, int HG, int HD, int elem) {
  return static_cast<size_t>(2) * (max_depth - 1 + tile) * (HG * HD * elem) +
         static_cast<size_t>(max_depth) * tile * sizeof(int16_t);
}
inline size_t kv_lds_bytes(int tile, int HG, int HD, int elem) {
  return static_cast<size_t>(2) * tile * (HG * HD * elem);
}

}  // namespace agpt_fast
