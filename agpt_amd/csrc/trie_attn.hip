// trie_attn.hip — trie-scoped attention (forward, softmax, backward) for
// MI355X / gfx950, behind the C ABI of include/agpt_attn.h.
//
// Data layout in HBM (all row-major, rows in DFS preorder so every subtree is
// a contiguous row range):
//   Q, K, V, O, dO : [T, D] fp32 or bf16     lse : [T, H] fp32
//   dQ, dK, dV     : [T, D] fp32
//   plan tables    : parent, depth, subtree_end [T] int32;
//                    tile_pref_off [n_tiles+1], tile_prefix [Σ A_t] int32
//   workspace      : Pk, Pv [Σ A_t, D] fp32 (per-tile partial dK/dV of the
//                    tile's out-of-tile ancestors), Ck, Cv [n_chunks, maxD, D]
//
// A tile is pl.tile consecutive rows [s, e) (64, 128 or 256). Every ancestor of a row in the
// tile that lies outside the tile is an ancestor of s (preorder), so a tile
// needs only its own rows plus the A_t = depth(s)-1 "prefix" rows on the path
// of s (tile_prefix, ordered by depth). Forward and the dQ half of backward
// walk each query's path through LDS tables (in-tile parent links, then the
// prefix list). dK/dV are key-centric: key a collects over the contiguous
// query range [max(a,s), min(end(a),e)) of the tile; keys whose subtree ends
// inside their own tile are final after one kernel, the others ("open" keys)
// are finished by a fixed-order segmented reduction over the later tiles'
// prefix partials (trie_bwd_chunk_kernel + trie_bwd_reduce_kernel). No
// floating-point atomics: results are bitwise reproducible.

#include "common.h"
#include "../../include/agpt_attn.h"

#include <algorithm>
#include <numeric>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

using namespace agpt;

namespace {

thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define HIP_TRY(expr)                                                                      \
  do {                                                                                     \
    hipError_t _e = (expr);                                                                \
    if (_e != hipSuccess)                                                                  \
      return set_error(AGPT_ERR_DEVICE, "%s failed: %s", #expr, hipGetErrorString(_e));   \
  } while (0)

// Claim counters: [3][kMaxHeads] of the block kernels, then the deep query
// side's per-XCD counters (forward, dQ kernel: agpt_deep::kXcdCtr.. +16).
// Deep key side by subtree range: the longest query range (tiles) a plan
// may have for it.
constexpr int kRangeTiles = 8;
constexpr size_t kSchedBytes = (3 * kMaxHeads + 2 * 8) * sizeof(int32_t);

struct PlanDev {
  const int32_t* parent;
  const int32_t* depth;
  const int32_t* end;
  const int32_t* pref_off;  // [n_tiles + 1]
  const int32_t* prefix;    // [pref_off[n_tiles]] rows; negative: context rows before the batch
  const int32_t* pref_end;  // [pref_off[n_tiles]] subtree end (batch rows) of each prefix entry
  int64_t T;
  int32_t n_tiles;
  int32_t max_depth;
  int32_t tile;  // rows per tile (<= kMaxTileRows)
  // Fast-kernel work items per tile (agpt_fast::make_item), longest first:
  const int32_t* q_items;     // query chain groups, by walk length
  const int32_t* q_item_off;  // [n_tiles + 1]
  const int32_t* k_items;     // key-set chain groups, by query-range length
  const int32_t* k_item_off;  // [n_tiles + 1]
  // Block kernels: tile chunks claimed from counters [kernel][head group]
  // (zeroed before each launch).
  int32_t* sched;
  int32_t chunk_tiles;
  int32_t n_chunks;
  int32_t n_prefix;  // pref_off[n_tiles]
  // Deep query side: the tile of claim i is tile_order[i] (tiles of more key
  // chunks first, DFS order within), or tile i when null.
  const int32_t* tile_order;
  // Deep query side without tile_order: each XCD claims from its own
  // contiguous range of units first (neighbouring tiles share prefix rows
  // in that XCD's L2), then from the other XCDs' ranges.
  int32_t xcd_claims;
  // Deep key side by subtree range (agpt_deep::bwd_kv_range_kernel).
  const int32_t* range_bend;
  const int32_t* range_order;
  // Chain-forest plans (agpt_chain): the chains longest first, chain k of
  // that order as (first row, rows) at chain_info[2k], [2k+1].
  const int32_t* chain_info;
  int32_t n_chains;
};

// ---------------------------------------------------------------------------
// Shared tile set-up: in-tile parent links, depths, subtree ends and the
// prefix path of the tile's first row.
// ---------------------------------------------------------------------------
struct TileShared {
  int32_t parent[kMaxTileRows];
  int32_t depth[kMaxTileRows];
  int32_t end[kMaxTileRows];
  int32_t prefix[kMaxDepth];
  int32_t prefix_end[kMaxDepth];
};

__device__ __forceinline__ void load_tile(const PlanDev& pl, int t, int64_t s, int ntile, int A,
                                          TileShared& sh, bool need_ends) {
  for (int i = threadIdx.x; i < ntile; i += blockDim.x) {
    sh.parent[i] = pl.parent[s + i];
    sh.depth[i] = pl.depth[s + i];
    if (need_ends) sh.end[i] = pl.end[s + i];
  }
  const int32_t off = pl.pref_off[t];
  for (int i = threadIdx.x; i < A; i += blockDim.x) {
    const int32_t a = pl.prefix[off + i];
    sh.prefix[i] = a;
    if (need_ends) sh.prefix_end[i] = pl.pref_end[off + i];
  }
}

// ---------------------------------------------------------------------------
// Forward: o_n = Σ_j softmax(q_n·k_j·scale) v_j over n's path; lse saved.
// One workgroup per tile; item = (query row, head); online softmax in the
// log2 domain.
// ---------------------------------------------------------------------------
template <int HD, typename Tin>
__global__ __launch_bounds__(256) void trie_fwd_kernel(PlanDev pl, const Tin* __restrict__ Q,
                                                       const Tin* __restrict__ K,
                                                       const Tin* __restrict__ V,
                                                       Tin* __restrict__ O,
                                                       float* __restrict__ lse, int H,
                                                       float scale) {
  __shared__ TileShared sh;
  const int t = blockIdx.x;
  const int64_t s = static_cast<int64_t>(t) * pl.tile;
  const int ntile = static_cast<int>(min<int64_t>(pl.tile, pl.T - s));
  const int A = pl.pref_off[t + 1] - pl.pref_off[t];
  load_tile(pl, t, s, ntile, A, sh, false);
  __syncthreads();

  const int D = H * HD;
  const float qscale = scale * kLog2e;
  for (int item = threadIdx.x; item < ntile * H; item += blockDim.x) {
    const int ql = item / H;
    const int h = item - ql * H;
    const int64_t n = s + ql;
    float q[HD];
    load_vec<HD>(Q + n * D + h * HD, q);
#pragma unroll
    for (int i = 0; i < HD; ++i) q[i] *= qscale;
    float m = -INFINITY, l = 0.0f;
    float acc[HD];
#pragma unroll
    for (int i = 0; i < HD; ++i) acc[i] = 0.0f;

    auto visit = [&](int64_t a) {
      float k[HD], v[HD];
      load_vec<HD>(K + a * D + h * HD, k);
      load_vec<HD>(V + a * D + h * HD, v);
      float sc = 0.0f;
#pragma unroll
      for (int i = 0; i < HD; ++i) sc += q[i] * k[i];
      const float m_new = fmaxf(m, sc);
      const float alpha = fast_exp2(m - m_new);
      const float p = fast_exp2(sc - m_new);
      l = l * alpha + p;
#pragma unroll
      for (int i = 0; i < HD; ++i) acc[i] = acc[i] * alpha + p * v[i];
      m = m_new;
    };

    int cur = ql;
    int rem;
    for (;;) {
      visit(s + cur);
      const int32_t par = sh.parent[cur];
      if (par < s) {
        rem = sh.depth[cur] - 1;  // ancestors left, all on the prefix path
        break;
      }
      cur = static_cast<int>(par - s);
    }
    for (int d = rem - 1; d >= 0; --d) visit(sh.prefix[d]);

    const float inv = 1.0f / l;
#pragma unroll
    for (int i = 0; i < HD; ++i) acc[i] *= inv;
    store_vec<HD>(O + n * D + h * HD, acc);
    lse[n * H + h] = (m + fast_log2(l)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Backward, per tile.
//   phase 0: lse and (fp32 inputs) δ = dO·O per (query, head) into LDS
//   phase 1: (bf16 inputs: δ = Σ_j w_j dO·v_j over the path, then)
//            dQ = Σ_j ds_j k_j over each query's path (+ inverse RoPE)
//   phase 2: per key of the tile's key set (prefix rows + tile rows):
//            dK_a = Σ_n ds_{n,a} q_n, dV_a = Σ_n w_{n,a} dO_n over the
//            tile's queries in subtree(a); finished keys are written in
//            final form, open keys leave partials (own tile: in dK/dV rows;
//            prefix keys: in Pk/Pv).
// ---------------------------------------------------------------------------
struct BwdShared {
  TileShared tile;
  float lse2[kMaxTileRows * kMaxHeads];
  float delta[kMaxTileRows * kMaxHeads];
};

struct RopeArgs {
  const float* cos_t;
  const float* sin_t;
  int seq_len;
};

__device__ __forceinline__ int rope_pos(int depth, int seq_len) {
  const int p = depth - 1;
  return p < seq_len - 1 ? p : seq_len - 1;
}

template <int HD, typename Tin>
__global__ __launch_bounds__(256) void trie_bwd_kernel(
    PlanDev pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const Tin* __restrict__ O, const float* __restrict__ lse, const Tin* __restrict__ dO,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV,
    float* __restrict__ Pk, float* __restrict__ Pv, const float* __restrict__ acc_dk,
    const float* __restrict__ acc_dv, RopeArgs rope, int H, float scale) {
  __shared__ BwdShared sh;
  const int t = blockIdx.x;
  const int64_t s = static_cast<int64_t>(t) * pl.tile;
  const int ntile = static_cast<int>(min<int64_t>(pl.tile, pl.T - s));
  const int64_t e = s + ntile;
  const int32_t poff = pl.pref_off[t];
  const int A = pl.pref_off[t + 1] - poff;
  load_tile(pl, t, s, ntile, A, sh.tile, true);
  const int D = H * HD;
  const float qscale = scale * kLog2e;

  // phase 0: lse (log2 units) and, for fp32 inputs, δ = dO·O. With bf16
  // inputs O is a rounded output, so δ is recomputed in phase 1 as
  // Σ_j w_j (dO·v_j) in fp32 (batched_depth_backward.cr:637-646).
  constexpr bool kDeltaFromO = sizeof(Tin) == sizeof(float);
  for (int item = threadIdx.x; item < ntile * H; item += blockDim.x) {
    const int ql = item / H;
    const int h = item - ql * H;
    const int64_t n = s + ql;
    if constexpr (kDeltaFromO) {
      float o[HD], g[HD];
      load_vec<HD>(O + n * D + h * HD, o);
      load_vec<HD>(dO + n * D + h * HD, g);
      float d = 0.0f;
#pragma unroll
      for (int i = 0; i < HD; ++i) d += o[i] * g[i];
      sh.delta[item] = d;
    }
    sh.lse2[item] = lse[n * H + h] * kLog2e;
  }
  __syncthreads();

  // phase 1: dQ
  for (int item = threadIdx.x; item < ntile * H; item += blockDim.x) {
    const int ql = item / H;
    const int h = item - ql * H;
    const int64_t n = s + ql;
    float q[HD], g[HD], dq[HD];
    load_vec<HD>(Q + n * D + h * HD, q);
    load_vec<HD>(dO + n * D + h * HD, g);
#pragma unroll
    for (int i = 0; i < HD; ++i) {
      q[i] *= qscale;
      dq[i] = 0.0f;
    }
    const float l2 = sh.lse2[item];
    // Walks n's path: in-tile parent links, then the tile's prefix list.
    auto walk = [&](auto&& visit) {
      int cur = ql;
      int rem;
      for (;;) {
        visit(s + cur);
        const int32_t par = sh.tile.parent[cur];
        if (par < s) {
          rem = sh.tile.depth[cur] - 1;
          break;
        }
        cur = static_cast<int>(par - s);
      }
      for (int d = rem - 1; d >= 0; --d) visit(sh.tile.prefix[d]);
    };
    float dl;
    if constexpr (kDeltaFromO) {
      dl = sh.delta[item];
    } else {
      dl = 0.0f;
      walk([&](int64_t a) {
        float k[HD], v[HD];
        load_vec<HD>(K + a * D + h * HD, k);
        load_vec<HD>(V + a * D + h * HD, v);
        float sc = 0.0f, dw = 0.0f;
#pragma unroll
        for (int i = 0; i < HD; ++i) {
          sc += q[i] * k[i];
          dw += g[i] * v[i];
        }
        dl += fast_exp2(sc - l2) * dw;
      });
      sh.delta[item] = dl;
    }
    walk([&](int64_t a) {
      float k[HD], v[HD];
      load_vec<HD>(K + a * D + h * HD, k);
      load_vec<HD>(V + a * D + h * HD, v);
      float sc = 0.0f, dw = 0.0f;
#pragma unroll
      for (int i = 0; i < HD; ++i) {
        sc += q[i] * k[i];
        dw += g[i] * v[i];
      }
      const float w = fast_exp2(sc - l2);
      const float ds = w * (dw - dl) * scale;
#pragma unroll
      for (int i = 0; i < HD; ++i) dq[i] += ds * k[i];
    });
    if (rope.cos_t) rope_inverse<HD>(dq, rope.cos_t, rope.sin_t, rope_pos(sh.tile.depth[ql], rope.seq_len));
    store_vec<HD>(dQ + n * D + h * HD, dq);
  }
  if constexpr (!kDeltaFromO) __syncthreads();  // phase 2 reads every query's δ

  // phase 2: dK / dV for the key set
  const int nk = A + ntile;
  for (int item = threadIdx.x; item < nk * H; item += blockDim.x) {
    const int ki = item / H;
    const int h = item - ki * H;
    int64_t a, end_a;
    int depth_a;
    if (ki < A) {
      a = sh.tile.prefix[ki];
      end_a = sh.tile.prefix_end[ki];
      depth_a = ki + 1;
    } else {
      a = s + (ki - A);
      end_a = sh.tile.end[ki - A];
      depth_a = sh.tile.depth[ki - A];
    }
    const int64_t q_lo = a > s ? a : s;
    const int64_t q_hi = end_a < e ? end_a : e;
    float k[HD], v[HD], dk[HD], dv[HD];
    load_vec<HD>(K + a * D + h * HD, k);
    load_vec<HD>(V + a * D + h * HD, v);
#pragma unroll
    for (int i = 0; i < HD; ++i) {
      k[i] *= qscale;
      dk[i] = 0.0f;
      dv[i] = 0.0f;
    }
    for (int64_t n = q_lo; n < q_hi; ++n) {
      const int qi = static_cast<int>(n - s) * H + h;
      float q[HD], g[HD];
      load_vec<HD>(Q + n * D + h * HD, q);
      load_vec<HD>(dO + n * D + h * HD, g);
      float sc = 0.0f, dw = 0.0f;
#pragma unroll
      for (int i = 0; i < HD; ++i) {
        sc += q[i] * k[i];
        dw += g[i] * v[i];
      }
      const float w = fast_exp2(sc - sh.lse2[qi]);
      const float ds = w * (dw - sh.delta[qi]) * scale;
#pragma unroll
      for (int i = 0; i < HD; ++i) {
        dk[i] += ds * q[i];
        dv[i] += w * g[i];
      }
    }
    if (ki < A) {
      const int64_t row = static_cast<int64_t>(poff) + ki;
      store_vec<HD>(Pk + row * D + h * HD, dk);
      store_vec<HD>(Pv + row * D + h * HD, dv);
    } else if (end_a <= e) {
      if (acc_dk) {
        float x[HD];
        load_vec<HD>(acc_dk + a * D + h * HD, x);
#pragma unroll
        for (int i = 0; i < HD; ++i) dk[i] += x[i];
      }
      if (acc_dv) {
        float x[HD];
        load_vec<HD>(acc_dv + a * D + h * HD, x);
#pragma unroll
        for (int i = 0; i < HD; ++i) dv[i] += x[i];
      }
      if (rope.cos_t) rope_inverse<HD>(dk, rope.cos_t, rope.sin_t, rope_pos(depth_a, rope.seq_len));
      store_vec<HD>(dK + a * D + h * HD, dk);
      store_vec<HD>(dV + a * D + h * HD, dv);
    } else {
      store_vec<HD>(dK + a * D + h * HD, dk);
      store_vec<HD>(dV + a * D + h * HD, dv);
    }
  }
}

// ---------------------------------------------------------------------------
// Reduction level 1: chunk c (kChunkTiles consecutive tiles) sums the prefix
// partials of slot k over its tiles, for the slots every tile of the chunk
// has (k < min A). Such a sum is used only when the whole chunk lies inside
// one key's span, where slot k names the same key in every tile.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void trie_bwd_chunk_kernel(PlanDev pl, const float* __restrict__ Pk,
                                                             const float* __restrict__ Pv,
                                                             float* __restrict__ Ck,
                                                             float* __restrict__ Cv, int D) {
  const int c = blockIdx.x;
  const int u0 = c * kChunkTiles;
  const int u1 = min(pl.n_tiles, u0 + kChunkTiles);
  __shared__ int min_a;
  if (threadIdx.x == 0) {
    int m = kMaxDepth;
    for (int u = u0; u < u1; ++u) m = min(m, pl.pref_off[u + 1] - pl.pref_off[u]);
    min_a = m;
  }
  __syncthreads();
  const int total = min_a * D;
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int k = idx / D;
    const int col = idx - k * D;
    float sk = 0.0f, sv = 0.0f;
    for (int u = u0; u < u1; ++u) {
      const int64_t row = static_cast<int64_t>(pl.pref_off[u]) + k;
      sk += Pk[row * D + col];
      sv += Pv[row * D + col];
    }
    const int64_t o = (static_cast<int64_t>(c) * pl.max_depth + k) * D + col;
    Ck[o] = sk;
    Cv[o] = sv;
  }
}

// ---------------------------------------------------------------------------
// Reduction level 2: one wave per open key a of tile t (the rows of tile t on
// the prefix path of tile t+1). dK_a = own-tile partial (already in dK) +
// Σ over tiles u in (t, tile(end_a - 1)] of slot depth(a)-1, in tile order,
// using chunk sums for whole chunks. Then seeds, inverse RoPE, final write.
// ---------------------------------------------------------------------------
// VW consecutive columns per lane: one walk over the tiles covers 64 * VW
// columns (D = 512 in one walk with VW = 8, 16-byte loads).
template <int VW>
__device__ __forceinline__ void ld_cols(const float* __restrict__ p, float (&x)[VW]) {
  if constexpr (VW == 2) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    x[0] = v.x;
    x[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < VW; i += 4) {
      const float4 v = *reinterpret_cast<const float4*>(p + i);
      x[i] = v.x;
      x[i + 1] = v.y;
      x[i + 2] = v.z;
      x[i + 3] = v.w;
    }
  }
}
template <int VW>
__device__ __forceinline__ void st_cols(float* __restrict__ p, const float (&x)[VW]) {
  if constexpr (VW == 2) {
    *reinterpret_cast<float2*>(p) = float2{x[0], x[1]};
  } else {
#pragma unroll
    for (int i = 0; i < VW; i += 4) *reinterpret_cast<float4*>(p + i) = float4{x[i], x[i + 1], x[i + 2], x[i + 3]};
  }
}
template <int VW>
__device__ __forceinline__ void add_cols(float (&x)[VW], const float* __restrict__ p) {
  float y[VW];
  ld_cols<VW>(p, y);
#pragma unroll
  for (int i = 0; i < VW; ++i) x[i] += y[i];
}

template <int HD, int VW>
__global__ __launch_bounds__(256) void trie_bwd_reduce_kernel(
    PlanDev pl, float* __restrict__ dK, float* __restrict__ dV, const float* __restrict__ Pk,
    const float* __restrict__ Pv, const float* __restrict__ Ck, const float* __restrict__ Cv,
    const float* __restrict__ acc_dk, const float* __restrict__ acc_dv, RopeArgs rope, int H) {
  const int t = blockIdx.x;  // tiles 0 .. n_tiles-2
  const int64_t s = static_cast<int64_t>(t) * pl.tile;
  const int32_t noff = pl.pref_off[t + 1];
  const int An = pl.pref_off[t + 2] - noff;
  const int D = H * HD;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  for (int k = An - 1 - wave; k >= 0; k -= nwaves) {
    const int64_t a = pl.prefix[noff + k];
    if (a < s) break;  // deeper-first scan: everything above is outside tile t
    const int u_last = static_cast<int>((pl.end[a] - 1) / pl.tile);
    const int pos = rope.cos_t ? rope_pos(k + 1, rope.seq_len) : 0;
    for (int col0 = lane * VW; col0 < D; col0 += 64 * VW) {
      float sk[VW], sv[VW];
      ld_cols<VW>(dK + a * D + col0, sk);
      ld_cols<VW>(dV + a * D + col0, sv);
      // The parts in tile order (a chunk sum for each whole chunk, else the
      // tile's partial), kR rows of each tensor in flight at a time.
      constexpr int kR = 4;
      int u = t + 1;
      while (u <= u_last) {
        const float* srck[kR];
        const float* srcv[kR];
        int n = 0;
        for (; n < kR && u <= u_last; ++n) {
          const int c = u / kChunkTiles;
          if (u == c * kChunkTiles && u + kChunkTiles - 1 <= u_last) {
            const int64_t o = (static_cast<int64_t>(c) * pl.max_depth + k) * D + col0;
            srck[n] = Ck + o;
            srcv[n] = Cv + o;
            u += kChunkTiles;
          } else {
            const int64_t o = (static_cast<int64_t>(pl.pref_off[u]) + k) * D + col0;
            srck[n] = Pk + o;
            srcv[n] = Pv + o;
            ++u;
          }
        }
        float yk[kR][VW], yv[kR][VW];
#pragma unroll
        for (int x = 0; x < kR; ++x)
          if (x < n) {
            ld_cols<VW>(srck[x], yk[x]);
            ld_cols<VW>(srcv[x], yv[x]);
          }
#pragma unroll
        for (int x = 0; x < kR; ++x)
          if (x < n)
#pragma unroll
            for (int i = 0; i < VW; ++i) {
              sk[i] += yk[x][i];
              sv[i] += yv[x][i];
            }
      }
      if (acc_dk) add_cols<VW>(sk, acc_dk + a * D + col0);
      if (acc_dv) add_cols<VW>(sv, acc_dv + a * D + col0);
      if (rope.cos_t) {
#pragma unroll
        for (int p = 0; p < VW; p += 2) {
          const int j = (col0 + p) % HD;  // even: pair (j, j+1) of the head
          const float c = rope.cos_t[pos * HD + j];
          const float sn = rope.sin_t[pos * HD + j];
          const float x0 = sk[p], x1 = sk[p + 1];
          sk[p] = x0 * c + x1 * sn;
          sk[p + 1] = -x0 * sn + x1 * c;
        }
      }
      st_cols<VW>(dK + a * D + col0, sk);
      st_cols<VW>(dV + a * D + col0, sv);
    }
  }
}

// ---------------------------------------------------------------------------
// Context rows of a range plan (agpt_attn_plan_range): the ancestors of the
// batch's row 0 that lie before the batch are prefix entries d = 0 ..
// n_ctx-1 of tile 0, read as keys by every tile in their subtree. Their
// share of dK/dV over the batch's queries sits in the backward's partials:
// entry d of every tile inside the key's subtree (Pk/Pv, tile by tile) or,
// with the path carry, of every chunk inside it (E: [chunk][P][2][D]). One
// workgroup per (key, 4 columns of dK or of dV): each thread sums a strided
// subset of the parts in order, then a fixed-order tree in LDS (no
// atomics: reruns give the same bytes); inverse RoPE at the key's depth;
// the result is added into the key's row (its owner batch wrote it) or
// written there (a packed batch).
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256) void trie_ctx_kernel(PlanDev pl, const float* __restrict__ Pk,
                                                       const float* __restrict__ Pv, int from_chunks, int P,
                                                       int rows_per_part, int n_parts, float* __restrict__ dK,
                                                       float* __restrict__ dV, RopeArgs rope, int H, int add) {
  const int d = blockIdx.y;
  const int D = H * HD;
  const int tv = static_cast<int>(blockIdx.x) / (D / 4);  // 0: dK, 1: dV
  const int col = (static_cast<int>(blockIdx.x) - tv * (D / 4)) * 4;
  const int64_t a = pl.prefix[d];
  const int64_t ea = pl.pref_end[d];
  const int np = static_cast<int>(min(static_cast<int64_t>(n_parts), (ea + rows_per_part - 1) / rows_per_part));
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int p = threadIdx.x; p < np; p += blockDim.x) {
    const float* src = from_chunks
                           ? Pk + ((static_cast<int64_t>(p) * P + d) * 2 + tv) * D + col
                           : (tv ? Pv : Pk) + (static_cast<int64_t>(pl.pref_off[p]) + d) * D + col;
    float y[4];
    load_vec<4>(src, y);
#pragma unroll
    for (int x = 0; x < 4; ++x) v[x] += y[x];
  }
  __shared__ float red[256][4];
#pragma unroll
  for (int x = 0; x < 4; ++x) red[threadIdx.x][x] = v[x];
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (static_cast<int>(threadIdx.x) < s)
#pragma unroll
      for (int x = 0; x < 4; ++x) red[threadIdx.x][x] += red[threadIdx.x + s][x];
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
#pragma unroll
  for (int x = 0; x < 4; ++x) v[x] = red[0][x];
  if (tv == 0 && rope.cos_t) {
    const int pos = rope_pos(d + 1, rope.seq_len);
#pragma unroll
    for (int p = 0; p < 4; p += 2) {
      const int j = (col + p) % HD;  // even: pair (j, j+1) of the head
      const float c = rope.cos_t[pos * HD + j];
      const float sn = rope.sin_t[pos * HD + j];
      const float x0 = v[p], x1 = v[p + 1];
      v[p] = x0 * c + x1 * sn;
      v[p + 1] = -x0 * sn + x1 * c;
    }
  }
  float* out = (tv ? dV : dK) + a * D + col;
  if (add) {
    float y[4];
    load_vec<4>(out, y);
#pragma unroll
    for (int x = 0; x < 4; ++x) v[x] += y[x];
  }
  store_vec<4>(out, v);
}

}  // namespace

#include "trie_fast.h"
#include "trie_block.h"
#include "trie_deep.h"
#include "trie_chain.h"

// ===========================================================================
// Host side: handle, plan, launches.
// ===========================================================================
struct agpt_attn_s {
  agpt_attn_config cfg{};
  int device = 0;
  // plan (host copies used for launch geometry)
  int64_t T = 0;
  int32_t tile = 0;
  int32_t n_tiles = 0;
  int32_t n_chunks = 0;
  int32_t max_depth = 0;
  int64_t sum_depth = 0;
  int64_t n_prefix_rows = 0;
  bool planned = false;
  // device tables
  int32_t* d_parent = nullptr;
  int32_t* d_depth = nullptr;
  int32_t* d_end = nullptr;
  int32_t* d_pref_off = nullptr;
  int32_t* d_prefix = nullptr;
  int32_t* d_pref_end = nullptr;
  // batch placement (agpt_attn_plan_range): the caller's tensors hold the
  // batch's row 0 at row row_off; n_ctx context rows (ancestors of row 0
  // before the batch) are keys only; ctx_add: their share of dK/dV is added
  // into their rows (else written)
  int64_t row_off = 0;
  int32_t n_ctx = 0;
  bool ctx_add = true;
  // workspace: prefix partials, chunk sums, δ
  float* d_Pk = nullptr;
  float* d_Pv = nullptr;
  float* d_Ck = nullptr;
  float* d_Cv = nullptr;
  float* d_Dl = nullptr;
  int32_t* d_sched = nullptr;  // [3][kMaxHeads] chunk counters of the block kernels
  int32_t chunk_tiles = 1, n_chunks_sched = 1;
  int32_t* d_q_items = nullptr;
  int32_t* d_k_items = nullptr;
  int32_t* d_q_item_off = nullptr;
  int32_t* d_k_item_off = nullptr;
  int32_t* d_tile_order = nullptr;  // deep query side: claim order of the tiles (null: tile order)
  int32_t* d_range_bend = nullptr;  // deep key side by subtree range: [n_tiles][4] block range ends
  int32_t* d_range_order = nullptr; // and the tiles by descending range
  int32_t* d_chain_info = nullptr;  // chain-forest plans: (first row, rows) of the chains, longest first
  int32_t n_chains = 0;
  // kernel family chosen at plan time: 0 = global-memory walk (any shape),
  // 5 = streaming chain-group walk (trie_fast.h), 6 = streaming block-sparse
  // 16x16 matrix tiles (trie_block.h)
  int variant = 0;
  int hg = 1, nw = 2, qb = 1, kb = 1;
  bool unit_all_heads = false;  // split block backward: a unit takes every head of the group
  int fwd_uh = 2;               // block forward: heads per unit (at most the group)
  bool fused = false;           // block kernels: one-pass backward (fp32)
  int fhg = 1;                  // heads per workgroup of the one-pass backward
  bool carry = false;           // one-pass backward carries path sums (E, F replace Pk, Pv)
  bool deep = false;            // block kernels at head_dim 64: streamed key set (trie_deep.h)
  bool deep_carry = false;      // deep key side carries path sums (E, F replace Pk, Pv)
  bool dq_one_pass = true;      // deep bf16 dQ kernel: δ and dQ in one pass over the keys
  bool xcd_claims = true;       // deep query side in tile order: claims by XCD ranges
  bool deep_range = false;      // deep key side over each tile's subtree range (short subtrees)
  bool chain_plan = false;      // bf16 head_dim 64 on a forest of chains: the agpt_chain kernels
  bool chain_fused = true;      // chain plans: the backward in one launch (AGPT_ATTN_CHAINFUSE=0: two)
  float* d_Cs = nullptr;        // deep carry: per-workgroup carry rows [slot][2][P][2][head_dim]
  int cs_slots = 0;             // workgroups the carry rows are sized for
  float* d_E = nullptr;         // carry: per-chunk partials [n_chunks][P][2][D]
  float* d_F = nullptr;
  size_t fb_lds = 0;
  bool split = true;  // cut long work items into parts (see agpt_fast::kCutSteps)
  int q_slots = 0, k_slots = 0;  // scratch slots of cut query / key items per tile
  size_t fwd_lds = 0, bq_lds = 0, kv_lds = 0, kv_range_lds = 0;
  int max_lds = 65536;
  std::string desc;
  // plan placed in the library's static scratch (agpt_attn_plan_static):
  // nothing to free; valid while static_gen is the device's latest
  bool static_plan = false;
  uint64_t static_gen = 0;
};

namespace {

void free_plan(agpt_attn_s* h) {
  // A static plan's buffers live in the library's scratch array: they are
  // dropped, not freed.
  const bool own = !h->static_plan;
  int32_t** ip[] = {&h->d_parent,   &h->d_depth,       &h->d_end,         &h->d_pref_off,
                    &h->d_prefix,   &h->d_pref_end,    &h->d_q_item_off,  &h->d_k_item_off,
                    &h->d_tile_order, &h->d_range_bend, &h->d_range_order, &h->d_chain_info};
  for (auto p : ip)
    if (*p) {
      if (own) (void)hipFree(*p);
      *p = nullptr;
    }
  float** fp[] = {&h->d_Pk, &h->d_Pv, &h->d_Ck, &h->d_Cv, &h->d_Dl, &h->d_E, &h->d_F, &h->d_Cs};
  for (auto p : fp)
    if (*p) {
      if (own) (void)hipFree(*p);
      *p = nullptr;
    }
  int32_t** op[] = {&h->d_q_items, &h->d_k_items, &h->d_sched};
  for (auto p : op)
    if (*p) {
      if (own) (void)hipFree(*p);
      *p = nullptr;
    }
  h->planned = false;
  h->static_plan = false;
}

// ---- static scratch (agpt_attn_plan_static) ---------------------------------
// A plan's device tables and workspace, for callers that cannot allocate,
// live in this file-scope array: one copy per device, held until the process
// ends. Host code never uses the array's name as an address: each device's
// copy is looked up once with hipGetSymbolAddress (that device current) and
// its address kept in g_scratch_ptr.
constexpr size_t kScratchBytes = AGPT_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxDevices] = {};
uint64_t g_scratch_gen[kMaxDevices] = {};  // the device's latest static plan

// Device address of the current device's scratch (looked up on first use).
int scratch_base(int dev, unsigned char** out) {
  if (dev < 0 || dev >= kMaxDevices) return set_error(AGPT_ERR_DEVICE, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = static_cast<unsigned char*>(p);
  }
  *out = g_scratch_ptr[dev];
  return AGPT_OK;
}

bool static_plan_current(const agpt_attn_s* h) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return h->static_gen == g_scratch_gen[h->device];
}

// Device buffers of a plan: hipMalloc, or 256-byte aligned slices of the
// static scratch. Past the scratch's end it keeps counting (no address is
// handed out) so the caller can report the bytes the batch needs.
struct Arena {
  unsigned char* base = nullptr;  // null: hipMalloc
  size_t used = 0;
  bool overflow = false;
  int get(void** p, size_t bytes) {
    bytes = std::max<size_t>(bytes, 16);
    if (!base) {
      HIP_TRY(hipMalloc(p, bytes));
      return AGPT_OK;
    }
    const size_t off = (used + 255) & ~static_cast<size_t>(255);
    used = off + bytes;
    if (used > kScratchBytes) overflow = true;
    *p = overflow ? nullptr : base + off;
    return AGPT_OK;
  }
};

bool head_dim_supported(int hd) { return hd == 4 || hd == 8 || hd == 16 || hd == 32 || hd == 64; }

PlanDev plan_dev(const agpt_attn_s* h) {
  PlanDev p;
  p.parent = h->d_parent;
  p.depth = h->d_depth;
  p.end = h->d_end;
  p.pref_off = h->d_pref_off;
  p.prefix = h->d_prefix;
  p.pref_end = h->d_pref_end;
  p.T = h->T;
  p.n_tiles = h->n_tiles;
  p.max_depth = h->max_depth;
  p.tile = h->tile;
  p.q_items = h->d_q_items;
  p.q_item_off = h->d_q_item_off;
  p.k_items = h->d_k_items;
  p.k_item_off = h->d_k_item_off;
  p.sched = h->d_sched;
  p.chunk_tiles = h->chunk_tiles;
  p.n_chunks = h->n_chunks_sched;
  p.n_prefix = static_cast<int32_t>(h->n_prefix_rows);
  p.tile_order = h->d_tile_order;
  p.xcd_claims = h->xcd_claims && !h->d_tile_order ? 1 : 0;
  p.range_bend = h->d_range_bend;
  p.range_order = h->d_range_order;
  p.chain_info = h->d_chain_info;
  p.n_chains = h->n_chains;
  return p;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return (v && *v) ? std::atoi(v) : dflt;
}

}  // namespace

int agpt_internal_set_error(int code, const char* msg) { return set_error(code, "%s", msg); }

extern "C" const char* agpt_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* agpt_version(void) {
  return "agpt_attn gfx950: wave-per-tile LDS-staged cost-balanced trie attention (fp32/bf16, hd 4..64)";
}

extern "C" int agpt_attn_check_tree(const int32_t* parent, int64_t n, int32_t* depth,
                                    int32_t* subtree_end) {
  if (n < 0 || (n > 0 && !parent)) return set_error(AGPT_ERR_INVALID_ARG, "null parent table");
  if (n >= (int64_t{1} << 31) - kMaxTileRows)
    return set_error(AGPT_ERR_INVALID_ARG, "n_nodes %lld exceeds int32 row indexing", (long long)n);
  std::vector<int32_t> dep(static_cast<size_t>(n)), en(static_cast<size_t>(n));
  // Preorder check with a stack of open subtrees: the parent of row i must be
  // the node on top of the stack after popping every subtree that i cannot
  // belong to; that makes every subtree a contiguous row range.
  std::vector<int32_t> stack;
  stack.reserve(kMaxDepth);
  for (int64_t i = 0; i < n; ++i) {
    const int32_t p = parent[i];
    if (p < -1 || p >= i)
      return set_error(AGPT_ERR_NOT_DFS, "parent[%lld] = %d is not an earlier row or -1",
                       (long long)i, p);
    while (!stack.empty() && stack.back() != p) {
      en[stack.back()] = static_cast<int32_t>(i);
      stack.pop_back();
    }
    if (p >= 0 && stack.empty())
      return set_error(AGPT_ERR_NOT_DFS,
                       "row %lld follows a closed subtree of its parent %d: not DFS preorder",
                       (long long)i, p);
    dep[i] = p < 0 ? 1 : dep[p] + 1;
    stack.push_back(static_cast<int32_t>(i));
  }
  while (!stack.empty()) {
    en[stack.back()] = static_cast<int32_t>(n);
    stack.pop_back();
  }
  if (depth) std::memcpy(depth, dep.data(), sizeof(int32_t) * n);
  if (subtree_end) std::memcpy(subtree_end, en.data(), sizeof(int32_t) * n);
  g_last_error.clear();
  return AGPT_OK;
}

extern "C" int agpt_attn_dfs_order(const int32_t* parent, int64_t n, int32_t* perm) {
  if (n < 0 || (n > 0 && (!parent || !perm))) return set_error(AGPT_ERR_INVALID_ARG, "null argument");
  std::vector<int64_t> cnt(static_cast<size_t>(n) + 1, 0);
  int64_t n_roots = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int32_t p = parent[i];
    if (p < -1 || p >= n || p == i) return set_error(AGPT_ERR_INVALID_ARG, "bad parent[%lld]=%d", (long long)i, p);
    if (p >= 0) cnt[p + 1]++;
    else n_roots++;
  }
  // CSR children lists, children in original order
  std::vector<int64_t> off(static_cast<size_t>(n) + 1, 0);
  for (int64_t i = 0; i < n; ++i) off[i + 1] = off[i] + cnt[i + 1];
  std::vector<int32_t> kids(static_cast<size_t>(off[n]));
  std::vector<int64_t> fill(off.begin(), off.end() - 1);
  std::vector<int32_t> roots;
  roots.reserve(static_cast<size_t>(n_roots));
  for (int64_t i = 0; i < n; ++i) {
    if (parent[i] >= 0) kids[fill[parent[i]]++] = static_cast<int32_t>(i);
    else roots.push_back(static_cast<int32_t>(i));
  }
  int64_t k = 0;
  std::vector<int32_t> stack;
  for (auto it = roots.rbegin(); it != roots.rend(); ++it) stack.push_back(*it);
  while (!stack.empty()) {
    const int32_t v = stack.back();
    stack.pop_back();
    if (k >= n) return set_error(AGPT_ERR_INVALID_ARG, "parent table has a cycle");
    perm[k++] = v;
    for (int64_t j = off[v + 1] - 1; j >= off[v]; --j) stack.push_back(kids[j]);
  }
  if (k != n) return set_error(AGPT_ERR_INVALID_ARG, "parent table has a cycle");
  return AGPT_OK;
}

extern "C" int agpt_attn_create(const agpt_attn_config* cfg, agpt_attn_handle* out) {
  if (!cfg || !out) return set_error(AGPT_ERR_INVALID_ARG, "null argument");
  *out = nullptr;
  if (cfg->n_heads < 1 || cfg->n_heads > kMaxHeads)
    return set_error(AGPT_ERR_UNSUPPORTED, "n_heads %d outside 1..%d", cfg->n_heads, kMaxHeads);
  if (!head_dim_supported(cfg->head_dim))
    return set_error(AGPT_ERR_UNSUPPORTED, "head_dim %d not built (4, 8, 16, 32, 64)", cfg->head_dim);
  if (cfg->max_depth < 1 || cfg->max_depth > kMaxDepth)
    return set_error(AGPT_ERR_UNSUPPORTED, "max_depth %d outside 1..%d", cfg->max_depth, kMaxDepth);
  if (cfg->dtype != AGPT_DTYPE_F32 && cfg->dtype != AGPT_DTYPE_BF16)
    return set_error(AGPT_ERR_UNSUPPORTED, "dtype %d", cfg->dtype);
  auto* h = new agpt_attn_s();
  h->cfg = *cfg;
  if (hipGetDevice(&h->device) != hipSuccess) {
    delete h;
    return set_error(AGPT_ERR_DEVICE, "no HIP device");
  }
  *out = h;
  return AGPT_OK;
}

extern "C" int agpt_attn_destroy(agpt_attn_handle h) {
  if (!h) return AGPT_OK;
  free_plan(h);
  delete h;
  return AGPT_OK;
}

namespace {

// Picks the kernel family and its shape for the planned batch: the
// streaming kernels (trie_fast.h, 64-row tiles) when the head slice fits
// whole 16-byte chunks, the head dim is 16 or 32 (four lane slices of 4 or 8
// elements; the per-lane registers stay in budget), and the tile context fits
// the workgroup LDS; otherwise the global-memory walk.
// Heads per workgroup are chosen so that one row slice is a 128-byte line;
// chain groups hold up to QB queries / KB keys (at most four).
// AGPT_ATTN_VARIANT / _HG / _TILE / _QB / _KB override (tuning).
void fit_scratch(agpt_attn_s* h);

void choose_variant(agpt_attn_s* h, int& tile) {
  const int hd = h->cfg.head_dim, H = h->cfg.n_heads;
  const int elem = h->cfg.dtype == AGPT_DTYPE_F32 ? 4 : 2;
  int lim = 65536;
  (void)hipDeviceGetAttribute(&lim, hipDeviceAttributeMaxSharedMemoryPerBlock, h->device);
  h->max_lds = lim;
  const int budget = lim - static_cast<int>(sizeof(agpt_fast::StreamTables<4>));
  {
    const int v = env_int("AGPT_ATTN_VARIANT", 6);
    h->variant = (v == 5 || v == 6) ? v : 0;
    h->fused = h->carry = false;
  }
  if (h->variant == 6) {
    int hg = env_int("AGPT_ATTN_HG", 0);
    if (hg == 0) {
      hg = 1;
      while (hg * 2 <= 4 && H % (hg * 2) == 0 && hg * 2 * hd * elem <= 128) hg *= 2;
    }
    h->hg = hg;
    h->unit_all_heads = env_int("AGPT_ATTN_UH", 1) != 1;
    // Forward units of two heads: two independent chains of matrix steps
    // and softmax work per wave, on one mask.
    h->fwd_uh = std::max(1, env_int("AGPT_ATTN_FUH", 2));
    tile = agpt_blk::kTile;
    h->fwd_lds = agpt_blk::block_lds_bytes(h->max_depth, hg, hd, elem, 1, false);
    h->bq_lds = agpt_blk::block_lds_bytes(h->max_depth, hg, hd, elem, 2, elem == 4);
    h->kv_lds = agpt_blk::block_lds_bytes(h->max_depth, hg, hd, elem, 2, false);
    // One-pass backward: the fewest heads per workgroup whose row segment
    // fills a 128-byte line (a half-used line is fetched whole, and its
    // other half by another workgroup, often on another XCD's L2).
    int fhg = env_int("AGPT_ATTN_FHG", 0);
    if (fhg == 0) {
      fhg = 1;
      while (fhg * 2 <= 2 && H % (fhg * 2) == 0 && fhg * hd * elem < 128) fhg *= 2;
    }
    h->fhg = fhg;
    h->fused = elem == 4 && hd <= 32 && env_int("AGPT_ATTN_FUSED", 1) != 0 && H % h->fhg == 0 &&
               (h->fhg == 1 || h->fhg == 2);
    h->fb_lds = agpt_blk::fused_lds_bytes(h->max_depth, h->fhg, hd, false);
    const int bbudget = lim - static_cast<int>(sizeof(agpt_blk::BlockTables<4>));
    // head_dim 64 runs one head per workgroup (a 256-byte fp32 / 128-byte
    // bf16 row segment already fills whole lines), its key set streamed
    // through a ring (trie_deep.h) instead of held whole in LDS.
    h->deep = hd == 64 && hg == 1 && env_int("AGPT_ATTN_DEEP", 1) != 0;
    h->dq_one_pass = env_int("AGPT_ATTN_DQ1", 1) != 0;
    h->xcd_claims = env_int("AGPT_ATTN_XCD", 1) != 0;
    h->deep_carry = h->deep && env_int("AGPT_ATTN_CARRY", 1) != 0;
    if (h->deep) {
      h->fwd_lds = agpt_deep::ring_lds_bytes(hd, elem);
      h->bq_lds = agpt_deep::ring_lds_bytes(hd, elem);
      // the key side's staged rows, and the carry kernel's prefetched table
      // inputs of the next tile
      h->kv_lds = agpt_deep::rows_lds_bytes(hd, elem) + agpt_deep::RawTabs::kBytes;
      h->kv_range_lds = agpt_deep::rows_lds_bytes(hd, elem);  // the staged query rows
    }
    const bool ok = (hd == 16 || hd == 32 || (hd == 64 && hg == 1)) && H % hg == 0 &&
                    (hg == 1 || hg == 2 || hg == 4) &&
                    (hg * hd * elem) % 16 == 0 && h->fwd_lds <= static_cast<size_t>(bbudget) &&
                    h->bq_lds <= static_cast<size_t>(bbudget) && h->kv_lds <= static_cast<size_t>(bbudget);
    if (h->fused && h->fb_lds > static_cast<size_t>(bbudget)) h->fused = false;
    // Path carry (head_dim 16: its dQ registers fit) when its LDS keeps the
    // workgroups per CU (registers hold the one-pass backward to two).
    {
      const size_t tabs = sizeof(agpt_blk::BlockTables<2>);
      auto per_cu = [&](size_t b) { return static_cast<size_t>(lim) / ((b + tabs + 511) & ~static_cast<size_t>(511)); };
      const size_t with = agpt_blk::fused_lds_bytes(h->max_depth, h->fhg, hd, true);
      h->carry = h->fused && hd == 16 && env_int("AGPT_ATTN_CARRY", 1) != 0 &&
                 per_cu(with) >= std::min<size_t>(per_cu(h->fb_lds), 2) && per_cu(with) >= 1;
      if (h->carry) h->fb_lds = with;
    }
    if (ok) return;
    h->variant = 5;  // try the chain-group walk
    h->fused = h->carry = h->deep = h->deep_carry = false;
  }
  if (h->variant != 5) {
    const int t = env_int("AGPT_ATTN_TILE", 64);
    tile = (t == 64 || t == 128 || t == 256) ? t : 64;
    return;
  }
  int hg = env_int("AGPT_ATTN_HG", 0);
  if (hg == 0) {
    hg = 1;
    while (hg * 2 <= 4 && H % (hg * 2) == 0 && hg * 2 * hd * elem <= 128) hg *= 2;
  }
  h->hg = hg;
  h->qb = env_int("AGPT_ATTN_QB", agpt_fast::kGroup);
  h->kb = env_int("AGPT_ATTN_KB", agpt_fast::kGroup);
  h->split = env_int("AGPT_ATTN_SPLIT", 1) != 0;
  tile = agpt_fast::kTile;
  h->fwd_lds = agpt_fast::stream_lds_bytes(h->max_depth, hg, hd, elem, 1, false, true);
  h->bq_lds = agpt_fast::stream_lds_bytes(h->max_depth, hg, hd, elem, 2, elem == 4, true);
  h->kv_lds = agpt_fast::stream_lds_bytes(h->max_depth, hg, hd, elem, 2, false, false);
  h->q_slots = h->k_slots = 0;
  const bool ok = hd >= 16 && hd <= 32 && H % hg == 0 && (hg == 1 || hg == 2 || hg == 4) &&
                  h->qb >= 1 && h->qb <= agpt_fast::kGroup && h->kb >= 1 && h->kb <= agpt_fast::kGroup &&
                  (hg * hd * elem) % 16 == 0 && h->fwd_lds <= static_cast<size_t>(budget) &&
                  h->bq_lds <= static_cast<size_t>(budget) && h->kv_lds <= static_cast<size_t>(budget);
  if (!ok) {
    h->variant = 0;
    tile = 64;
    return;
  }
  if (h->split) fit_scratch(h);
}

template <typename T>
int upload(Arena& ar, T** dst, const std::vector<T>& src) {
  const size_t bytes = std::max<size_t>(src.size(), 1) * sizeof(T);
  int rc = ar.get(reinterpret_cast<void**>(dst), bytes);
  if (rc != AGPT_OK) return rc;
  if (*dst && !src.empty()) HIP_TRY(hipMemcpy(*dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice));
  return AGPT_OK;
}

// Plans the batch rows A0 .. n_ext-1 of an extended parent table whose first
// A0 rows are the batch's context: the ancestors of its first row that lie
// before the batch (a chain, root first). ctx_local[j] is the row of context
// row j in the caller's tensors, relative to the batch's row 0 (negative).
// The device tables cover the batch rows only; prefix entries name rows in
// that relative numbering, so a context row is an ordinary prefix key.
int plan_impl(agpt_attn_s* h, const int32_t* ext, int64_t n_ext, int32_t A0,
              const std::vector<int32_t>& ctx_local, Arena& ar) {
  free_plan(h);
  std::vector<int32_t> dext(static_cast<size_t>(n_ext)), eext(static_cast<size_t>(n_ext));
  int rc = agpt_attn_check_tree(ext, n_ext, dext.data(), eext.data());
  if (rc != AGPT_OK) return rc;
  const int64_t n = n_ext - A0;
  auto loc = [&](int32_t x) -> int32_t { return x < 0 ? -1 : x < A0 ? ctx_local[x] : x - A0; };
  std::vector<int32_t> parent(static_cast<size_t>(n)), depth(static_cast<size_t>(n)), end(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) {
    parent[i] = loc(ext[A0 + i]);
    depth[i] = dext[A0 + i];
    end[i] = static_cast<int32_t>(eext[A0 + i] - A0);
  }
  int32_t maxd = 1;
  int64_t sumd = 0;
  for (int64_t i = 0; i < n; ++i) {
    maxd = std::max(maxd, depth[i]);
    sumd += depth[i];
  }
  if (maxd > h->cfg.max_depth)
    return set_error(AGPT_ERR_TOO_DEEP, "tree depth %d exceeds config max_depth %d", maxd, h->cfg.max_depth);
  h->max_depth = maxd;
  int tile = 64;
  choose_variant(h, tile);
  // A static plan (fixed scratch) keeps the deep key side's per-tile
  // partials: the carry's per-workgroup rows would not fit beside them.
  if (ar.base) h->deep_carry = false;
  const int32_t n_tiles = static_cast<int32_t>((n + tile - 1) / tile);
  std::vector<int32_t> pref_off(static_cast<size_t>(n_tiles) + 2, 0);
  for (int32_t t = 0; t < n_tiles; ++t) pref_off[t + 1] = pref_off[t] + depth[static_cast<int64_t>(t) * tile] - 1;
  pref_off[n_tiles + 1] = pref_off[n_tiles];  // sentinel read by the reducer
  std::vector<int32_t> prefix(static_cast<size_t>(pref_off[n_tiles]));
  std::vector<int32_t> pref_end(prefix.size());
  for (int32_t t = 0; t < n_tiles; ++t) {
    const int64_t s = static_cast<int64_t>(t) * tile;
    int32_t a = ext[A0 + s];  // walked in the extended table
    for (int d = depth[s] - 2; d >= 0; --d) {
      prefix[pref_off[t] + d] = loc(a);
      pref_end[pref_off[t] + d] = static_cast<int32_t>(eext[a] - A0);
      a = ext[a];
    }
  }
  // Work items of the fast kernels: chain groups (each row the previous
  // row's child) of up to qb queries / kb key-set entries. Per tile the
  // longest items (more than kCutSteps 4-row steps) are cut into parts while
  // scratch slots last; items are then sorted by steps, longest first
  // (stable).
  std::vector<int32_t> q_items, k_items;
  std::vector<int32_t> q_off(static_cast<size_t>(n_tiles) + 1, 0), k_off(static_cast<size_t>(n_tiles) + 1, 0);
  if (h->variant == 5) {
    struct Raw {
      int len, first, count;  // len: keys walked (queries) / query range (keys)
    };
    std::vector<Raw> raw;
    std::vector<int> order;
    std::vector<std::pair<int, int32_t>> items;
    auto emit = [&](bool cut, int slots, int max_parts, std::vector<int32_t>& out) {
      const size_t m = raw.size();
      std::vector<int> nparts(m, 1), slot(m, 0);
      order.resize(m);
      for (size_t i = 0; i < m; ++i) order[i] = static_cast<int>(i);
      std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return raw[a].len > raw[b].len; });
      int used = 0;
      for (int i : order) {
        const int nb = (raw[i].len + 3) / 4;
        if (!cut || used >= slots || nb <= agpt_fast::kCutSteps) break;
        nparts[i] = std::min(max_parts, (nb + agpt_fast::kCutSteps - 1) / agpt_fast::kCutSteps);
        slot[i] = used++;
      }
      for (size_t i = 0; i < m; ++i) {
        const int nb = (raw[i].len + 3) / 4;
        for (int p = 0; p < nparts[i]; ++p) {
          const int b0 = agpt_fast::part_begin(nb, p, nparts[i]);
          const int b1 = agpt_fast::part_begin(nb, p + 1, nparts[i]);
          items.emplace_back(b1 - b0,
                             agpt_fast::make_item(raw[i].first, raw[i].count, b0, b1, p, nparts[i], slot[i]));
        }
      }
      std::stable_sort(items.begin(), items.end(),
                       [](const std::pair<int, int32_t>& a, const std::pair<int, int32_t>& b) {
                         return a.first > b.first;
                       });
      for (const auto& it : items) out.push_back(it.second);
      items.clear();
      raw.clear();
    };
    // Query parts are merged from partial softmax states (forward) and dQ
    // partials; the bf16 backward needs δ over the whole path first, so its
    // query items stay whole.
    const bool cut_q = h->cfg.dtype == AGPT_DTYPE_F32;
    for (int32_t t = 0; t < n_tiles; ++t) {
      const int64_t s = static_cast<int64_t>(t) * tile;
      const int nt = static_cast<int>(std::min<int64_t>(tile, n - s));
      const int A = pref_off[t + 1] - pref_off[t];
      for (int r = 0; r < nt;) {
        int c = 1;
        while (c < h->qb && r + c < nt && parent[s + r + c] == s + r + c - 1) ++c;
        raw.push_back({depth[s + r + c - 1], r, c});
        r += c;
      }
      emit(cut_q, h->q_slots, agpt_fast::kQParts, q_items);
      q_off[t + 1] = static_cast<int32_t>(q_items.size());
      // Key-set entry k: prefix[k] for k < A (entry k-1 is its parent), else
      // tile row k - A (chained when its parent is the previous entry).
      auto chained = [&](int k) {
        if (k < A) return true;
        const int c = k - A;
        return c == 0 ? A > 0 : parent[s + c] == s + c - 1;
      };
      auto range_len = [&](int k) {
        if (k < A) return static_cast<int>(std::min<int64_t>(pref_end[pref_off[t] + k] - s, nt));
        const int c = k - A;
        return static_cast<int>(std::min<int64_t>(end[s + c] - s, nt)) - c;
      };
      const int nk = A + nt;
      for (int k = 0; k < nk;) {
        int c = 1;
        while (c < h->kb && k + c < nk && chained(k + c)) ++c;
        raw.push_back({range_len(k), k, c});
        k += c;
      }
      emit(h->split, h->k_slots, agpt_fast::kKParts, k_items);
      k_off[t + 1] = static_cast<int32_t>(k_items.size());
    }
  }
  const int D = h->cfg.n_heads * h->cfg.head_dim;
  h->T = n;
  h->tile = tile;
  h->n_tiles = n_tiles;
  h->n_chunks = (n_tiles + kChunkTiles - 1) / kChunkTiles;
  h->sum_depth = sumd;
  h->n_prefix_rows = pref_off[n_tiles];
  h->static_plan = ar.base != nullptr;  // from here on free_plan must not free
  if ((rc = upload(ar, &h->d_parent, parent)) != AGPT_OK) return rc;
  if ((rc = upload(ar, &h->d_depth, depth)) != AGPT_OK) return rc;
  if ((rc = upload(ar, &h->d_end, end)) != AGPT_OK) return rc;
  if ((rc = upload(ar, &h->d_pref_off, pref_off)) != AGPT_OK) return rc;
  if ((rc = upload(ar, &h->d_prefix, prefix)) != AGPT_OK) return rc;
  if ((rc = upload(ar, &h->d_pref_end, pref_end)) != AGPT_OK) return rc;
  if (h->variant == 5) {
    if ((rc = upload(ar, &h->d_q_items, q_items)) != AGPT_OK) return rc;
    if ((rc = upload(ar, &h->d_k_items, k_items)) != AGPT_OK) return rc;
    if ((rc = upload(ar, &h->d_q_item_off, q_off)) != AGPT_OK) return rc;
    if ((rc = upload(ar, &h->d_k_item_off, k_off)) != AGPT_OK) return rc;
  }
  if (h->variant == 6) {
    if ((rc = ar.get(reinterpret_cast<void**>(&h->d_sched), kSchedBytes)) != AGPT_OK) return rc;
    // Deep query side with few units per workgroup (plans of < 16 tiles per
    // CU, one head per unit): tiles of more key chunks are claimed first, so
    // that the last claims of the launch are the short ones. Larger plans
    // keep the tile order, in which neighbouring claims share their prefix.
    {
      int cus0 = 256;
      (void)hipDeviceGetAttribute(&cus0, hipDeviceAttributeMultiprocessorCount, h->device);
      if (h->deep && env_int("AGPT_ATTN_LPT", n_tiles < 16 * cus0 ? 1 : 0) != 0) {
        std::vector<int32_t> order(n_tiles);
        std::vector<int32_t> nch(n_tiles);
        for (int32_t t = 0; t < n_tiles; ++t) {
          order[t] = t;
          const int64_t nk = (pref_off[t + 1] - pref_off[t]) + std::min<int64_t>(tile, n - int64_t(t) * tile);
          nch[t] = static_cast<int32_t>((nk + agpt_deep::kChunk - 1) / agpt_deep::kChunk);
        }
        std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return nch[a] > nch[b]; });
        if ((rc = upload(ar, &h->d_tile_order, order)) != AGPT_OK) return rc;
      }
    }
    // Deep key side by subtree range: when every tile's rows have their
    // subtrees end within kRangeTiles tiles (and the plan has no context
    // rows, whose shares only the carry path collects), each tile's keys
    // take their queries from the contiguous rows [s, E) in one unit.
    h->deep_range = false;
    if (h->deep && A0 == 0 && tile == agpt_deep::kTile && env_int("AGPT_ATTN_RANGE", 1) != 0) {
      std::vector<int32_t> bend(static_cast<size_t>(n_tiles) * 4, 0), nq(n_tiles);
      bool fits = true;
      for (int32_t t = 0; t < n_tiles && fits; ++t) {
        const int64_t s = int64_t(t) * tile;
        const int nt = static_cast<int>(std::min<int64_t>(tile, n - s));
        int64_t te = s;
        for (int r = 0; r < nt; ++r) {
          bend[4 * t + r / agpt_blk::kBlk] = std::max(bend[4 * t + r / agpt_blk::kBlk], end[s + r]);
          te = std::max<int64_t>(te, end[s + r]);
        }
        nq[t] = static_cast<int32_t>((te - s + tile - 1) / tile);
        fits = nq[t] <= kRangeTiles;
      }
      if (fits) {
        std::vector<int32_t> order(n_tiles);
        for (int32_t t = 0; t < n_tiles; ++t) order[t] = t;
        std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return nq[a] > nq[b]; });
        if ((rc = upload(ar, &h->d_range_bend, bend)) != AGPT_OK) return rc;
        if ((rc = upload(ar, &h->d_range_order, order)) != AGPT_OK) return rc;
        h->deep_range = true;
        h->deep_carry = false;  // nothing to carry: no partials, E, F or carry rows
      }
    }
    // A forest of chains (each row's parent the row before it, or none) at
    // bf16 head_dim 64: plain causal attention per chain (agpt_chain).
    h->chain_plan = false;
    h->n_chains = 0;
    if (h->deep && A0 == 0 && h->cfg.dtype == AGPT_DTYPE_BF16 && env_int("AGPT_ATTN_CHAIN", 1) != 0) {
      bool chains = true;
      std::vector<int32_t> starts;
      for (int64_t r = 0; r < n && chains; ++r) {
        if (parent[r] < 0) starts.push_back(static_cast<int32_t>(r));
        else chains = parent[r] == r - 1;
      }
      // (the chain kernels number their (chain, head) units in 32 bits)
      if (chains && static_cast<int64_t>(starts.size()) * h->cfg.n_heads < (int64_t{1} << 31) - 2 * 65536) {
        const int32_t nc = static_cast<int32_t>(starts.size());
        starts.push_back(static_cast<int32_t>(n));
        std::vector<int32_t> order(nc);
        for (int32_t k = 0; k < nc; ++k) order[k] = k;
        std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
          return starts[a + 1] - starts[a] > starts[b + 1] - starts[b];
        });
        std::vector<int32_t> info(2 * static_cast<size_t>(nc));
        for (int32_t k = 0; k < nc; ++k) {
          info[2 * k] = starts[order[k]];
          info[2 * k + 1] = starts[order[k] + 1] - starts[order[k]];
        }
        if ((rc = upload(ar, &h->d_chain_info, info)) != AGPT_OK) return rc;
        h->n_chains = nc;
        h->chain_plan = true;
        h->chain_fused = env_int("AGPT_ATTN_CHAINFUSE", 1) != 0;
      }
    }
    // Up to 24 tiles per claim (the carry's reach), but at least ~8 chunks
    // per CU: a plan of few tiles (C5: 2048) would otherwise leave most
    // workgroups without a chunk.
    int cus = 256;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, h->device);
    // The deep key side's units are (chunk, head): ~8 per CU, and chunks up
    // to 96 tiles (fewer chunk partials and carry work: C4 83.0 -> 81.6 ms
    // at 48, the carry kernel 0.70 -> 0.39 ms at 96).
    // Claims are (chunk, head group) pairs (heads one by one on the deep key side).
    const int64_t per_claim = static_cast<int64_t>(n_tiles) *
                              (h->deep_carry ? h->cfg.n_heads : std::max(1, h->cfg.n_heads / std::max(1, h->hg)));
    const int cap = h->deep_carry ? 96 : 24;
    const int dflt = static_cast<int>(std::min<int64_t>(cap, std::max<int64_t>(1, per_claim / (8 * std::max(cus, 1)))));
    h->chunk_tiles = std::max(1, env_int("AGPT_ATTN_CHUNK", dflt));
    h->n_chunks_sched = std::max<int32_t>(1, n_tiles / h->chunk_tiles);
    // Chunks of one tile would carry nothing: the per-tile partials serve.
    if (h->chunk_tiles < 2) h->deep_carry = false;
    h->cs_slots = h->deep_carry ? static_cast<int>(std::min<int64_t>(static_cast<int64_t>(h->n_chunks_sched) *
                                                                          h->cfg.n_heads,
                                                                      8LL * std::max(cus, 1)))
                                : 0;
  }
  auto fl = [&](float** p, size_t bytes) { return ar.get(reinterpret_cast<void**>(p), bytes); };
  if (h->carry || h->deep_carry) {
    const size_t ebytes = static_cast<size_t>(h->n_chunks_sched) * agpt_blk::prefix_cap(maxd) * 2 * D * sizeof(float);
    if ((rc = fl(&h->d_E, ebytes)) != AGPT_OK || (rc = fl(&h->d_F, ebytes)) != AGPT_OK) return rc;
    if (h->deep_carry &&
        (rc = fl(&h->d_Cs, static_cast<size_t>(h->cs_slots) * 2 * agpt_blk::prefix_cap(maxd) * 2 *
                               h->cfg.head_dim * sizeof(float))) != AGPT_OK)
      return rc;
  } else if (!h->deep_range) {
    const size_t pbytes = std::max<size_t>(1, static_cast<size_t>(h->n_prefix_rows) * D) * sizeof(float);
    if ((rc = fl(&h->d_Pk, pbytes)) != AGPT_OK || (rc = fl(&h->d_Pv, pbytes)) != AGPT_OK) return rc;
    const size_t cbytes = std::max<size_t>(1, static_cast<size_t>(h->n_chunks) * maxd * D) * sizeof(float);
    if ((rc = fl(&h->d_Ck, cbytes)) != AGPT_OK || (rc = fl(&h->d_Cv, cbytes)) != AGPT_OK) return rc;
  }
  if (h->variant == 5 || h->variant == 6)
    if ((rc = fl(&h->d_Dl, static_cast<size_t>(n) * h->cfg.n_heads * sizeof(float))) != AGPT_OK) return rc;
  if (ar.overflow)
    return set_error(AGPT_ERR_INVALID_ARG,
                     "agpt_attn_plan_static: the batch needs %zu bytes of device tables and workspace, more "
                     "than the %zu bytes of static scratch (AGPT_STATIC_SCRATCH_BYTES); use agpt_attn_plan",
                     ar.used, kScratchBytes);
  h->planned = true;
  g_last_error.clear();
  return AGPT_OK;
}

}  // namespace

extern "C" int agpt_attn_plan(agpt_attn_handle h, const int32_t* parent, int64_t n) {
  if (!h) return set_error(AGPT_ERR_INVALID_ARG, "null handle");
  if (n < 1 || !parent) return set_error(AGPT_ERR_INVALID_ARG, "empty tree or null parent table");
  HIP_TRY(hipSetDevice(h->device));
  Arena ar;
  const int rc = plan_impl(h, parent, n, 0, {}, ar);
  if (rc != AGPT_OK) free_plan(h);
  h->row_off = 0;
  h->n_ctx = 0;
  return rc;
}

extern "C" int agpt_attn_plan_range(agpt_attn_handle h, const int32_t* parent, int64_t n_total,
                                    int64_t row_begin, int64_t row_end, int ctx_mode) {
  if (!h) return set_error(AGPT_ERR_INVALID_ARG, "null handle");
  if (!parent || row_begin < 0 || row_end <= row_begin || row_end > n_total)
    return set_error(AGPT_ERR_INVALID_ARG, "need 0 <= row_begin < row_end <= n_total and a parent table");
  if (ctx_mode != AGPT_CTX_GLOBAL && ctx_mode != AGPT_CTX_PACKED)
    return set_error(AGPT_ERR_INVALID_ARG, "ctx_mode %d", ctx_mode);
  if (n_total >= (int64_t{1} << 31) - kMaxTileRows)
    return set_error(AGPT_ERR_INVALID_ARG, "n_total %lld exceeds int32 row indexing", (long long)n_total);
  // The context: ancestors of row_begin, root first (ascending rows).
  std::vector<int64_t> chain;
  for (int64_t a = parent[row_begin]; a >= 0; a = parent[a]) {
    if (a >= row_begin || parent[a] >= a || parent[a] < -1)
      return set_error(AGPT_ERR_NOT_DFS, "ancestor %lld of row_begin is not an earlier row", (long long)a);
    if (static_cast<int>(chain.size()) >= kMaxDepth)
      return set_error(AGPT_ERR_TOO_DEEP, "row_begin is deeper than %d", kMaxDepth);
    chain.push_back(a);
  }
  std::reverse(chain.begin(), chain.end());
  const int32_t A0 = static_cast<int32_t>(chain.size());
  const int64_t n = row_end - row_begin;
  std::vector<int32_t> ext(static_cast<size_t>(A0 + n));
  for (int32_t j = 0; j < A0; ++j) ext[j] = j - 1;
  for (int64_t g = row_begin; g < row_end; ++g) {
    const int32_t p = parent[g];
    int32_t e;
    if (p >= g || p < -1) {
      return set_error(AGPT_ERR_NOT_DFS, "parent[%lld] = %d is not an earlier row or -1", (long long)g, p);
    } else if (p >= row_begin) {
      e = static_cast<int32_t>(A0 + (p - row_begin));
    } else if (p < 0) {
      e = -1;
    } else {
      const auto it = std::lower_bound(chain.begin(), chain.end(), static_cast<int64_t>(p));
      if (it == chain.end() || *it != p)
        return set_error(AGPT_ERR_NOT_DFS,
                         "row %lld: its parent %d lies before the range and is not an ancestor of row_begin",
                         (long long)g, p);
      e = static_cast<int32_t>(it - chain.begin());
    }
    ext[A0 + (g - row_begin)] = e;
  }
  std::vector<int32_t> ctx_local(static_cast<size_t>(A0));
  for (int32_t j = 0; j < A0; ++j)
    ctx_local[j] = static_cast<int32_t>(ctx_mode == AGPT_CTX_PACKED ? j - A0 : chain[j] - row_begin);
  HIP_TRY(hipSetDevice(h->device));
  Arena ar;
  const int rc = plan_impl(h, ext.data(), A0 + n, A0, ctx_local, ar);
  if (rc != AGPT_OK) {
    free_plan(h);
    return rc;
  }
  h->row_off = ctx_mode == AGPT_CTX_PACKED ? A0 : row_begin;
  h->n_ctx = A0;
  h->ctx_add = ctx_mode == AGPT_CTX_GLOBAL;
  return AGPT_OK;
}

extern "C" int agpt_attn_plan_static(agpt_attn_handle h, const int32_t* parent, int64_t n) {
  if (!h) return set_error(AGPT_ERR_INVALID_ARG, "null handle");
  if (n < 1 || !parent) return set_error(AGPT_ERR_INVALID_ARG, "empty tree or null parent table");
  if (h->planned && !h->static_plan)
    return set_error(AGPT_ERR_INVALID_ARG,
                     "agpt_attn_plan_static: the handle holds an allocated plan (freeing it would call "
                     "hipFree); use a handle without one");
  HIP_TRY(hipSetDevice(h->device));
  Arena ar;
  int rc = scratch_base(h->device, &ar.base);
  if (rc != AGPT_OK) return rc;
  {
    // Claim the scratch and upload into it under one lock: an earlier static
    // plan on this device stops being valid whatever happens next, and two
    // threads planning static on one device never write the scratch at once
    // (the later claim's tables are the ones left in it).
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    h->static_gen = ++g_scratch_gen[h->device];
    rc = plan_impl(h, parent, n, 0, {}, ar);
  }
  if (rc != AGPT_OK) free_plan(h);
  h->row_off = 0;
  h->n_ctx = 0;
  return rc;
}

// The radix tree's node-token rows: node r's edge rows follow each other,
// the first one's parent being the last row of radix_parent[r]'s edge.
extern "C" int agpt_attn_radix_rows(const int32_t* radix_parent, const int32_t* edge_len, int64_t n_radix,
                                    int32_t* parent_out, int64_t cap, int64_t* n_rows) {
  if (n_radix < 1 || !radix_parent || !edge_len || !n_rows)
    return set_error(AGPT_ERR_INVALID_ARG, "empty radix tree or null table");
  int64_t rows = 0;
  for (int64_t r = 0; r < n_radix; ++r) {
    const int32_t rp = radix_parent[r];
    if (rp < -1 || rp >= r)
      return set_error(AGPT_ERR_NOT_DFS, "radix_parent[%lld] = %d is not an earlier node or -1",
                       (long long)r, rp);
    if (edge_len[r] < 1) return set_error(AGPT_ERR_INVALID_ARG, "edge_len[%lld] = %d", (long long)r, edge_len[r]);
    rows += edge_len[r];
    if (rows >= (int64_t{1} << 31) - kMaxTileRows)
      return set_error(AGPT_ERR_INVALID_ARG, "more than 2^31 rows by radix node %lld", (long long)r);
  }
  *n_rows = rows;
  if (!parent_out) return AGPT_OK;
  if (cap < rows) return set_error(AGPT_ERR_INVALID_ARG, "cap %lld < %lld rows", (long long)cap, (long long)rows);
  std::vector<int32_t> last_row(static_cast<size_t>(n_radix));
  int32_t next = 0;
  for (int64_t r = 0; r < n_radix; ++r) {
    int32_t prev = radix_parent[r] < 0 ? -1 : last_row[radix_parent[r]];
    for (int32_t j = 0; j < edge_len[r]; ++j, ++next) {
      parent_out[next] = prev;
      prev = next;
    }
    last_row[r] = prev;
  }
  return AGPT_OK;
}

extern "C" int agpt_attn_plan_radix(agpt_attn_handle h, const int32_t* radix_parent,
                                    const int32_t* edge_len, int64_t n_radix) {
  if (!h) return set_error(AGPT_ERR_INVALID_ARG, "null handle");
  int64_t rows = 0;
  int rc = agpt_attn_radix_rows(radix_parent, edge_len, n_radix, nullptr, 0, &rows);
  if (rc != AGPT_OK) return rc;
  std::vector<int32_t> parent(static_cast<size_t>(rows));
  if ((rc = agpt_attn_radix_rows(radix_parent, edge_len, n_radix, parent.data(), rows, &rows)) != AGPT_OK)
    return rc;
  return agpt_attn_plan(h, parent.data(), rows);
}

extern "C" const char* agpt_attn_describe(agpt_attn_handle h) {
  if (!h) return "null handle";
  if (!h->planned) return "no plan";
  char buf[400];
  if (h->variant == 6 && h->deep && h->chain_plan)
    snprintf(buf, sizeof(buf),
             "dense-causal chain kernels (a forest of %d chains; unit = chain x head, %d waves, the chain's rows "
             "in LDS), %s: lds=%zu lds_limit=%d",
             h->n_chains, agpt_chain::kWaves,
             h->chain_fused ? "one-launch backward (query side, then key side per unit; nothing to reduce)"
                            : "split backward with the key side by subtree range",
             agpt_chain::lds_bytes(), h->max_lds);
  else if (h->variant == 6 && h->deep)
    snprintf(buf, sizeof(buf),
             "streamed key ring (deep prefixes) 16x16 mfma, split backward%s: tile_rows=%d tiles=%d "
             "heads_per_wg=1 key_chunk=%d fwd_lds=%zu bwd_q_lds=%zu bwd_kv_lds=%zu lds_limit=%d",
             h->deep_range ? " with the key side by subtree range"
             : h->deep_carry ? " with path-carry"
                             : "",
             h->tile, h->n_tiles, agpt_deep::kChunk, h->fwd_lds, h->bq_lds,
             h->kv_lds, h->max_lds);
  else if (h->variant == 6)
    snprintf(buf, sizeof(buf),
             "streaming block-sparse 16x16 mfma, %s backward: tile_rows=%d tiles=%d heads_per_wg=%d "
             "heads_per_unit=%d/%d fwd_lds=%zu bwd_lds=%zu/%zu lds_limit=%d",
             h->fused ? (h->carry ? "one-pass path-carry" : "one-pass") : "split", h->tile, h->n_tiles, h->hg, std::min(h->fwd_uh >= 4 ? 4 : h->fwd_uh >= 2 ? 2 : 1, h->hg),
             h->unit_all_heads ? h->hg : 1,
             h->fwd_lds, h->fused ? h->fb_lds : h->bq_lds, h->fused ? 0 : h->kv_lds, h->max_lds);
  else if (h->variant == 5)
    snprintf(buf, sizeof(buf),
             "streaming chain-grouped mfma, split backward: tile_rows=%d tiles=%d heads_per_wg=%d "
             "query_group=%d key_group=%d cut_slots=%d/%d fwd_lds=%zu bwd_q_lds=%zu bwd_kv_lds=%zu "
             "lds_limit=%d",
             h->tile, h->n_tiles, h->hg, h->qb, h->kb, h->q_slots, h->k_slots, h->fwd_lds, h->bq_lds,
             h->kv_lds, h->max_lds);
  else
    snprintf(buf, sizeof(buf), "global-memory walk: tile_rows=%d tiles=%d", h->tile, h->n_tiles);
  h->desc = buf;
  if (h->n_ctx > 0) {
    snprintf(buf, sizeof(buf), "; range batch: %d context rows (%s)", h->n_ctx,
             h->ctx_add ? "dK/dV added into their rows" : "dK/dV written to the packed rows");
    h->desc += buf;
  }
  return h->desc.c_str();
}

extern "C" int agpt_attn_plan_info(agpt_attn_handle h, int64_t* n_nodes, int64_t* n_tiles,
                                   int64_t* sum_depth, int32_t* max_depth) {
  if (!h) return set_error(AGPT_ERR_INVALID_ARG, "null handle");
  if (!h->planned) return set_error(AGPT_ERR_NO_PLAN, "no plan");
  if (n_nodes) *n_nodes = h->T;
  if (n_tiles) *n_tiles = h->n_tiles;
  if (sum_depth) *sum_depth = h->sum_depth;
  if (max_depth) *max_depth = h->max_depth;
  return AGPT_OK;
}

namespace {

int check_opts(const agpt_attn_opts* o) {
  if (o && o->rope_cos) {
    if (!o->rope_sin || o->rope_seq_len < 1)
      return set_error(AGPT_ERR_INVALID_ARG, "RoPE needs both tables and rope_seq_len >= 1");
  }
  return AGPT_OK;
}

float scale_of(const agpt_attn_s* h, const agpt_attn_opts* o) {
  if (o && o->scale != 0.0f) return o->scale;
  return static_cast<float>(1.0 / std::sqrt(static_cast<double>(h->cfg.head_dim)));
}

// Records the caller's profiling event `i` (see agpt_attn_opts.prof_events).
struct ProfMarks {
  void** ev = nullptr;
  int n = 0;
  hipStream_t st = nullptr;
  void mark(int i) const {
    if (ev && i < n && ev[i]) (void)hipEventRecord(static_cast<hipEvent_t>(ev[i]), st);
  }
};

// Persistent grid of a streaming kernel: as many workgroups as fit on the
// device at once, a multiple of 8 (XCDs) and of the head-group count, and no
// more than one per (tile, head group).
// Workgroups of `fn` resident per CU with `lds` dynamic LDS bytes: the
// runtime's estimate, capped by the LDS a CU holds when each workgroup's
// static + dynamic LDS is allocated in 512-byte granules (the runtime's
// estimate does not round, and an over-count leaves the persistent grid's
// last workgroups waiting for a whole earlier workgroup to finish). 0 if
// `fn` cannot launch with `lds`.
template <typename Fn>
int wg_per_cu(Fn fn, size_t lds, int lds_per_cu, int threads = agpt_fast::kThreads) {
  hipFuncAttributes fa{};
  if (hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(fn)) != hipSuccess) return 0;
  const size_t total = (fa.sharedSizeBytes + lds + 511) & ~static_cast<size_t>(511);
  if (total > static_cast<size_t>(lds_per_cu)) return 0;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), threads,
                                                   lds) != hipSuccess)
    return 0;
  return std::min(n, static_cast<int>(lds_per_cu / total));
}

template <typename Fn>
int stream_grid(const agpt_attn_s* h, Fn fn, size_t lds, int hg = 0) {
  int per_cu = wg_per_cu(fn, lds, h->max_lds), cus = 256;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, h->device);
  const int n_hg = h->cfg.n_heads / (hg > 0 ? hg : h->hg);
  const int m = std::lcm(agpt_fast::kXcds, n_hg);
  const int64_t units = static_cast<int64_t>(h->n_tiles) * n_hg;
  int64_t g = static_cast<int64_t>(std::max(per_cu, 1)) * cus;
  g = std::min(g, (units + m - 1) / m * m);
  g = std::max<int64_t>(g / m * m, m);
  return static_cast<int>(g);
}

// Workgroups of a chain-forest kernel: as many as fit the chip, at most one
// per (chain, head) unit.
template <typename Fn>
int chain_grid(const agpt_attn_s* h, Fn fn) {
  int cus = 256;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, h->device);
  const int64_t units = static_cast<int64_t>(h->n_chains) * h->cfg.n_heads;
  const int64_t g =
      static_cast<int64_t>(std::max(wg_per_cu(fn, agpt_chain::lds_bytes(), h->max_lds, agpt_chain::kThreads), 1)) * cus;
  return static_cast<int>(std::max<int64_t>(1, std::min(g, units)));
}

// Heads per unit of the deep-prefix kernels: all heads of a tile when the
// plan has tiles enough for ~16 units per CU (tables built once per tile,
// heads streamed back to back; half of them in the forward from 8 heads
// on), else two (units enough to fill the chip, each unit's tables shared
// by two heads; one for an odd head count). AGPT_ATTN_DHPU overrides (a
// divisor of the head count).
int deep_heads_per_unit(const agpt_attn_s* h, bool fwd = false) {
  const int H = h->cfg.n_heads;
  int cus = 256;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, h->device);
  // The forward's units are lighter (no δ pass): with 8 or more heads it
  // takes half of them per unit, twice the units for the same tables
  // (C4: fwd 18.3 -> 17.95 ms; the dQ kernel is faster with all heads).
  const int big = fwd && H >= 8 && H % 2 == 0 ? H / 2 : H;
  int hpu = env_int("AGPT_ATTN_DHPU", h->n_tiles >= 16 * cus ? big : H % 2 == 0 ? 2 : 1);
  if (hpu < 1 || hpu > H || H % hpu != 0) hpu = 1;
  return hpu;
}

// Clears the block kernels' chunk counters on the stream with a kernel, not
// a memset node: the launch sequence stays valid under stream capture
// (memset nodes in captured graphs have given wrong results on replays).
__global__ void zero_i32_kernel(int32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

void clear_sched(const agpt_attn_s* h, hipStream_t st) {
  hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(64), 0, st, h->d_sched,
                     static_cast<int>(kSchedBytes / sizeof(int32_t)));
}

template <typename Fn>
void set_lds(Fn fn, size_t bytes) {
  if (bytes > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

template <typename Fn>
void with_124(int v, Fn&& fn) {  // v in {1, 2, 4}
  if (v == 4) fn(std::integral_constant<int, 4>{});
  else if (v == 2) fn(std::integral_constant<int, 2>{});
  else fn(std::integral_constant<int, 1>{});
}

// Block kernels: heads per workgroup (1, 2, 4) and heads per unit (all or one).
// Block-kernel shapes that are built: head_dim 16 and 32 with 1, 2 or 4
// heads per workgroup; head_dim 64 with one.
constexpr bool block_shape_ok(int hd, int hg, int uh) { return hd <= 32 || (hg == 1 && uh == 1); }

template <typename Fn>
void with_block_heads(const agpt_attn_s* h, int uh, Fn&& fn) {
  with_124(h->hg, [&](auto hgc) {
    constexpr int HG = decltype(hgc)::value;
    if constexpr (HG >= 4) {
      if (uh >= 4) {
        fn(hgc, std::integral_constant<int, 4>{});
        return;
      }
    }
    if constexpr (HG >= 2) {
      if (uh >= 2) {
        fn(hgc, std::integral_constant<int, 2>{});
        return;
      }
    }
    fn(hgc, std::integral_constant<int, 1>{});
  });
}

template <int HD, typename Tin>
void launch_fwd(const agpt_attn_s* h, const void* q, const void* k, const void* v, void* o,
                float* lse, float scale, hipStream_t st, const ProfMarks& pm) {
  pm.mark(0);
  if (h->variant == 6 && h->deep) {
    if constexpr (HD == 64 && sizeof(Tin) == 2) {
      if (h->chain_plan) {  // units dealt by the grid: no counters to clear
        auto fn = agpt_chain::fwd_kernel<PlanDev>;
        set_lds(fn, agpt_chain::lds_bytes());
        hipLaunchKernelGGL(fn, dim3(chain_grid(h, fn)), dim3(agpt_chain::kThreads), agpt_chain::lds_bytes(), st,
                           plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                           static_cast<const Tin*>(v), static_cast<Tin*>(o), lse, h->cfg.n_heads, scale);
        pm.mark(1);
        return;
      }
    }
    if constexpr (HD == 64) {
      clear_sched(h, st);
      const int hpu = deep_heads_per_unit(h, true);
      auto fn = agpt_deep::fwd_kernel<HD, Tin, PlanDev>;
      set_lds(fn, h->fwd_lds);
      hipLaunchKernelGGL(fn, dim3(stream_grid(h, fn, h->fwd_lds, hpu)), dim3(agpt_deep::kThreads), h->fwd_lds, st,
                         plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                         static_cast<const Tin*>(v), static_cast<Tin*>(o), lse, h->cfg.n_heads, hpu, scale);
    }
  } else if (h->variant == 6) {
    if constexpr (HD == 16 || HD == 32 || HD == 64) {
      clear_sched(h, st);
      with_block_heads(h, h->fwd_uh, [&](auto hgc, auto uhc) {
        constexpr int HG = decltype(hgc)::value, UH = decltype(uhc)::value;
        if constexpr (block_shape_ok(HD, HG, UH)) {
          auto fn = agpt_blk::fwd_kernel<HD, Tin, HG, UH, PlanDev>;
          set_lds(fn, h->fwd_lds);
          hipLaunchKernelGGL(fn, dim3(stream_grid(h, fn, h->fwd_lds)), dim3(agpt_blk::kThreads), h->fwd_lds,
                             st, plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                             static_cast<const Tin*>(v), static_cast<Tin*>(o), lse, h->cfg.n_heads, scale);
        }
      });
    }
  } else if (h->variant == 5) {
    if constexpr (HD >= 16 && HD <= 32) {
      with_124(h->hg, [&](auto hgc) {
        constexpr int HG = decltype(hgc)::value;
        auto fn = agpt_fast::fwd_kernel<HD, Tin, HG, PlanDev>;
        set_lds(fn, h->fwd_lds);
        hipLaunchKernelGGL(fn, dim3(stream_grid(h, fn, h->fwd_lds)), dim3(agpt_fast::kThreads), h->fwd_lds,
                           st, plan_dev(h),
                           static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                           static_cast<const Tin*>(v), static_cast<Tin*>(o), lse, h->cfg.n_heads,
                           scale);
      });
    }
  } else {
    hipLaunchKernelGGL((trie_fwd_kernel<HD, Tin>), dim3(h->n_tiles), dim3(256), 0, st, plan_dev(h),
                       static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                       static_cast<const Tin*>(v), static_cast<Tin*>(o), lse, h->cfg.n_heads, scale);
  }
  pm.mark(1);
}

// Finishes the context rows' share of dK/dV (range plans; see trie_ctx_kernel).
template <int HD>
void launch_ctx(const agpt_attn_s* h, float* dk, float* dv, RopeArgs rope, hipStream_t st, hipEvent_t wait) {
  if (h->n_ctx <= 0) return;
  if (wait) (void)hipStreamWaitEvent(st, wait, 0);
  const int D = h->cfg.n_heads * HD;
  const bool chunks = h->variant == 6 && ((h->fused && h->carry) || h->deep_carry);
  const int P = agpt_blk::prefix_cap(h->max_depth);
  const int rows = chunks ? h->chunk_tiles * agpt_blk::kTile : h->tile;
  const int parts = chunks ? h->n_chunks_sched : h->n_tiles;
  hipLaunchKernelGGL((trie_ctx_kernel<HD>), dim3(2 * D / 4, h->n_ctx), dim3(256), 0, st, plan_dev(h),
                     chunks ? h->d_E : h->d_Pk, chunks ? h->d_E : h->d_Pv, chunks ? 1 : 0, P, rows, parts, dk, dv,
                     rope, h->cfg.n_heads, h->ctx_add ? 1 : 0);
}

template <int HD, typename Tin>
void launch_bwd(const agpt_attn_s* h, const void* q, const void* k, const void* v, const void* o,
                const float* lse, const void* dO, float* dq, float* dk, float* dv,
                const float* acc_dk, const float* acc_dv, RopeArgs rope, float scale,
                hipStream_t st, const ProfMarks& pm, hipEvent_t ctx_wait) {
  const int D = h->cfg.n_heads * HD;
  pm.mark(0);
  bool fused_done = false;
  if constexpr ((HD == 16 || HD == 32) && std::is_same<Tin, float>::value) {
    if (h->variant == 6 && h->fused) {
      clear_sched(h, st);
      auto run = [&](auto hgc, auto cc) {
        constexpr int HG = decltype(hgc)::value;
        constexpr bool kCarry = decltype(cc)::value;
        if constexpr (HG <= 2) {
          auto fb = agpt_blk::bwd_kernel<HD, Tin, HG, kCarry, PlanDev, RopeArgs>;
          set_lds(fb, h->fb_lds);
          hipLaunchKernelGGL(fb, dim3(stream_grid(h, fb, h->fb_lds, HG)), dim3(agpt_blk::kThreads), h->fb_lds,
                             st, plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                             static_cast<const Tin*>(v), static_cast<const Tin*>(o), lse,
                             static_cast<const Tin*>(dO), dq, dk, dv, kCarry ? h->d_E : h->d_Pk,
                             kCarry ? h->d_F : h->d_Pv, acc_dk, acc_dv, rope, h->cfg.n_heads, scale);
        }
      };
      with_124(h->fhg, [&](auto hgc) {
        if constexpr (HD == 16) {
          if (h->carry) {
            run(hgc, std::true_type{});
            return;
          }
        }
        run(hgc, std::false_type{});
      });
      pm.mark(1);
      fused_done = true;
      if (h->carry) {
        pm.mark(2);
        pm.mark(3);
        if (HD == 16 && h->n_chunks_sched > 1)
          hipLaunchKernelGGL((agpt_blk::bwd_carry_kernel<HD, PlanDev, RopeArgs>), dim3(h->n_chunks_sched - 1),
                             dim3(256), 0, st, plan_dev(h), h->d_E, h->d_F, dk, dv, acc_dk, acc_dv, rope,
                             h->cfg.n_heads);
        launch_ctx<HD>(h, dk, dv, rope, st, ctx_wait);
        pm.mark(4);
        return;
      }
    }
  }
  if (fused_done) {
  } else if (h->variant == 6 && h->deep) {
    if constexpr (HD == 64 && sizeof(Tin) == 2) {
      if (h->chain_plan && h->chain_fused) {  // units dealt by the grid: no counters to clear
        auto fb = agpt_chain::bwd_kernel<PlanDev, RopeArgs>;
        set_lds(fb, agpt_chain::lds_bytes());
        hipLaunchKernelGGL(fb, dim3(chain_grid(h, fb)), dim3(agpt_chain::kThreads), agpt_chain::lds_bytes(), st,
                           plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                           static_cast<const Tin*>(v), lse, static_cast<const Tin*>(dO), dq, dk, dv, acc_dk,
                           acc_dv, rope, h->cfg.n_heads, scale);
        pm.mark(1);
        pm.mark(2);
        pm.mark(3);
        pm.mark(4);
        return;
      }
      if (h->chain_plan) {
        auto fq = agpt_chain::bwd_q_kernel<PlanDev, RopeArgs>;
        set_lds(fq, agpt_chain::lds_bytes());
        hipLaunchKernelGGL(fq, dim3(chain_grid(h, fq)), dim3(agpt_chain::kThreads), agpt_chain::lds_bytes(), st,
                           plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                           static_cast<const Tin*>(v), lse, static_cast<const Tin*>(dO), dq, h->d_Dl, rope,
                           h->cfg.n_heads, scale);
        pm.mark(1);
        auto fk = agpt_chain::bwd_kv_kernel<PlanDev, RopeArgs>;
        set_lds(fk, agpt_chain::lds_bytes());
        hipLaunchKernelGGL(fk, dim3(chain_grid(h, fk)), dim3(agpt_chain::kThreads), agpt_chain::lds_bytes(), st,
                           plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                           static_cast<const Tin*>(v), lse, h->d_Dl, static_cast<const Tin*>(dO), dk, dv, acc_dk,
                           acc_dv, rope, h->cfg.n_heads, scale);
        pm.mark(2);
        pm.mark(3);
        pm.mark(4);
        return;
      }
    }
    if constexpr (HD == 64) {
      clear_sched(h, st);
      const int hpu = deep_heads_per_unit(h);
      auto launch_q = [&](auto fq) {
        set_lds(fq, h->bq_lds);
        hipLaunchKernelGGL(fq, dim3(stream_grid(h, fq, h->bq_lds, hpu)), dim3(agpt_deep::kThreads), h->bq_lds, st,
                           plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                           static_cast<const Tin*>(v), static_cast<const Tin*>(o), lse,
                           static_cast<const Tin*>(dO), dq, h->d_Dl, rope, h->cfg.n_heads, hpu, scale);
      };
      // bf16: δ and dQ in one pass over the key chunks (AGPT_ATTN_DQ1=0: a δ pass, then dQ)
      if constexpr (sizeof(Tin) == 2) {
        if (h->dq_one_pass) launch_q(agpt_deep::bwd_q_kernel<HD, Tin, PlanDev, RopeArgs, true>);
        else launch_q(agpt_deep::bwd_q_kernel<HD, Tin, PlanDev, RopeArgs, false>);
      } else {
        launch_q(agpt_deep::bwd_q_kernel<HD, Tin, PlanDev, RopeArgs, false>);
      }
      pm.mark(1);
      if (h->deep_range) {
        auto fr = agpt_deep::bwd_kv_range_kernel<HD, Tin, PlanDev, RopeArgs>;
        set_lds(fr, h->kv_range_lds);
        int cus = 256;
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, h->device);
        const int64_t units = static_cast<int64_t>(h->n_tiles) * h->cfg.n_heads;
        const int grid = static_cast<int>(
            std::max<int64_t>(1, std::min<int64_t>(int64_t(wg_per_cu(fr, h->kv_range_lds, h->max_lds)) * cus, units)));
        hipLaunchKernelGGL(fr, dim3(grid), dim3(agpt_deep::kThreads), h->kv_range_lds, st, plan_dev(h),
                           static_cast<const Tin*>(q), static_cast<const Tin*>(k), static_cast<const Tin*>(v), lse,
                           h->d_Dl, static_cast<const Tin*>(dO), dk, dv, acc_dk, acc_dv, rope, h->cfg.n_heads,
                           scale);
        pm.mark(2);
        pm.mark(3);
        pm.mark(4);
        return;
      }
      if (h->deep_carry) {
        // Key slots of a tile: prefix_cap + 64. A plan to depth 128 keeps
        // every slot's sums in registers (4 kRegIters blocks of 16) and, in
        // bf16, each slot's K/V slices in an LDS cache tagged by row;
        // deeper plans (or AGPT_ATTN_REGITERS=2) keep the first 4
        // kRegItersDeep blocks in registers and the rest in the carry rows.
        const bool regs = env_int("AGPT_ATTN_REGCARRY", 1) != 0;
        const bool all_regs = agpt_blk::prefix_cap(h->max_depth) + agpt_deep::kTile <= 64 * agpt_deep::kRegIters &&
                              env_int("AGPT_ATTN_REGITERS", agpt_deep::kRegIters) == agpt_deep::kRegIters;
        auto fc = !regs      ? agpt_deep::bwd_kv_carry_kernel<HD, Tin, 0, PlanDev, RopeArgs>
                  : all_regs ? agpt_deep::bwd_kv_carry_kernel<HD, Tin, agpt_deep::kRegIters, PlanDev, RopeArgs>
                             : agpt_deep::bwd_kv_carry_kernel<HD, Tin, agpt_deep::kRegItersDeep, PlanDev, RopeArgs>;
        const size_t lds =
            h->kv_lds + agpt_deep::kv_cache_bytes(regs && all_regs ? agpt_deep::kRegIters : 0, sizeof(Tin));
        set_lds(fc, lds);
        int cus = 256;
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, h->device);
        const int grid = std::max(1, std::min(wg_per_cu(fc, lds, h->max_lds) * cus, h->cs_slots));
        hipLaunchKernelGGL(fc, dim3(grid), dim3(agpt_deep::kThreads), lds, st, plan_dev(h),
                           static_cast<const Tin*>(q), static_cast<const Tin*>(k), static_cast<const Tin*>(v), lse,
                           h->d_Dl, static_cast<const Tin*>(dO), dk, dv, h->d_E, h->d_F, h->d_Cs, acc_dk, acc_dv,
                           rope, h->cfg.n_heads, scale);
        pm.mark(2);
        pm.mark(3);
        if (h->n_chunks_sched > 1)
          hipLaunchKernelGGL((agpt_blk::bwd_carry_kernel<HD, PlanDev, RopeArgs>), dim3(h->n_chunks_sched - 1),
                             dim3(256), 0, st, plan_dev(h), h->d_E, h->d_F, dk, dv, acc_dk, acc_dv, rope,
                             h->cfg.n_heads);
        launch_ctx<HD>(h, dk, dv, rope, st, ctx_wait);
        pm.mark(4);
        return;
      }
      auto fk = agpt_deep::bwd_kv_kernel<HD, Tin, PlanDev, RopeArgs>;
      set_lds(fk, h->kv_lds);
      hipLaunchKernelGGL(fk, dim3(stream_grid(h, fk, h->kv_lds, hpu)), dim3(agpt_deep::kThreads), h->kv_lds, st,
                         plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                         static_cast<const Tin*>(v), lse, h->d_Dl, static_cast<const Tin*>(dO), dk, dv,
                         h->d_Pk, h->d_Pv, acc_dk, acc_dv, rope, h->cfg.n_heads, hpu, scale);
    }
  } else if (h->variant == 6) {
    if constexpr (HD == 16 || HD == 32 || HD == 64) {
      clear_sched(h, st);
      with_block_heads(h, h->unit_all_heads ? h->hg : 1, [&](auto hgc, auto uhc) {
        constexpr int HG = decltype(hgc)::value, UH = decltype(uhc)::value;
        if constexpr (block_shape_ok(HD, HG, UH)) {
          auto fq = agpt_blk::bwd_q_kernel<HD, Tin, HG, UH, PlanDev, RopeArgs>;
          set_lds(fq, h->bq_lds);
          hipLaunchKernelGGL(fq, dim3(stream_grid(h, fq, h->bq_lds)), dim3(agpt_blk::kThreads), h->bq_lds,
                             st, plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                             static_cast<const Tin*>(v), static_cast<const Tin*>(o), lse,
                             static_cast<const Tin*>(dO), dq, h->d_Dl, rope, h->cfg.n_heads, scale);
          pm.mark(1);
          auto fk = agpt_blk::bwd_kv_kernel<HD, Tin, HG, UH, PlanDev, RopeArgs>;
          set_lds(fk, h->kv_lds);
          hipLaunchKernelGGL(fk, dim3(stream_grid(h, fk, h->kv_lds)), dim3(agpt_blk::kThreads), h->kv_lds,
                             st, plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                             static_cast<const Tin*>(v), lse, h->d_Dl, static_cast<const Tin*>(dO), dk, dv,
                             h->d_Pk, h->d_Pv, acc_dk, acc_dv, rope, h->cfg.n_heads, scale);
        }
      });
    }
  } else if (h->variant == 5) {
    if constexpr (HD >= 16 && HD <= 32) {
      with_124(h->hg, [&](auto hgc) {
        constexpr int HG = decltype(hgc)::value;
        auto fq = agpt_fast::bwd_q_kernel<HD, Tin, HG, PlanDev, RopeArgs>;
        set_lds(fq, h->bq_lds);
        hipLaunchKernelGGL(fq, dim3(stream_grid(h, fq, h->bq_lds)), dim3(agpt_fast::kThreads), h->bq_lds,
                           st, plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                           static_cast<const Tin*>(v), static_cast<const Tin*>(o), lse,
                           static_cast<const Tin*>(dO), dq, h->d_Dl, rope, h->cfg.n_heads, scale);
        pm.mark(1);
        auto fk = agpt_fast::bwd_kv_kernel<HD, Tin, HG, PlanDev, RopeArgs>;
        set_lds(fk, h->kv_lds);
        hipLaunchKernelGGL(fk, dim3(stream_grid(h, fk, h->kv_lds)), dim3(agpt_fast::kThreads), h->kv_lds,
                           st, plan_dev(h), static_cast<const Tin*>(q), static_cast<const Tin*>(k),
                           static_cast<const Tin*>(v), lse, h->d_Dl, static_cast<const Tin*>(dO), dk, dv,
                           h->d_Pk, h->d_Pv, acc_dk, acc_dv, rope, h->cfg.n_heads, scale);
      });
    }
  } else {
    hipLaunchKernelGGL((trie_bwd_kernel<HD, Tin>), dim3(h->n_tiles), dim3(256), 0, st, plan_dev(h),
                       static_cast<const Tin*>(q), static_cast<const Tin*>(k), static_cast<const Tin*>(v),
                       static_cast<const Tin*>(o), lse, static_cast<const Tin*>(dO), dq, dk, dv, h->d_Pk,
                       h->d_Pv, acc_dk, acc_dv, rope, h->cfg.n_heads, scale);
    pm.mark(1);
  }
  pm.mark(2);
  if (h->n_tiles > 1) {
    hipLaunchKernelGGL(trie_bwd_chunk_kernel, dim3(h->n_chunks), dim3(256), 0, st, plan_dev(h), h->d_Pk,
                       h->d_Pv, h->d_Ck, h->d_Cv, D);
    pm.mark(3);
    auto reduce = [&](auto vw) {
      constexpr int VW = decltype(vw)::value;
      hipLaunchKernelGGL((trie_bwd_reduce_kernel<HD, VW>), dim3(h->n_tiles - 1), dim3(256), 0, st, plan_dev(h),
                         dk, dv, h->d_Pk, h->d_Pv, h->d_Ck, h->d_Cv, acc_dk, acc_dv, rope, h->cfg.n_heads);
    };
    // the widest column group that divides D (16-byte loads need VW >= 4)
    if (D % 512 == 0) reduce(std::integral_constant<int, 8>{});
    else if (D % 256 == 0) reduce(std::integral_constant<int, 4>{});
    else reduce(std::integral_constant<int, 2>{});
  } else {
    pm.mark(3);
  }
  launch_ctx<HD>(h, dk, dv, rope, st, ctx_wait);
  pm.mark(4);
}

template <typename Fn>
int dispatch_hd(int hd, Fn&& fn) {
  switch (hd) {
    case 4: fn(std::integral_constant<int, 4>{}); return AGPT_OK;
    case 8: fn(std::integral_constant<int, 8>{}); return AGPT_OK;
    case 16: fn(std::integral_constant<int, 16>{}); return AGPT_OK;
    case 32: fn(std::integral_constant<int, 32>{}); return AGPT_OK;
    case 64: fn(std::integral_constant<int, 64>{}); return AGPT_OK;
    default: return set_error(AGPT_ERR_UNSUPPORTED, "head_dim %d", hd);
  }
}

// Most scratch slots (up to `cap`) that keep the kernel's workgroups per CU
// at what it reaches with none; `base` is its LDS without scratch.
template <typename Fn>
int slots_at_full_occupancy(Fn fn, size_t base, size_t per_slot, int cap, size_t limit) {
  hipFuncAttributes fa{};
  if (hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(fn)) != hipSuccess) return 0;
  const size_t max_dyn = limit > fa.sharedSizeBytes ? limit - fa.sharedSizeBytes : 0;
  auto occ = [&](size_t lds) {
    if (lds > max_dyn) return 0;
    set_lds(fn, lds);
    return wg_per_cu(fn, lds, static_cast<int>(limit));
  };
  const int full = occ(base);
  if (full == 0) return 0;
  int s = 0;
  while (s < cap && occ(base + (s + 1) * per_slot) >= full) ++s;
  return s;
}

// Scratch slots of cut items (agpt_fast::kCutSteps): as many as the LDS left
// beside each streaming kernel holds without costing a workgroup per CU.
// Query items are shared by the forward and the query-side backward, and
// are cut for fp32 only. AGPT_ATTN_QSLOTS / AGPT_ATTN_KSLOTS cap the counts.
template <int HD, typename Tin>
void fit_scratch_t(agpt_attn_s* h) {
  with_124(h->hg, [&](auto hgc) {
    constexpr int HG = decltype(hgc)::value;
    const size_t lim = static_cast<size_t>(h->max_lds);
    const size_t fq = agpt_fast::q_scratch_bytes(HG, HD, true) / agpt_fast::kQSlots;
    const size_t bq = agpt_fast::q_scratch_bytes(HG, HD, false) / agpt_fast::kQSlots;
    const size_t kq = agpt_fast::k_scratch_bytes(HG, HD) / agpt_fast::kKSlots;
    int qs = 0;
    if (std::is_same<Tin, float>::value) {
      const int cap = std::min(agpt_fast::kQSlots, env_int("AGPT_ATTN_QSLOTS", agpt_fast::kQSlots));
      qs = std::min(
          slots_at_full_occupancy(agpt_fast::fwd_kernel<HD, Tin, HG, PlanDev>, h->fwd_lds, fq, cap, lim),
          slots_at_full_occupancy(agpt_fast::bwd_q_kernel<HD, Tin, HG, PlanDev, RopeArgs>, h->bq_lds, bq, cap,
                                  lim));
    }
    const int kcap = std::min(agpt_fast::kKSlots, env_int("AGPT_ATTN_KSLOTS", agpt_fast::kKSlots));
    const int ks =
        slots_at_full_occupancy(agpt_fast::bwd_kv_kernel<HD, Tin, HG, PlanDev, RopeArgs>, h->kv_lds, kq, kcap, lim);
    h->q_slots = qs;
    h->k_slots = ks;
    h->fwd_lds += qs * fq;
    h->bq_lds += qs * bq;
    h->kv_lds += ks * kq;
  });
}

void fit_scratch(agpt_attn_s* h) {
  if (h->cfg.head_dim == 16) {
    if (h->cfg.dtype == AGPT_DTYPE_F32) fit_scratch_t<16, float>(h);
    else fit_scratch_t<16, bf16_t>(h);
  } else if (h->cfg.head_dim == 32) {
    if (h->cfg.dtype == AGPT_DTYPE_F32) fit_scratch_t<32, float>(h);
    else fit_scratch_t<32, bf16_t>(h);
  }
  (void)hipGetLastError();  // a failed probe only means fewer slots
}

}  // namespace

namespace {
// A tensor pointer moved to the batch's row 0 (range plans place it at row
// row_off of the caller's tensors); rows are `bytes` long.
template <typename T>
T* at_batch(T* p, const agpt_attn_s* h, int64_t bytes) {
  using C = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return p ? reinterpret_cast<T*>(reinterpret_cast<C*>(p) + h->row_off * bytes) : p;
}
}  // namespace

extern "C" int agpt_attn_fwd(agpt_attn_handle h, const void* q, const void* k, const void* v,
                             void* o, float* lse, const agpt_attn_opts* opts) {
  if (!h) return set_error(AGPT_ERR_INVALID_ARG, "null handle");
  if (!h->planned) return set_error(AGPT_ERR_NO_PLAN, "agpt_attn_fwd before agpt_attn_plan");
  if (h->static_plan && !static_plan_current(h))
    return set_error(AGPT_ERR_NO_PLAN, "agpt_attn_fwd: a later agpt_attn_plan_static on this device took the scratch");
  if (!q || !k || !v || !o || !lse) return set_error(AGPT_ERR_INVALID_ARG, "null tensor");
  {
    const int64_t row = static_cast<int64_t>(h->cfg.n_heads) * h->cfg.head_dim *
                        (h->cfg.dtype == AGPT_DTYPE_F32 ? 4 : 2);
    q = at_batch(q, h, row);
    k = at_batch(k, h, row);
    v = at_batch(v, h, row);
    o = at_batch(o, h, row);
    lse = at_batch(lse, h, 4 * static_cast<int64_t>(h->cfg.n_heads));
  }
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return set_error(AGPT_ERR_INVALID_ARG, "tensors must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(lse) & 3u) != 0)  // read and written one float at a time
    return set_error(AGPT_ERR_INVALID_ARG, "lse must be 4-byte aligned");
  int rc = check_opts(opts);
  if (rc != AGPT_OK) return rc;
  HIP_TRY(hipSetDevice(h->device));
  const float scale = scale_of(h, opts);
  hipStream_t st = opts ? static_cast<hipStream_t>(opts->stream) : nullptr;
  ProfMarks pm;
  if (opts) pm = ProfMarks{opts->prof_events, opts->n_prof_events, st};
  rc = dispatch_hd(h->cfg.head_dim, [&](auto hdc) {
    constexpr int HD = decltype(hdc)::value;
    if (h->cfg.dtype == AGPT_DTYPE_F32) launch_fwd<HD, float>(h, q, k, v, o, lse, scale, st, pm);
    else launch_fwd<HD, bf16_t>(h, q, k, v, o, lse, scale, st, pm);
  });
  if (rc != AGPT_OK) return rc;
  HIP_TRY(hipGetLastError());
  return AGPT_OK;
}

extern "C" int agpt_attn_bwd(agpt_attn_handle h, const void* q, const void* k, const void* v,
                             const void* o, const float* lse, const void* d_o, float* dq,
                             float* dk, float* dv, const float* acc_dk, const float* acc_dv,
                             const agpt_attn_opts* opts) {
  if (!h) return set_error(AGPT_ERR_INVALID_ARG, "null handle");
  if (!h->planned) return set_error(AGPT_ERR_NO_PLAN, "agpt_attn_bwd before agpt_attn_plan");
  if (h->static_plan && !static_plan_current(h))
    return set_error(AGPT_ERR_NO_PLAN, "agpt_attn_bwd: a later agpt_attn_plan_static on this device took the scratch");
  if (!q || !k || !v || !o || !lse || !d_o || !dq || !dk || !dv)
    return set_error(AGPT_ERR_INVALID_ARG, "null tensor");
  {
    const int64_t D = static_cast<int64_t>(h->cfg.n_heads) * h->cfg.head_dim;
    const int64_t row = D * (h->cfg.dtype == AGPT_DTYPE_F32 ? 4 : 2);
    q = at_batch(q, h, row);
    k = at_batch(k, h, row);
    v = at_batch(v, h, row);
    o = at_batch(o, h, row);
    d_o = at_batch(d_o, h, row);
    lse = at_batch(lse, h, 4 * static_cast<int64_t>(h->cfg.n_heads));
    dq = at_batch(dq, h, 4 * D);
    dk = at_batch(dk, h, 4 * D);
    dv = at_batch(dv, h, 4 * D);
    acc_dk = at_batch(acc_dk, h, 4 * D);
    acc_dv = at_batch(acc_dv, h, 4 * D);
  }
  const void* ptrs[] = {q, k, v, o, d_o, dq, dk, dv, acc_dk, acc_dv};
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return set_error(AGPT_ERR_INVALID_ARG, "tensors must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(lse) & 3u) != 0)  // read one float at a time
    return set_error(AGPT_ERR_INVALID_ARG, "lse must be 4-byte aligned");
  int rc = check_opts(opts);
  if (rc != AGPT_OK) return rc;
  HIP_TRY(hipSetDevice(h->device));
  const float scale = scale_of(h, opts);
  hipStream_t st = opts ? static_cast<hipStream_t>(opts->stream) : nullptr;
  RopeArgs rope{nullptr, nullptr, 1};
  if (opts && opts->rope_cos) rope = RopeArgs{opts->rope_cos, opts->rope_sin, opts->rope_seq_len};
  ProfMarks pm;
  if (opts) pm = ProfMarks{opts->prof_events, opts->n_prof_events, st};
  const hipEvent_t ctx_wait = opts ? static_cast<hipEvent_t>(opts->ctx_wait) : nullptr;
  rc = dispatch_hd(h->cfg.head_dim, [&](auto hdc) {
    constexpr int HD = decltype(hdc)::value;
    if (h->cfg.dtype == AGPT_DTYPE_F32)
      launch_bwd<HD, float>(h, q, k, v, o, lse, d_o, dq, dk, dv, acc_dk, acc_dv, rope, scale, st, pm, ctx_wait);
    else
      launch_bwd<HD, bf16_t>(h, q, k, v, o, lse, d_o, dq, dk, dv, acc_dk, acc_dv, rope, scale, st, pm, ctx_wait);
  });
  if (rc != AGPT_OK) return rc;
  HIP_TRY(hipGetLastError());
  return AGPT_OK;
}

extern "C" int agpt_sync(void) {
  HIP_TRY(hipDeviceSynchronize());
  return AGPT_OK;
}
