// trie_deep.h — head_dim 64 trie-attention kernels for deep prefixes
// (included by trie_attn.hip after trie_block.h).
//
// The block kernels of trie_block.h keep a tile's whole key set (the
// prefix path of its first row and its own rows) in LDS. At head_dim 64 a
// deep trie's key set is up to 255 + 64 rows, 80-110 KB of K and V per
// workgroup: one workgroup per CU, one wave per SIMD, and every block pair
// waits on the latency of the one before it. Here the key set streams:
//
//   query side (forward; backward dQ): a workgroup takes one (tile, head);
//     each of its four waves owns one 16-row query block, whose Q (and dO)
//     slices sit in registers. The tile's keys (prefix rows in depth order,
//     then the tile rows) pass through a double-buffered LDS ring in chunks
//     of 64: while the waves work on one chunk, the next is loaded from
//     memory by row index (the plan's prefix list) into registers and
//     written to the other buffer at the chunk's end.
//   key side (backward dK, dV): the tile's Q and dO rows are staged in LDS;
//     each wave takes key blocks of 16 keys, loads their K and V slices
//     straight into registers, and walks the query blocks that see them.
//
// LDS per workgroup is 37 KB (bf16 ring) or 18 KB (bf16 staged rows)
// instead of 80-110 KB; every tile in it is row-major, and the bf16
// operands that a product needs transposed are read with ds_read_b64_tr_b16
// (read_tr). The block pairs, masks and lane layouts are those of
// trie_block.h: 16x16 tiles on the matrix instructions, and per key the
// interval of tile rows that see it (in DFS preorder the rows below a key
// are consecutive). The key side leaves the partials bwd_kv_kernel leaves
// (a prefix key's share over the tile in Pk/Pv at row pref_off[t] +
// depth - 1; an open tile row's share in dK/dV), which
// trie_bwd_chunk_kernel and trie_bwd_reduce_kernel finish.
//
// A workgroup takes a unit of one tile and hpu of its heads (all of them
// when the plan has tiles enough to fill the chip, else one) and runs the
// heads one after the other: the tables are built once per unit, and the
// next head's operands are in flight while the current head is worked on.
// Units are claimed from one counter per kernel; the claim for the next
// unit is sent at the start of the current one. No result depends on which
// workgroup takes a unit.
#pragma once

namespace agpt_deep {

using namespace agpt;
using agpt_blk::group_max;
using agpt_blk::group_sum;
using agpt_blk::in_interval;
using agpt_blk::kBlk;
using agpt_blk::kRescaleLog2;
using agpt_blk::ld1;
using agpt_blk::mfma16;
using agpt_blk::pack_bf16;
using agpt_blk::Slice;
using agpt_blk::slice_dot;
using agpt_fast::f4;
using agpt_fast::u4;
using agpt_fast::uniform;

constexpr int kTile = 64;
constexpr int kThreads = 256;
constexpr int kChunk = 64;  // keys per streamed chunk: one 16-key block per wave-sized step
constexpr int kKeyCap = (kMaxDepth - 1 + kTile + kChunk - 1) / kChunk * kChunk;
// Key blocks per wave of the carry key side with its sums in registers:
// kRegItersDeep blocks per wave (key slots 0 .. 16 * 4 * kRegItersDeep - 1),
// the default; or, on request, every key slot of a tile of a plan to depth
// kRegDepth (prefix_cap + 64 keys in 4 kRegIters blocks of 16), which at
// the register limit spills inside the key-block loop.
constexpr int kRegIters = 3;
constexpr int kRegDepth = 4 * kRegIters * 16 - kTile;  // 128
constexpr int kRegItersDeep = 2;
// Running max of a query before it has seen a key: finite, so that exp2 of
// a masked score (-inf) minus it is 0, never NaN.
constexpr float kNoMax = -1.0e30f;

__host__ __device__ constexpr int row_stride(int hd, int elem) { return hd + 16 / elem; }
// One buffer of the query side's key ring: K rows, then V rows [kChunk][WS].
// (bf16 operands of the second products, P·V and dS·K, are read from the
// row-major tiles with read_tr.)
__host__ __device__ constexpr size_t ring_buf_elems(int hd, int elem) {
  return 2 * static_cast<size_t>(kChunk) * row_stride(hd, elem);
}
// Dynamic LDS: the query-side ring (two buffers) or the key side's staged
// rows [Q, dO][kTile][WS] (bf16 operands of P^T·dO and dS^T·Q read from
// them transposed, read_tr).
__host__ __device__ constexpr size_t ring_lds_bytes(int hd, int elem) {
  return 2 * ring_buf_elems(hd, elem) * elem;
}
__host__ __device__ constexpr size_t rows_lds_bytes(int hd, int elem) {
  return static_cast<size_t>(2 * kTile) * row_stride(hd, elem) * elem;
}

// The A operand of v_mfma_f32_16x16x16_bf16 for the 16 x 16 block
// M[m][k] = R[k0 + k][m0 + m] of a row-major bf16 tile R in LDS (row stride
// ws elements, 8-byte aligned rows): lane (l = lane % 16, g = lane / 16)
// needs R[k0 + 4g + i][m0 + l], i = 0 .. 3. ds_read_b64_tr_b16 transposes
// within each 16-lane group: lane l receives element l % 4 of the 8 bytes
// read by lane 4i + l / 4 of its group, so lane l reads
// R[k0 + 4g + l / 4][m0 + 4 (l % 4) ..]. One read per operand where a gather
// of four rows takes four 2-byte reads and two packing instructions.
__device__ __forceinline__ agpt_blk::bf16x4_bits read_tr(const bf16_t* R, int ws, int k0, int m0, int lane) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  const int l = lane & 15, g = lane >> 4;
  const bf16_t* p = R + (k0 + 4 * g + (l >> 2)) * ws + m0 + 4 * (l & 3);
  const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(p));
  return __builtin_bit_cast(agpt_blk::bf16x4_bits, v);
}
__device__ __forceinline__ f4 mfma_a_bf16(agpt_blk::bf16x4_bits a, uint2 wb, f4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, __builtin_bit_cast(agpt_blk::bf16x4_bits, wb), acc, 0, 0, 0);
}
// acc + a0·b0 + a1·b1 (each as in mfma_a_bf16) in one 32-deep step, which
// takes the time of one 16-deep step: a lane's eight reduction elements are
// its four of a0 (b0) then its four of a1 (b1) in both operands, so each
// element of A meets its own element of B.
__device__ __forceinline__ f4 mfma_a2_bf16(agpt_blk::bf16x4_bits a0, agpt_blk::bf16x4_bits a1, uint2 b0, uint2 b1,
                                           f4 acc) {
  typedef __attribute__((ext_vector_type(8))) __bf16 b8;
  const uint2 x0 = __builtin_bit_cast(uint2, a0), x1 = __builtin_bit_cast(uint2, a1);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, uint4{x0.x, x0.y, x1.x, x1.y}),
                                                 __builtin_bit_cast(b8, uint4{b0.x, b0.y, b1.x, b1.y}), acc, 0, 0,
                                                 0);
}

// The tile's key list and row tables. Keys 0 .. A-1 are the prefix rows
// (depth 1 .. A), keys A .. A+ntile-1 the tile rows; the list is padded to
// whole chunks with empty keys that name row s (finite data, never live).
// The query side keeps only the key list (KeyTables, 2.7 KB, so that four
// forward workgroups fit a CU); the key side adds the row tables.
struct alignas(16) KeyTables {
  alignas(16) int32_t kint[kKeyCap];  // per key: lo | len << 16, the tile rows [lo, lo + len) that see it
  int32_t krow[kKeyCap];  // per key: its row in the tensors (negative: a context row of a range plan)
  alignas(16) int32_t blo[kKeyCap / kBlk];  // per key block: least lo of its live keys (kTile if none)
  alignas(16) int32_t bhi[kKeyCap / kBlk];  // per key block: greatest lo + len
  int32_t next[2];       // claims, alternating by unit
};
struct alignas(16) Tables : KeyTables {
  int32_t pend[kKeyCap];  // per prefix key: its subtree end (rows of the plan)
  int32_t rdep[kTile];   // depth of the tile rows
  int32_t rend[kTile];   // subtree end of the tile rows
  alignas(16) float l2[kTile];  // lse * log2(e) of the tile rows (key side)
  alignas(16) float dl[kTile];  // δ of the tile rows (key side)
};

// The tile of unit t; fills its key list and tables.
struct Unit {
  int t, s, ntile, A, poff, nk, nch;
};

// Fills the tables of tile t, whose prefix list is entries poff .. poff+A-1
// of the plan's; src gives the prefix rows and their subtree ends (entry j
// of the tile's list) and the tile rows' subtree ends and depths.
template <typename TB, typename Src>
__device__ __forceinline__ Unit fill_tables(TB& tb, int t, int64_t T, int poff, int A, bool row_tabs,
                                            const Src& src) {
  constexpr bool kRows = std::is_same<TB, Tables>::value;  // the key side's row tables
  Unit w;
  w.t = t;
  w.s = w.t * kTile;
  w.ntile = static_cast<int>(min(static_cast<int64_t>(kTile), T - w.s));
  w.poff = poff;
  w.A = A;
  w.nk = w.A + w.ntile;
  w.nch = (w.nk + kChunk - 1) / kChunk;
  const int tid = threadIdx.x;
  for (int j = tid; j < w.nch * kChunk; j += kThreads) {
    int iv = 0, row = w.s;
    if (j < w.A) {
      row = src.pre(j);
      const int e = src.pend(j);
      iv = min(e - w.s, w.ntile) << 16;
      if constexpr (kRows) {
        if (row_tabs) tb.pend[j] = e;
      }
    } else if (j < w.nk) {
      const int r = j - w.A;
      row = w.s + r;
      const int e = src.end(r);
      iv = r | ((min(e - w.s, w.ntile) - r) << 16);
      if constexpr (kRows) {
        if (row_tabs) {
          tb.rdep[r] = src.dep(r);
          tb.rend[r] = e;
        }
      }
    }
    tb.kint[j] = iv;
    tb.krow[j] = row;
  }
  __syncthreads();
  for (int b = tid; b < w.nch * (kChunk / kBlk); b += kThreads) {
    int lo = kTile, hi = 0;
    for (int x = 0; x < kBlk; ++x) {
      const int iv = tb.kint[b * kBlk + x];
      const int len = iv >> 16;
      if (len > 0) {
        lo = min(lo, iv & 0xffff);
        hi = max(hi, (iv & 0xffff) + len);
      }
    }
    tb.blo[b] = lo;
    tb.bhi[b] = hi;
  }
  __syncthreads();
  return w;
}

// The plan's tables in global memory as the source.
template <typename PlanT>
struct PlanSrc {
  const PlanT& pl;
  int poff, s;
  __device__ __forceinline__ int pre(int j) const { return pl.prefix[poff + j]; }
  __device__ __forceinline__ int pend(int j) const { return pl.pref_end[poff + j]; }
  __device__ __forceinline__ int end(int r) const { return pl.end[s + r]; }
  __device__ __forceinline__ int dep(int r) const { return pl.depth[s + r]; }
};

template <typename PlanT, typename TB>
__device__ __forceinline__ Unit build_tables(const PlanT& pl, TB& tb, int t, bool row_tabs) {
  const int poff = pl.pref_off[t];
  const int A = pl.pref_off[t + 1] - poff;
  return fill_tables(tb, t, pl.T, poff, A, row_tabs, PlanSrc<PlanT>{pl, poff, t * kTile});
}

// A tile's table inputs copied into LDS ahead of use (RawTabs::gather), as
// the source of fill_tables: prefix rows and their subtree ends, then the
// tile rows' subtree ends and depths.
struct RawTabs {
  int32_t* base;  // [2][kKeyCap] prefix rows, subtree ends; [2][kTile] row ends, depths
  __device__ __forceinline__ int pre(int j) const { return base[j]; }
  __device__ __forceinline__ int pend(int j) const { return base[kKeyCap + j]; }
  __device__ __forceinline__ int end(int r) const { return base[2 * kKeyCap + r]; }
  __device__ __forceinline__ int dep(int r) const { return base[2 * kKeyCap + kTile + r]; }
  static constexpr size_t kBytes = (2 * kKeyCap + 2 * kTile) * sizeof(int32_t);
  // Issues the copies of tile t's inputs (prefix entries poff .. poff+A-1)
  // with direct-to-LDS loads: the waves take 64-entry segments in turn; lane
  // L of a segment writes entry 64 seg + L (its source index clamped to the
  // list, so every address is in bounds). They complete under vmcnt: wait
  // for them (wait_loads) before the barrier after which they are read.
  template <typename PlanT>
  __device__ __forceinline__ void gather(const PlanT& pl, int t, int poff, int A, int wave, int lane) const {
    const int64_t s = static_cast<int64_t>(t) * kTile;
    const int last = static_cast<int>(min(static_cast<int64_t>(kTile), pl.T - s)) - 1;
    const int nseg = (A + 63) / 64;
    typedef __attribute__((address_space(3))) void* lds_ptr;
    for (int k = wave; k < 2 * nseg + 2; k += kThreads / 64) {
      if (k < 2 * nseg) {
        const int seg = k >> 1;
        const int j = min(64 * seg + lane, A - 1);
        const int32_t* src = (k & 1) ? pl.pref_end : pl.prefix;
        int32_t* dst = base + ((k & 1) ? kKeyCap : 0) + 64 * seg;
        __builtin_amdgcn_global_load_lds(src + poff + j, (lds_ptr)(dst), 4, 0, 0);
      } else {
        const int32_t* src = (k & 1) ? pl.depth : pl.end;
        int32_t* dst = base + 2 * kKeyCap + ((k & 1) ? kTile : 0);
        __builtin_amdgcn_global_load_lds(src + s + min(lane, last), (lds_ptr)(dst), 4, 0, 0);
      }
    }
  }
};

// Waits until every vector-memory load of this wave has returned (vmcnt 0,
// expcnt and lgkmcnt left alone). Placed after the loads of a unit's
// register slices, before its step loop: the compiler's wait bookkeeping
// then knows the slices are in at the loop head. Without it the first use
// of a slice inside the loop carries a vmcnt(0) wait on every pass, which
// also waits for the key-ring prefetch issued at the top of that pass.
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// The tile of claim i of a query-side or per-tile key-side kernel.
template <typename PlanT>
__device__ __forceinline__ int tile_of(const PlanT& pl, int i) {
  return pl.tile_order ? pl.tile_order[i] : i;
}

// Claims of the query-side kernels (thread 0 calls next()). One counter over
// all units, or, with pl.xcd_claims, kXcds counters at ctr[x]: XCD x (the
// workgroups b with b % kXcds == x, which the dispatcher deals round robin
// over the XCDs) takes units [n x / kXcds, n (x + 1) / kXcds) in order, so
// the tiles in flight on one XCD are neighbours whose prefix rows its L2
// already holds; a range used up is left for the next XCD's, at most kXcds
// claims that fail per workgroup. Returns n when every range is used up.
constexpr int kXcdCtr = 3 * kMaxHeads;  // first per-XCD counter in pl.sched
struct Claims {
  int* ctr;
  int64_t n;
  int xcd, probe;
  bool ranged;
  __device__ int next() {
    if (!ranged) return atomicAdd(ctr, 1);
    while (probe < agpt_fast::kXcds) {
      const int x = (xcd + probe) % agpt_fast::kXcds;
      const int64_t lo = n * x / agpt_fast::kXcds, hi = n * (x + 1) / agpt_fast::kXcds;
      const int k = atomicAdd(ctr + x, 1);
      if (lo + k < hi) return static_cast<int>(lo + k);
      ++probe;
    }
    return static_cast<int>(n);
  }
};
template <typename PlanT>
__device__ __forceinline__ Claims make_claims(const PlanT& pl, int kernel, int64_t n_units) {
  Claims q;
  q.ranged = pl.xcd_claims != 0;
  q.ctr = pl.sched + (q.ranged ? kXcdCtr + agpt_fast::kXcds * kernel : kernel);
  q.n = n_units;
  q.xcd = static_cast<int>(blockIdx.x % agpt_fast::kXcds);
  q.probe = 0;
  return q;
}

// The key blocks of chunk ch with a live pair for query block i (rows 16i ..
// 16i+15): bit bl for key block 4 ch + bl, a wave-uniform value. One pair of
// 16-byte reads per chunk, and a scalar bit test per block, where a test per
// block would make two dependent LDS round trips and an exec-mask branch.
static_assert(kChunk / kBlk == 4, "four key blocks per chunk");
__device__ __forceinline__ int chunk_live(const KeyTables& tb, int ch, int i) {
  const int4 lo = *reinterpret_cast<const int4*>(tb.blo + 4 * ch);
  const int4 hi = *reinterpret_cast<const int4*>(tb.bhi + 4 * ch);
  const int r0 = kBlk * i, r1 = r0 + kBlk;
  const int m = static_cast<int>(r0 < hi.x && r1 > lo.x) | static_cast<int>(r0 < hi.y && r1 > lo.y) << 1 |
                static_cast<int>(r0 < hi.z && r1 > lo.z) << 2 | static_cast<int>(r0 < hi.w && r1 > lo.w) << 3;
  return uniform(m);
}

// Whether query block i (rows 16i .. 16i+15) has a live pair with key block b.
__device__ __forceinline__ bool block_live(const KeyTables& tb, int b, int i) {
  return kBlk * i < uniform(tb.bhi[b]) && kBlk * i + kBlk > uniform(tb.blo[b]);
}

// The double-buffered key ring of the query side: chunk c of the tile's key
// list, K and V slices of one head; per buffer K rows [kChunk][WS], then V
// rows [kChunk][WS].
template <int HD, typename Tin>
struct KeyRing {
  static constexpr int EPC = 16 / static_cast<int>(sizeof(Tin));  // elements per 16-byte piece
  static constexpr int WS = row_stride(HD, sizeof(Tin));
  static constexpr int PIECES = HD / EPC;    // pieces per key slice
  static constexpr int PER_T = kChunk * PIECES;  // pieces per tensor per chunk
  static constexpr int PER = 2 * PER_T / kThreads;
  static constexpr int BUF = static_cast<int>(ring_buf_elems(HD, sizeof(Tin)));
  static_assert(PER_T % kThreads == 0, "whole rounds of the workgroup per tensor");
  Tin* base;
  u4 r[PER];
  __device__ __forceinline__ Tin* ks(int buf) const { return base + buf * BUF; }
  __device__ __forceinline__ Tin* vs(int buf) const { return base + buf * BUF + kChunk * WS; }
  __device__ __forceinline__ void load(const KeyTables& tb, const Tin* K, const Tin* V, int D, int h, int c) {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int ten = k * kThreads / PER_T;  // a constant once unrolled
      const int j = static_cast<int>(threadIdx.x) + k * kThreads - ten * PER_T;
      const int key = j / PIECES;
      const int64_t row = tb.krow[c * kChunk + key];
      r[k] = *reinterpret_cast<const u4*>((ten ? V : K) + row * D + h * HD + (j % PIECES) * EPC);
    }
  }
  __device__ __forceinline__ void store(int buf) {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int ten = k * kThreads / PER_T;
      const int j = static_cast<int>(threadIdx.x) + k * kThreads - ten * PER_T;
      const int key = j / PIECES, d0 = (j % PIECES) * EPC;
      *reinterpret_cast<u4*>((ten ? vs(buf) : ks(buf)) + key * WS + d0) = r[k];
    }
  }
};

// ---------------------------------------------------------------------------
// Forward: O and lse. A workgroup takes a tile and runs its heads one after
// the other as one stream of key chunks (the key list is the same for every
// head): the chunk after the current one, in the next head or not, is in
// flight while the current one is worked on, and the next head's Q slices
// are fetched during the current head's last chunk. S^T = K Q^T puts query
// c in lane column c (keys 4g .. 4g+3 in its registers); online softmax
// with the lazy rescale of trie_block.h; O^T += V^T P^T (V^T blocks read
// transposed from the ring's V rows).
// ---------------------------------------------------------------------------
template <int HD, typename Tin, typename PlanT>
__global__ __launch_bounds__(kThreads) void fwd_kernel(PlanT pl, const Tin* __restrict__ Q,
                                                       const Tin* __restrict__ K, const Tin* __restrict__ V,
                                                       Tin* __restrict__ O, float* __restrict__ lse, int H,
                                                       int hpu, float scale) {
  constexpr int KD = HD / 4;
  constexpr int MT = HD / 16;
  using Ring = KeyRing<HD, Tin>;
  constexpr int WS = Ring::WS;
  __shared__ KeyTables tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  Ring ring;
  ring.base = reinterpret_cast<Tin*>(dyn);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const float qscale = scale * kLog2e;
  // bf16 scores come unscaled (the fp32 operands are scaled once): the
  // scale goes into the exponent's multiply-add.
  const float sfac = Slice<Tin, HD / 4>::kPre ? 1.0f : qscale;
  const int ngr = H / hpu;  // head groups: unit u = (tile u / ngr, heads hpu * (u % ngr) ..)
  const int64_t n_units = static_cast<int64_t>(pl.n_tiles) * ngr;
  Claims claims = make_claims(pl, 0, n_units);
  if (threadIdx.x == 0) tb.next[1] = claims.next();
  __syncthreads();
  int u = uniform(tb.next[1]);
  for (int par = 0; u < n_units; par ^= 1) {
    if (threadIdx.x == 0) tb.next[par] = claims.next();
    const int h0 = (u % ngr) * hpu;
    const Unit w = build_tables(pl, tb, tile_of(pl, u / ngr), false);
    const int q = kBlk * wave + c;  // this lane's query row in the tile
    const int64_t qbase = (w.s + min(q, w.ntile - 1)) * static_cast<int64_t>(D) + KD * g;
    Slice<Tin, KD> qf, qn;
    qf.load(Q + qbase + h0 * HD);
    ring.load(tb, K, V, D, h0, 0);
    // The live key blocks of every chunk for this wave's query block, 4 bits
    // per chunk (nch <= 5), once per unit.
    uint32_t lm_all = 0;
    for (int ch = 0; ch < w.nch; ++ch) lm_all |= static_cast<uint32_t>(chunk_live(tb, ch, wave)) << (4 * ch);
    wait_loads();
    ring.store(0);
    __syncthreads();
    qf.scale(qscale);
    float m = kNoMax, l = 0.0f;
    f4 o[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) o[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    const int nsteps = hpu * w.nch;
    __builtin_assume(nsteps > 0);  // no guard block for the slice loads to sink into
    // Step st is chunk ch of head h0 + hl; the counters advance at its end.
    int hl = 0, ch = 0;
    for (int st = 0; st < nsteps; ++st) {
      __builtin_amdgcn_s_setprio(0);
      const int h = h0 + hl;
      const bool last = ch + 1 == w.nch;
      const int nxc = last ? 0 : ch + 1;
      const int nxh = last ? hl + 1 : hl;
      const bool more = st + 1 < nsteps;
      if (more) ring.load(tb, K, V, D, h0 + nxh, nxc);
      if (last && hl + 1 < hpu) qn.load(Q + qbase + (h + 1) * HD);
      const Tin* Ks = ring.ks(st & 1);
      const Tin* Vs = ring.vs(st & 1);
      const int lmask = (lm_all >> (4 * ch)) & 15;
#pragma unroll
      for (int bl = 0; bl < kChunk / kBlk; ++bl) {
        const int b = ch * (kChunk / kBlk) + bl;
        if (!((lmask >> bl) & 1)) continue;
        const int4 iv = *reinterpret_cast<const int4*>(tb.kint + kBlk * b + 4 * g);
        const bool live[4] = {in_interval(q, iv.x), in_interval(q, iv.y), in_interval(q, iv.z),
                              in_interval(q, iv.w)};
        Slice<Tin, KD> kf;
        kf.load(Ks + (kBlk * bl + c) * WS + KD * g);
        f4 sv = slice_dot(kf, qf, f4{0.0f, 0.0f, 0.0f, 0.0f});  // key 16b+4g+r against query q
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = live[r] ? sv[r] : -__builtin_inff();
        // The scale (> 0) goes on the maximum, and into the exponent's
        // multiply-add.
        const float lmx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])) * sfac;
        if (__any(lmx > m + kRescaleLog2)) {
          const float mx = group_max(lmx);
          const bool resc = mx > m + kRescaleLog2;
          const float a = resc ? fast_exp2(m - mx) : 1.0f;
          m = resc ? mx : m;
          l *= a;
#pragma unroll
          for (int j = 0; j < MT; ++j) o[j] *= a;
        }
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = fast_exp2(__builtin_fmaf(sc[r], sfac, -m));  // masked: exp2(-inf) = 0
          l += p[r];
        }
        if constexpr (sizeof(Tin) == 2) {
          const uint2 pw = pack_bf16(p);  // V^T block: dims 16j .., keys 16bl ..
#pragma unroll
          for (int j = 0; j < MT; ++j) o[j] = mfma_a_bf16(read_tr(Vs, WS, kBlk * bl, kBlk * j, lane), pw, o[j]);
        } else {
#pragma unroll
          for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              o[j] = mfma16(ld1(Vs + (kBlk * bl + 4 * g + r) * WS + kBlk * j + c), p[r], o[j]);
        }
      }
      // the next chunk's ring store and the step's barrier ahead of the
      // other workgroups' products
      __builtin_amdgcn_s_setprio(3);
      if (more) ring.store((st + 1) & 1);
      if (last) {
        if (q < w.ntile) {
          const int64_t row = static_cast<int64_t>(w.s) + q;
          const float le = group_sum(l);
          const float inv = __builtin_amdgcn_rcpf(le);
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            float v[4] = {o[j][0] * inv, o[j][1] * inv, o[j][2] * inv, o[j][3] * inv};
            store_vec<4>(O + row * D + h * HD + kBlk * j + 4 * g, v);
          }
          if (g == 0) lse[row * H + h] = (m + fast_log2(le)) * kLn2;
        }
        if (hl + 1 < hpu) {  // the next head starts from zero
          qf = qn;
          qf.scale(qscale);
          m = kNoMax;
          l = 0.0f;
#pragma unroll
          for (int j = 0; j < MT; ++j) o[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
      hl = nxh;
      ch = nxc;
      __syncthreads();
    }
    u = uniform(tb.next[par]);
  }
}

// ---------------------------------------------------------------------------
// Backward, query side: δ and dQ, a tile's heads as one stream of key chunks
// as in the forward. fp32 inputs: δ = dO·O from the O rows. bf16 inputs: O
// is a rounded output, so δ = Σ_j w_j dO·v_j is recomputed over the path in
// fp32 (batched_depth_backward.cr:637-646): each head makes one pass over
// the key chunks for δ, then one for dQ. δ goes to Dl [T, H] for the key
// side; dQ gets the inverse rotation at the query's depth.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, typename PlanT, typename RopeT, bool kOnePass = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kOnePass ? 3 : 2))) void bwd_q_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const Tin* __restrict__ O, const float* __restrict__ lse, const Tin* __restrict__ dO,
    float* __restrict__ dQ, float* __restrict__ Dl, RopeT rope, int H, int hpu, float scale) {
  // kOnePass (bf16): one pass over the key chunks. With a_j = w_j dw_j,
  // dQ = scale (Σ_j a_j k_j − δ Σ_j w_j k_j) and δ = Σ_j a_j, so the pass
  // accumulates δ and both sums and combines them at the end. The two sums
  // nearly cancel where the dw_j are close to δ, so their bf16 operands
  // a_j and w_j each go in as a high and a low bf16 part (two products per
  // output tile, 2^-17 relative per operand) instead of dS rounded once.
  static_assert(!kOnePass || sizeof(Tin) == 2, "the fp32 inputs take δ = dO·O in one pass already");
  constexpr int KD = HD / 4;
  constexpr int MT = HD / 16;
  constexpr bool kDeltaFromO = sizeof(Tin) == sizeof(float);
  constexpr int NP = kDeltaFromO || kOnePass ? 1 : 2;  // passes over the key chunks per head
  using Ring = KeyRing<HD, Tin>;
  constexpr int WS = Ring::WS;
  __shared__ KeyTables tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  Ring ring;
  ring.base = reinterpret_cast<Tin*>(dyn);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const float qscale = scale * kLog2e;
  // bf16 scores come unscaled (the fp32 operands are scaled once): the
  // scale goes into the exponent's multiply-add.
  const float sfac = Slice<Tin, HD / 4>::kPre ? 1.0f : qscale;
  const int ngr = H / hpu;  // head groups: unit u = (tile u / ngr, heads hpu * (u % ngr) ..)
  const int64_t n_units = static_cast<int64_t>(pl.n_tiles) * ngr;
  Claims claims = make_claims(pl, 1, n_units);
  if (threadIdx.x == 0) tb.next[1] = claims.next();
  __syncthreads();
  int u = uniform(tb.next[1]);
  for (int par = 0; u < n_units; par ^= 1) {
    if (threadIdx.x == 0) tb.next[par] = claims.next();
    const int h0 = (u % ngr) * hpu;
    const Unit w = build_tables(pl, tb, tile_of(pl, u / ngr), false);
    const int q = kBlk * wave + c;
    const int64_t qrow = w.s + min(q, w.ntile - 1);
    const int64_t qbase = qrow * D + KD * g;
    // This lane's query of head h: Q, dO slices, lse (and O for δ, fp32).
    // lse is taken to log2 units where it is first used, not where it is
    // fetched, so that the next head's fetch does not wait for its load.
    Slice<Tin, KD> qf, gf, qn, gn;
    float l2, l2n = 0.0f, dl = 0.0f;
    float ov[kDeltaFromO ? KD : 1], on[kDeltaFromO ? KD : 1];
    auto fetch = [&](int h, Slice<Tin, KD>& a, Slice<Tin, KD>& b, float& le, float (&oo)[kDeltaFromO ? KD : 1]) {
      a.load(Q + qbase + h * HD);
      b.load(dO + qbase + h * HD);
      le = lse[qrow * H + h];
      if constexpr (kDeltaFromO) load_vec<KD>(reinterpret_cast<const float*>(O) + qbase + h * HD, oo);
    };
    fetch(h0, qf, gf, l2, ov);
    const int qdep = pl.depth[qrow];
    ring.load(tb, K, V, D, h0, 0);
    // The live key blocks of every chunk for this wave's query block, 4 bits
    // per chunk (nch <= 5), once per unit.
    uint32_t lm_all = 0;
    for (int ch = 0; ch < w.nch; ++ch) lm_all |= static_cast<uint32_t>(chunk_live(tb, ch, wave)) << (4 * ch);
    wait_loads();
    l2 *= kLog2e;
    ring.store(0);
    __syncthreads();
    // Scores and dO·v of key block bl of the buffer: register r holds key
    // 16b+4g+r against query q.
    auto scores = [&](const Tin* Ks, const Tin* Vs, int bl, f4& sv, f4& tv) {
      Slice<Tin, KD> kf, vf;
      kf.load(Ks + (kBlk * bl + c) * WS + KD * g);
      vf.load(Vs + (kBlk * bl + c) * WS + KD * g);
      sv = slice_dot(kf, qf, f4{0.0f, 0.0f, 0.0f, 0.0f});
      tv = slice_dot(vf, gf, f4{0.0f, 0.0f, 0.0f, 0.0f});
    };
    auto mask = [&](int b, bool (&live)[4]) {
      const int4 iv = *reinterpret_cast<const int4*>(tb.kint + kBlk * b + 4 * g);
      live[0] = in_interval(q, iv.x);
      live[1] = in_interval(q, iv.y);
      live[2] = in_interval(q, iv.z);
      live[3] = in_interval(q, iv.w);
    };
    f4 dq[MT], dqw[kOnePass ? MT : 1];  // kOnePass: Σ a_j k_j and Σ w_j k_j
    float acc;
    // A head's state at its first step.
    auto start_head = [&]() {
      qf.scale(qscale);
      acc = 0.0f;
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        dq[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (kOnePass) dqw[j] = dq[j];
      }
      if constexpr (kDeltaFromO) {
        float x = 0.0f;
#pragma unroll
        for (int j = 0; j < KD; ++j) x += gf.v[j] * ov[j];
        dl = group_sum(x);
      }
    };
    start_head();
    const int nsteps = hpu * NP * w.nch;
    __builtin_assume(nsteps > 0);
    // Step st is chunk ch of pass `pass` (0: δ, bf16 two-pass only; 1: dQ)
    // of head h0 + hl; the counters advance at its end.
    int hl = 0, pass = NP == 2 ? 0 : 1, ch = 0;
    for (int st = 0; st < nsteps; ++st) {
      __builtin_amdgcn_s_setprio(0);
      const int h = h0 + hl;
      const bool pend = ch + 1 == w.nch;  // the pass's last chunk
      const bool last = pend && pass == 1;  // the head's last step
      const int nxc = pend ? 0 : ch + 1;
      const int nxp = pend ? (last ? (NP == 2 ? 0 : 1) : 1) : pass;
      const int nxh = last ? hl + 1 : hl;
      const bool more = st + 1 < nsteps;
      if (more) ring.load(tb, K, V, D, h0 + nxh, nxc);
      if (last && hl + 1 < hpu) fetch(h + 1, qn, gn, l2n, on);
      const Tin* Ks = ring.ks(st & 1);
      const Tin* Vs = ring.vs(st & 1);
      const int lmask = (lm_all >> (4 * ch)) & 15;
#pragma unroll
      for (int bl = 0; bl < kChunk / kBlk; ++bl) {
        const int b = ch * (kChunk / kBlk) + bl;
        if (!((lmask >> bl) & 1)) continue;
        bool live[4];
        mask(b, live);
        f4 sv, tv;
        scores(Ks, Vs, bl, sv, tv);
        if (pass == 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc += fast_exp2(live[r] ? __builtin_fmaf(sv[r], sfac, -l2) : -__builtin_inff()) * tv[r];
          continue;
        }
        // bf16: the K^T blocks of the dQ product read before the softmax,
        // so the reads overlap it.
        agpt_blk::bf16x4_bits tkv[sizeof(Tin) == 2 ? MT : 1];
        if constexpr (sizeof(Tin) == 2) {
#pragma unroll
          for (int j = 0; j < MT; ++j) tkv[j] = read_tr(Ks, WS, kBlk * bl, kBlk * j, lane);
          __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (kOnePass) {
          float pw[4], aw[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {  // masked: exp2(-inf) = 0
            pw[r] = fast_exp2(live[r] ? __builtin_fmaf(sv[r], sfac, -l2) : -__builtin_inff());
            aw[r] = pw[r] * tv[r];
            acc += aw[r];
          }
          const uint2 ph = pack_bf16(pw), ah = pack_bf16(aw);
          const float plo[4] = {pw[0] - __uint_as_float(ph.x << 16), pw[1] - __uint_as_float(ph.x & 0xffff0000u),
                                pw[2] - __uint_as_float(ph.y << 16), pw[3] - __uint_as_float(ph.y & 0xffff0000u)};
          const float alo[4] = {aw[0] - __uint_as_float(ah.x << 16), aw[1] - __uint_as_float(ah.x & 0xffff0000u),
                                aw[2] - __uint_as_float(ah.y << 16), aw[3] - __uint_as_float(ah.y & 0xffff0000u)};
          const uint2 pl2 = pack_bf16(plo), al2 = pack_bf16(alo);
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            dq[j] = mfma_a2_bf16(tkv[j], tkv[j], ah, al2, dq[j]);  // high and low bf16 parts in one step
            dqw[j] = mfma_a2_bf16(tkv[j], tkv[j], ph, pl2, dqw[j]);
          }
          continue;
        }
        float ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)  // masked: exp2(-inf) = 0, no branch per pair
          ds[r] = fast_exp2(live[r] ? __builtin_fmaf(sv[r], sfac, -l2) : -__builtin_inff()) * (tv[r] - dl) * scale;
        if constexpr (sizeof(Tin) == 2) {  // dS rounded to bf16, one 16-deep step per output tile
          const uint2 dw = pack_bf16(ds);
#pragma unroll
          for (int j = 0; j < MT; ++j) dq[j] = mfma_a_bf16(tkv[j], dw, dq[j]);
        } else {
#pragma unroll
          for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              dq[j] = mfma16(ld1(Ks + (kBlk * bl + 4 * g + r) * WS + kBlk * j + c), ds[r], dq[j]);
        }
      }
      if (pass == 0 && ch + 1 == w.nch) dl = group_sum(acc);
      // the next chunk's ring store and the step's barrier ahead of the
      // other workgroups' products
      __builtin_amdgcn_s_setprio(3);
      if (more) ring.store((st + 1) & 1);
      if (last) {
        if constexpr (kOnePass) {
          dl = group_sum(acc);
#pragma unroll
          for (int j = 0; j < MT; ++j) dq[j] = (dq[j] - dl * dqw[j]) * scale;
        }
        if (q < w.ntile) {
          const int64_t row = static_cast<int64_t>(w.s) + q;
          const int pos = rope.cos_t ? rope_pos(qdep, rope.seq_len) : 0;
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            float v[4] = {dq[j][0], dq[j][1], dq[j][2], dq[j][3]};
            if (rope.cos_t) agpt_fast::rope_inverse_part<4, HD>(v, rope.cos_t, rope.sin_t, pos, kBlk * j + 4 * g);
            store_vec<4>(dQ + row * D + h * HD + kBlk * j + 4 * g, v);
          }
          if (g == 0) Dl[row * H + h] = dl;
        }
        if (hl + 1 < hpu) {  // the next head's operands, its state from zero
          qf = qn;
          gf = gn;
          l2 = l2n * kLog2e;
          if constexpr (kDeltaFromO) {
#pragma unroll
            for (int j = 0; j < KD; ++j) ov[j] = on[j];
          }
          start_head();
        }
      }
      hl = nxh;
      pass = nxp;
      ch = nxc;
      __syncthreads();
    }
    u = uniform(tb.next[par]);
  }
}

// ---------------------------------------------------------------------------
// Backward, key side: dK, dV of the tile's key list, head after head. The
// head's Q and dO rows, lse and δ are staged in LDS (the next head's are
// fetched into registers while the current one is worked on). S = Q_i K^T
// puts key c in lane column c (queries 4g .. 4g+3 in its registers);
// dV^T += dO^T P, dK^T += Q^T dS. Key blocks are dealt to the waves in
// turn; a wave loads the K and V slices of its next (head, key block) while
// it works on the current one.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) void bwd_kv_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const float* __restrict__ lse, const float* __restrict__ Dl, const Tin* __restrict__ dO,
    float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ Pk, float* __restrict__ Pv,
    const float* __restrict__ acc_dk, const float* __restrict__ acc_dv, RopeT rope, int H, int hpu,
    float scale) {
  constexpr int KD = HD / 4;
  constexpr int MT = HD / 16;
  constexpr int EPC = 16 / static_cast<int>(sizeof(Tin));
  constexpr int WS = row_stride(HD, sizeof(Tin));
  constexpr int PIECES = HD / EPC;
  constexpr int ROWJ = kTile * PIECES;  // 16-byte pieces of one staged tensor
  constexpr int RPER = ROWJ / kThreads;
  static_assert(ROWJ % kThreads == 0, "whole rounds of the workgroup per staged tensor");
  __shared__ Tables tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  Tin* Qs = reinterpret_cast<Tin*>(dyn);
  Tin* Gs = Qs + kTile * WS;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const float qscale = scale * kLog2e;
  // bf16 scores come unscaled (the fp32 operands are scaled once): the
  // scale goes into the exponent's multiply-add.
  const float sfac = Slice<Tin, HD / 4>::kPre ? 1.0f : qscale;
  int* ctr = pl.sched + 2;
  if (threadIdx.x == 0) tb.next[1] = atomicAdd(ctr, 1);
  __syncthreads();
  int u = uniform(tb.next[1]);
  const int ngr = H / hpu;  // head groups: unit u = (tile u / ngr, heads hpu * (u % ngr) ..)
  const int64_t n_units = static_cast<int64_t>(pl.n_tiles) * ngr;
  for (int par = 0; u < n_units; par ^= 1) {
    if (threadIdx.x == 0) tb.next[par] = atomicAdd(ctr, 1);
    const int t = tile_of(pl, u / ngr);
    const int h0 = (u % ngr) * hpu;
    const int h1 = h0 + hpu;
    const int s = t * kTile;
    const int ntile = static_cast<int>(min(static_cast<int64_t>(kTile), pl.T - s));
    // Staged rows of head h (rows past a short tile repeat its last row).
    u4 rq[RPER], rg[RPER];
    float rl = 0.0f, rd = 0.0f;
    auto fetch_rows = [&](int h) {
#pragma unroll
      for (int k = 0; k < RPER; ++k) {
        const int j = static_cast<int>(threadIdx.x) + k * kThreads;
        const int64_t off = (static_cast<int64_t>(s) + min(j / PIECES, ntile - 1)) * D + h * HD + (j % PIECES) * EPC;
        rq[k] = *reinterpret_cast<const u4*>(Q + off);
        rg[k] = *reinterpret_cast<const u4*>(dO + off);
      }
      if (threadIdx.x < kTile) {
        const int64_t r = static_cast<int64_t>(s) + min(static_cast<int>(threadIdx.x), ntile - 1);
        rl = lse[r * H + h];
        rd = Dl[r * H + h];
      }
    };
    auto stage_rows = [&]() {
#pragma unroll
      for (int k = 0; k < RPER; ++k) {
        const int j = static_cast<int>(threadIdx.x) + k * kThreads;
        *reinterpret_cast<u4*>(Qs + (j / PIECES) * WS + (j % PIECES) * EPC) = rq[k];
        *reinterpret_cast<u4*>(Gs + (j / PIECES) * WS + (j % PIECES) * EPC) = rg[k];
      }
      if (threadIdx.x < kTile) {
        tb.l2[threadIdx.x] = rl * kLog2e;
        tb.dl[threadIdx.x] = rd;
      }
    };
    fetch_rows(h0);
    const Unit w = build_tables(pl, tb, t, true);
    stage_rows();
    __syncthreads();
    const int poff = w.poff;
    const int A = w.A;
    const int nkb = (A + ntile + kBlk - 1) / kBlk;
    // K and V slices of (head h, key block b); keys past the list name row s.
    Slice<Tin, KD> kf, vf, nkf, nvf;
    auto fetch = [&](int h, int b, Slice<Tin, KD>& a, Slice<Tin, KD>& v) {
      const int64_t row = tb.krow[kBlk * b + c];
      a.load(K + row * D + h * HD + KD * g);
      v.load(V + row * D + h * HD + KD * g);
    };
    if (wave < nkb) fetch(h0, wave, nkf, nvf);
    for (int h = h0; h < h1; ++h) {
      if (h + 1 < h1) fetch_rows(h + 1);
      for (int b = wave; b < nkb; b += 4) {
        kf = nkf;
        vf = nvf;
        if (b + 4 < nkb) fetch(h, b + 4, nkf, nvf);
        else if (h + 1 < h1) fetch(h + 1, wave, nkf, nvf);
        kf.scale(qscale);
        f4 dk[MT], dv[MT];
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          dk[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
          dv[j] = dk[j];
        }
        const int key = kBlk * b + c;
        const int iv = tb.kint[key];
        const int i0 = uniform(tb.blo[b]) / kBlk;
        const int i1 = (uniform(tb.bhi[b]) + kBlk - 1) / kBlk;
        for (int i = i0; i < i1; ++i) {
          const int qr = kBlk * i + c;  // query row this lane supplies
          const int q0 = kBlk * i + 4 * g;
          bool live[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) live[r] = in_interval(q0 + r, iv);
          Slice<Tin, KD> qa, ga;
          qa.load(Qs + qr * WS + KD * g);
          ga.load(Gs + qr * WS + KD * g);
          f4 sv = slice_dot(qa, kf, f4{0.0f, 0.0f, 0.0f, 0.0f});  // sv[r]: query q0+r against key `key`
          const f4 tv = slice_dot(ga, vf, f4{0.0f, 0.0f, 0.0f, 0.0f});
          const f4 l2v = *reinterpret_cast<const f4*>(&tb.l2[q0]);
          const f4 dlv = *reinterpret_cast<const f4*>(&tb.dl[q0]);
          float p[4], ds[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {  // masked: exp2(-inf) = 0, no branch per pair
            p[r] = fast_exp2(live[r] ? __builtin_fmaf(sv[r], sfac, -l2v[r]) : -__builtin_inff());
            ds[r] = p[r] * (tv[r] - dlv[r]) * scale;
          }
          if constexpr (sizeof(Tin) == 2) {  // P and dS rounded to bf16, one 16-deep step per tile
            const uint2 pw = pack_bf16(p), dw = pack_bf16(ds);
#pragma unroll
            for (int j = 0; j < MT; ++j) {  // dO^T, Q^T blocks: dims 16j .., queries 16i ..
              dv[j] = mfma_a_bf16(read_tr(Gs, WS, kBlk * i, kBlk * j, lane), pw, dv[j]);
              dk[j] = mfma_a_bf16(read_tr(Qs, WS, kBlk * i, kBlk * j, lane), dw, dk[j]);
            }
          } else {
#pragma unroll
            for (int j = 0; j < MT; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int row = (q0 + r) * WS + kBlk * j + c;
                dv[j] = mfma16(ld1(Gs + row), p[r], dv[j]);
                dk[j] = mfma16(ld1(Qs + row), ds[r], dk[j]);
              }
          }
        }
        // Emit dims 16j+4g.. of the key.
        if (key < A) {
          const int64_t prow = static_cast<int64_t>(poff) + key;  // prefix entry `key` = depth key+1
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            float a[4] = {dk[j][0], dk[j][1], dk[j][2], dk[j][3]};
            float v[4] = {dv[j][0], dv[j][1], dv[j][2], dv[j][3]};
            store_vec<4>(Pk + prow * D + h * HD + kBlk * j + 4 * g, a);
            store_vec<4>(Pv + prow * D + h * HD + kBlk * j + 4 * g, v);
          }
        } else if (key < A + ntile) {
          const int r = key - A;
          const int64_t a = static_cast<int64_t>(s) + r;
          const bool done = tb.rend[r] <= s + ntile;
          const int pos = rope.cos_t ? rope_pos(tb.rdep[r], rope.seq_len) : 0;
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            const int d0 = kBlk * j + 4 * g;
            float gk[4] = {dk[j][0], dk[j][1], dk[j][2], dk[j][3]};
            float gv[4] = {dv[j][0], dv[j][1], dv[j][2], dv[j][3]};
            if (done) {
              if (acc_dk) {
                float y[4];
                load_vec<4>(acc_dk + a * D + h * HD + d0, y);
#pragma unroll
                for (int x = 0; x < 4; ++x) gk[x] += y[x];
              }
              if (acc_dv) {
                float y[4];
                load_vec<4>(acc_dv + a * D + h * HD + d0, y);
#pragma unroll
                for (int x = 0; x < 4; ++x) gv[x] += y[x];
              }
              if (rope.cos_t) agpt_fast::rope_inverse_part<4, HD>(gk, rope.cos_t, rope.sin_t, pos, d0);
            }
            store_vec<4>(dK + a * D + h * HD + d0, gk);
            store_vec<4>(dV + a * D + h * HD + d0, gv);
          }
        }
      }
      __syncthreads();  // the head's staged rows are no longer read
      if (h + 1 < h1) {
        stage_rows();
        __syncthreads();
      }
    }
    u = uniform(tb.next[par]);
  }
}


// ---------------------------------------------------------------------------
// Key side over each tile's subtree range, for plans whose subtrees end
// within a few tiles (chains of a few hundred rows, C5). In DFS preorder
// the rows that see key row k are k .. end[k]-1, so every query of a tile's
// keys lies in the contiguous rows [s, E), E the greatest subtree end of the
// tile's rows. A unit is (tile, head): wave w owns the tile's key block w
// (16 keys, K and V slices in registers) and the rows [s, E) pass through
// LDS 64 at a time (the head's Q and dO rows, lse, δ; the next 64 in
// registers while the current ones are worked on). Every key's dK/dV is
// complete at the unit's end: no partials, no carry, no reduction kernel.
// pl.range_bend[4 t + w]: the greatest subtree end of key block w of tile t
// (0 for a block past a short tile); pl.range_order: the tiles by
// descending query range, claimed in that order.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(sizeof(Tin) == 2 ? 3 : 2))) void bwd_kv_range_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const float* __restrict__ lse, const float* __restrict__ Dl, const Tin* __restrict__ dO,
    float* __restrict__ dK, float* __restrict__ dV, const float* __restrict__ acc_dk,
    const float* __restrict__ acc_dv, RopeT rope, int H, float scale) {
  constexpr int KD = HD / 4;
  constexpr int MT = HD / 16;
  constexpr int EPC = 16 / static_cast<int>(sizeof(Tin));
  constexpr int WS = row_stride(HD, sizeof(Tin));
  constexpr int PIECES = HD / EPC;
  constexpr int ROWJ = kTile * PIECES;  // 16-byte pieces of one staged tensor
  constexpr int RPER = ROWJ / kThreads;
  static_assert(ROWJ % kThreads == 0, "whole rounds of the workgroup per staged tensor");
  __shared__ int32_t next[2];
  __shared__ alignas(16) float l2s[kTile];  // lse * log2(e) of the staged rows
  __shared__ alignas(16) float dls[kTile];  // δ of the staged rows
  extern __shared__ __align__(16) unsigned char dyn[];
  Tin* Qs = reinterpret_cast<Tin*>(dyn);
  Tin* Gs = Qs + kTile * WS;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const float qscale = scale * kLog2e;
  // bf16 scores come unscaled (the fp32 operands are scaled once): the
  // scale goes into the exponent's multiply-add.
  const float sfac = Slice<Tin, HD / 4>::kPre ? 1.0f : qscale;
  const int64_t n_units = static_cast<int64_t>(pl.n_tiles) * H;
  int* ctr = pl.sched + 2;
  if (threadIdx.x == 0) next[1] = atomicAdd(ctr, 1);
  __syncthreads();
  // The next unit's first query rows, its keys' K and V slices, subtree
  // ends and block range ends are loaded during the current unit's last
  // query tile (its claim is known from the unit's first barrier on), so a
  // unit starts on rows already in registers.
  u4 rq[RPER], rg[RPER];
  float rl = 0.0f, rd = 0.0f;
  // Rows qs .. qs+63 of head hh (rows past the plan repeat its last row).
  auto fetch_rows = [&](int64_t qs, int hh) {
    const int last = static_cast<int>(min(static_cast<int64_t>(kTile), pl.T - qs)) - 1;
#pragma unroll
    for (int k = 0; k < RPER; ++k) {
      const int j = static_cast<int>(threadIdx.x) + k * kThreads;
      const int64_t off = (qs + min(j / PIECES, last)) * D + hh * HD + (j % PIECES) * EPC;
      rq[k] = *reinterpret_cast<const u4*>(Q + off);
      rg[k] = *reinterpret_cast<const u4*>(dO + off);
    }
    if (threadIdx.x < kTile) {
      const int64_t r = qs + min(static_cast<int>(threadIdx.x), last);
      rl = lse[r * H + hh];
      rd = Dl[r * H + hh];
    }
  };
  auto stage_rows = [&]() {
#pragma unroll
    for (int k = 0; k < RPER; ++k) {
      const int j = static_cast<int>(threadIdx.x) + k * kThreads;
      *reinterpret_cast<u4*>(Qs + (j / PIECES) * WS + (j % PIECES) * EPC) = rq[k];
      *reinterpret_cast<u4*>(Gs + (j / PIECES) * WS + (j % PIECES) * EPC) = rg[k];
    }
    if (threadIdx.x < kTile) {
      l2s[threadIdx.x] = rl * kLog2e;
      dls[threadIdx.x] = rd;
    }
  };
  const int key = kBlk * wave + c;  // this lane's key of the tile (block `wave`, column c)
  Slice<Tin, KD> nkf, nvf;
  int nkend = 0;
  int nbend = 0;  // lane l < 4: the greatest subtree end of key block l
  auto prefetch = [&](int uu, int tt) {
    const int hh = uu % H;
    const int64_t s0 = static_cast<int64_t>(tt) * kTile;
    const int nt = static_cast<int>(min(static_cast<int64_t>(kTile), pl.T - s0));
    const int64_t kr = s0 + min(key, nt - 1);
    fetch_rows(s0, hh);
    nkf.load(K + kr * D + hh * HD + KD * g);
    nvf.load(V + kr * D + hh * HD + KD * g);
    nkend = pl.end[kr];
    nbend = pl.range_bend[4 * tt + (lane & 3)];
  };
  int u = uniform(next[1]);
  int t = u < n_units ? uniform(pl.range_order[u / H]) : 0;
  if (u < n_units) prefetch(u, t);
  for (int par = 0; u < n_units; par ^= 1) {
    if (threadIdx.x == 0) next[par] = atomicAdd(ctr, 1);
    const int h = u % H;
    const int64_t s = static_cast<int64_t>(t) * kTile;
    const int ntile = static_cast<int>(min(static_cast<int64_t>(kTile), pl.T - s));
    const bool kvalid = key < ntile;
    const int64_t krow = s + min(key, ntile - 1);
    const int64_t kend = kvalid ? static_cast<int64_t>(nkend) : 0;
    // The block's query range end, and the tile's: the greatest over its blocks.
    const int bend = __builtin_amdgcn_readlane(nbend, wave);
    const int tend = max(max(__builtin_amdgcn_readlane(nbend, 0), __builtin_amdgcn_readlane(nbend, 1)),
                         max(__builtin_amdgcn_readlane(nbend, 2), __builtin_amdgcn_readlane(nbend, 3)));
    const int nq = static_cast<int>((tend - s + kTile - 1) / kTile);
    Slice<Tin, KD> kf = nkf, vf = nvf;
    f4 dk[MT], dv[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      dk[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      dv[j] = dk[j];
    }
    stage_rows();
    kf.scale(qscale);
    __syncthreads();
    const int un = uniform(next[par]);  // the next unit (claimed above, published by the barrier)
    const int tn_raw = un < n_units ? pl.range_order[un / H] : 0;
    int tn = 0;
    for (int qt = 0; qt < nq; ++qt) {
      const int64_t qs = s + static_cast<int64_t>(qt) * kTile;
      if (qt + 1 < nq) {
        fetch_rows(qs + kTile, h);
      } else if (un < n_units) {
        tn = uniform(tn_raw);
        prefetch(un, tn);
      }
      // The key's rows [krow, kend) over the staged rows; query blocks of
      // the first tile before the key block never see it.
      const int lo = static_cast<int>(max(krow - qs, static_cast<int64_t>(0)));
      const int hi = static_cast<int>(max(min(kend - qs, static_cast<int64_t>(kTile)), static_cast<int64_t>(lo)));
      const int iv = lo | ((hi - lo) << 16);
      const int i0 = uniform(qt == 0 ? wave : 0);
      const int i1 = uniform(static_cast<int>(
          min(max(static_cast<int64_t>(bend) - qs + kBlk - 1, static_cast<int64_t>(0)) / kBlk,
              static_cast<int64_t>(kTile / kBlk))));
      for (int i = i0; i < i1; ++i) {
        const int qr = kBlk * i + c;  // query row this lane supplies
        const int q0 = kBlk * i + 4 * g;
        bool live[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) live[r] = in_interval(q0 + r, iv);
        Slice<Tin, KD> qa, ga;
        qa.load(Qs + qr * WS + KD * g);
        ga.load(Gs + qr * WS + KD * g);
        f4 sv = slice_dot(qa, kf, f4{0.0f, 0.0f, 0.0f, 0.0f});  // sv[r]: query q0+r against the key
        const f4 tv = slice_dot(ga, vf, f4{0.0f, 0.0f, 0.0f, 0.0f});
        const f4 l2v = *reinterpret_cast<const f4*>(&l2s[q0]);
        const f4 dlv = *reinterpret_cast<const f4*>(&dls[q0]);
        agpt_blk::bf16x4_bits tgv[sizeof(Tin) == 2 ? MT : 1], tqv[sizeof(Tin) == 2 ? MT : 1];
        if constexpr (sizeof(Tin) == 2) {
#pragma unroll
          for (int j = 0; j < MT; ++j) {  // dO^T, Q^T blocks: dims 16j .., queries 16i ..
            tgv[j] = read_tr(Gs, WS, kBlk * i, kBlk * j, lane);
            tqv[j] = read_tr(Qs, WS, kBlk * i, kBlk * j, lane);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        float p[4], ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // masked: exp2(-inf) = 0, no branch per pair
          p[r] = fast_exp2(live[r] ? __builtin_fmaf(sv[r], sfac, -l2v[r]) : -__builtin_inff());
          // times scale once per key when dK is emitted (1/8 at head_dim
          // 64: a power of two, so the bf16 rounding below is unchanged)
          ds[r] = p[r] * (tv[r] - dlv[r]);
        }
        if constexpr (sizeof(Tin) == 2) {  // P and dS rounded to bf16, one 16-deep step per tile
          const uint2 pw = pack_bf16(p), dw = pack_bf16(ds);
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            dv[j] = mfma_a_bf16(tgv[j], pw, dv[j]);
            dk[j] = mfma_a_bf16(tqv[j], dw, dk[j]);
          }
        } else {
#pragma unroll
          for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = (q0 + r) * WS + kBlk * j + c;
              dv[j] = mfma16(ld1(Gs + row), p[r], dv[j]);
              dk[j] = mfma16(ld1(Qs + row), ds[r], dk[j]);
            }
        }
      }
      __syncthreads();  // the staged rows are no longer read
      if (qt + 1 < nq) {
        stage_rows();
        __syncthreads();
      }
    }
    // dims 16j+4g.. of the key: + seeds, inverse RoPE of dK at its depth.
    if (kvalid) {
      const int pos = rope.cos_t ? rope_pos(pl.depth[krow], rope.seq_len) : 0;
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int d0 = kBlk * j + 4 * g;
        float gk[4] = {dk[j][0] * scale, dk[j][1] * scale, dk[j][2] * scale, dk[j][3] * scale};
        float gv[4] = {dv[j][0], dv[j][1], dv[j][2], dv[j][3]};
        if (acc_dk) {
          float y[4];
          load_vec<4>(acc_dk + krow * D + h * HD + d0, y);
#pragma unroll
          for (int x = 0; x < 4; ++x) gk[x] += y[x];
        }
        if (acc_dv) {
          float y[4];
          load_vec<4>(acc_dv + krow * D + h * HD + d0, y);
#pragma unroll
          for (int x = 0; x < 4; ++x) gv[x] += y[x];
        }
        if (rope.cos_t) agpt_fast::rope_inverse_part<4, HD>(gk, rope.cos_t, rope.sin_t, pos, d0);
        store_vec<4>(dK + krow * D + h * HD + d0, gk);
        store_vec<4>(dV + krow * D + h * HD + d0, gv);
      }
    }
    u = un;
    t = tn;
  }
}

// The key side's K/V slice cache (bf16, every key slot in registers: NI ==
// kRegIters): per wave and register block, four 16-byte pieces per lane.
__host__ __device__ constexpr size_t kv_cache_bytes(int ni, int elem) {
  return ni == kRegIters && elem == 2 ? static_cast<size_t>(kThreads / 64) * kRegIters * 4 * 64 * 16 : 0;
}
static_assert(rows_lds_bytes(64, 2) % 16 == 0 && RawTabs::kBytes % 16 == 0, "16-byte aligned cache entries");
// A 16-dim bf16 slice from / to two 16-byte pieces.
template <typename S>
__device__ __forceinline__ void slice_set(S& s, u4 lo, u4 hi) {
  s.w[0] = lo.x;
  s.w[1] = lo.y;
  s.w[2] = lo.z;
  s.w[3] = lo.w;
  s.w[4] = hi.x;
  s.w[5] = hi.y;
  s.w[6] = hi.z;
  s.w[7] = hi.w;
}
template <typename S>
__device__ __forceinline__ void slice_put(const S& s, u4& lo, u4& hi) {
  lo = u4{s.w[0], s.w[1], s.w[2], s.w[3]};
  hi = u4{s.w[4], s.w[5], s.w[6], s.w[7]};
}
// threadIdx.x through an opaque move: lane addresses derived from it are
// formed where they are used, not hoisted out of the loops (where they
// would hold registers across the whole unit).
__device__ __forceinline__ int opaque_tid() {
  int t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"(static_cast<int>(threadIdx.x)));
  return t;
}

// ---------------------------------------------------------------------------
// Key side with a path carry. A unit is (chunk of consecutive tiles, head);
// the workgroup walks the chunk's tiles in order. The keys a tile leaves
// open (subtree not finished) are exactly the next tile's prefix, one per
// depth, so the sums of the current path's keys are carried from tile to
// tile by depth instead of being left as per-tile partials. A prefix key
// sits at the same key slot (depth - 1) in every tile that sees it, and so
// does a tile row that continues a chain from the tile's first row (row r
// at slot A + r = depth - 1; in a deep trie most tiles lie inside such
// chains). With NI > 0 the wave that owns a key block keeps the block's
// sums in registers, as the accumulators of its matrix products, from one
// tile to the next: a key that stays in its slot never leaves them. NI ==
// kRegItersDeep covers the first 16 * 4 NI slots of a tile; NI == kRegIters
// (plans to depth kRegDepth) covers every key slot.
// The other sums go through this workgroup's carry rows Cs
// [parity][depth][dK, dV][HD] (global memory, read and written only by this
// workgroup; a tile reads the rows of its parity and writes the next
// tile's into the other, with a barrier between tiles): open tile rows
// whose slot changes, keys past the register slots, and with NI == 0 every
// carried sum. A prefix key the next tile still sees adds its
// tile sum to the carry; one it does not see is finished: to dK/dV (a key
// first seen in the chunk whose subtree ended), to the chunk partial
// E[chunk][depth] (a key from before the chunk), or at the chunk's last
// tile to F[chunk][depth] (a key of this chunk still open). Open tile rows
// start their depth's sum. agpt_blk::bwd_carry_kernel then finishes the
// keys whose sums cross chunks (F of their chunk plus E of the later
// chunks, in chunk order).
// E, F: [n_chunks][P][2][D].
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int NI, typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(NI > 0 ? 2 : 3))) void bwd_kv_carry_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const float* __restrict__ lse, const float* __restrict__ Dl, const Tin* __restrict__ dO,
    float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ E, float* __restrict__ F,
    float* __restrict__ Cs, const float* __restrict__ acc_dk, const float* __restrict__ acc_dv, RopeT rope,
    int H, float scale) {
  constexpr int KD = HD / 4;
  constexpr int MT = HD / 16;
  constexpr int EPC = 16 / static_cast<int>(sizeof(Tin));
  constexpr int WS = row_stride(HD, sizeof(Tin));
  constexpr int PIECES = HD / EPC;
  constexpr int ROWJ = kTile * PIECES;  // 16-byte pieces of one staged tensor
  constexpr int RPER = ROWJ / kThreads;
  static_assert(ROWJ % kThreads == 0, "whole rounds of the workgroup per staged tensor");
  __shared__ Tables tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  Tin* Qs = reinterpret_cast<Tin*>(dyn);
  Tin* Gs = Qs + kTile * WS;
  const RawTabs raw{reinterpret_cast<int32_t*>(dyn + rows_lds_bytes(HD, sizeof(Tin)))};
  constexpr bool kCache = kv_cache_bytes(NI, sizeof(Tin)) > 0;
  u4* const kvc = reinterpret_cast<u4*>(dyn + rows_lds_bytes(HD, sizeof(Tin)) + RawTabs::kBytes) +
                  (kCache ? (threadIdx.x >> 6) * NI * 4 * 64 : 0);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const int P = agpt_blk::prefix_cap(pl.max_depth);
  const float qscale = scale * kLog2e;
  // bf16 scores come unscaled (the fp32 operands are scaled once): the
  // scale goes into the exponent's multiply-add.
  const float sfac = Slice<Tin, HD / 4>::kPre ? 1.0f : qscale;
  float* const cs = Cs + static_cast<int64_t>(blockIdx.x) * 2 * P * 2 * HD;
  const int64_t n_units = static_cast<int64_t>(pl.n_chunks) * H;
  int* ctr = pl.sched + 2;
  if (threadIdx.x == 0) tb.next[1] = atomicAdd(ctr, 1);
  __syncthreads();
  int u = uniform(tb.next[1]);
  for (int par = 0; u < n_units; par ^= 1) {
    if (threadIdx.x == 0) tb.next[par] = atomicAdd(ctr, 1);
    const int chunk = u / H;
    const int h = u - chunk * H;
    const int t0 = chunk * pl.chunk_tiles;
    const int t1 = chunk + 1 == pl.n_chunks ? pl.n_tiles : t0 + pl.chunk_tiles;
    const int64_t s_first = static_cast<int64_t>(t0) * kTile;  // keys with rows before it come from before the chunk
    // Staged rows of tile t (rows past a short tile repeat its last row).
    u4 rq[RPER], rg[RPER];
    float rl = 0.0f, rd = 0.0f;
    auto fetch_rows = [&](int t) {
      const int64_t s = static_cast<int64_t>(t) * kTile;
      const int last = static_cast<int>(min(static_cast<int64_t>(kTile), pl.T - s)) - 1;
      const int tid = opaque_tid();
#pragma unroll
      for (int k = 0; k < RPER; ++k) {
        const int j = tid + k * kThreads;
        const int64_t off = (s + min(j / PIECES, last)) * D + h * HD + (j % PIECES) * EPC;
        rq[k] = *reinterpret_cast<const u4*>(Q + off);
        rg[k] = *reinterpret_cast<const u4*>(dO + off);
      }
      if (threadIdx.x < kTile) {
        const int64_t r = s + min(static_cast<int>(threadIdx.x), last);
        rl = lse[r * H + h];
        rd = Dl[r * H + h];
      }
    };
    fetch_rows(t0);
    // Carry registers: the sums of key block wave + 4i (i < NI), one lane
    // column per key slot; zero in the lanes of keys that do not continue.
    constexpr int NR = NI > 0 ? NI : 1;
    // With every key slot in registers (bf16), each lane also keeps the K
    // and V slices of its key in each of its blocks in LDS, tagged with the
    // key's row: a key that stays in its slot from tile to tile (a prefix
    // key of consecutive tiles, a chain row) is loaded from HBM once per
    // chunk instead of once per tile. Entry (wave, turn i): four 16-byte
    // pieces (K low, K high, V low, V high) of 64 lanes each.
    // No entry yet: a tag no key takes (a range plan's context rows sit at
    // negative rows before the range, down to -(its depth)).
    int crow[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) crow[i] = INT32_MIN;
    f4 ck[NR][MT], cv[NR][MT];
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        ck[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        cv[i][j] = ck[i][j];
      }
    int a_prev = 0;  // the previous tile's prefix length
    // The next tile's prefix list: pref_off[t + 1], pref_off[t + 2], loaded
    // a tile ahead; its table inputs are copied into LDS (raw) during the
    // current tile's key blocks, so only the chunk's first tile waits on
    // the plan's tables in global memory.
    int po1 = pl.pref_off[min(t0 + 1, pl.n_tiles)], po2 = pl.pref_off[min(t0 + 2, pl.n_tiles)];
    for (int t = t0; t < t1; ++t) {
      const bool first = t == t0;
      const bool last = t + 1 == t1;
      const int cur = (t - t0) & 1;
      const Unit w = first ? build_tables(pl, tb, t, true) : fill_tables(tb, t, pl.T, po1, po2 - po1, true, raw);
      if (!first) {
        po1 = po2;
        po2 = pl.pref_off[min(t + 2, pl.n_tiles)];
      }
#pragma unroll
      for (int k = 0; k < RPER; ++k) {
        const int j = static_cast<int>(threadIdx.x) + k * kThreads;
        *reinterpret_cast<u4*>(Qs + (j / PIECES) * WS + (j % PIECES) * EPC) = rq[k];
        *reinterpret_cast<u4*>(Gs + (j / PIECES) * WS + (j % PIECES) * EPC) = rg[k];
      }
      if (threadIdx.x < kTile) {
        tb.l2[threadIdx.x] = rl * kLog2e;
        tb.dl[threadIdx.x] = rd;
      }
      __syncthreads();
      if (!last) {
        raw.gather(pl, t + 1, po1, po2 - po1, wave, lane);
        fetch_rows(t + 1);
      }
      const int s = w.s, ntile = w.ntile, A = w.A;
      const int nkb = (A + ntile + kBlk - 1) / kBlk;
      Slice<Tin, KD> kf, vf, nkf, nvf;
      bool nmiss = false;  // the prefetched block's slices came from HBM (kCache)
      auto fetch = [&](int b, Slice<Tin, KD>& a, Slice<Tin, KD>& v) {
        const int64_t row = tb.krow[kBlk * b + c];
        a.load(K + row * D + h * HD + KD * g);
        v.load(V + row * D + h * HD + KD * g);
      };
      // Key block b, accumulated into dk, dv: with reg, this wave's carry
      // registers of the block (the carried sums of its prefix keys, zero in
      // every other lane), which keep the sums that continue into the next
      // tile and are zero again in every other lane at the end.
      // The slices of key block b (turn i of this wave) through the cache:
      // lanes whose key is the tagged row read LDS, the others HBM (their
      // entries are written when the block is taken, kmiss).
      auto fetch_c = [&](int b, int i, Slice<Tin, KD>& a, Slice<Tin, KD>& v, bool& miss) {
        if constexpr (kCache) {
          const int row = tb.krow[kBlk * b + c];
          miss = row != crow[i];
          if (miss) {
            a.load(K + static_cast<int64_t>(row) * D + h * HD + KD * g);
            v.load(V + static_cast<int64_t>(row) * D + h * HD + KD * g);
            crow[i] = row;
          } else {
            const u4* e = kvc + i * 4 * 64 + lane;
            const u4 x0 = e[0], x1 = e[64], y0 = e[128], y1 = e[192];
            slice_set(a, x0, x1);
            slice_set(v, y0, y1);
          }
        }
      };
      auto key_block = [&](int b, f4 (&dk)[MT], f4 (&dv)[MT], bool reg, int turn) {
        int tid;
        asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"(static_cast<int>(threadIdx.x)));
        const int lane = tid & 63;
        const int g = lane >> 4, c = lane & 15;
        kf = nkf;
        vf = nvf;
        if constexpr (kCache) {
          if (nmiss) {
            u4* e = kvc + turn * 4 * 64 + lane;
            slice_put(kf, e[0], e[64]);
            slice_put(vf, e[128], e[192]);
          }
          if (b + 4 < nkb && turn + 1 < NR) fetch_c(b + 4, turn + 1, nkf, nvf, nmiss);
        } else {
          if (b + 4 < nkb) fetch(b + 4, nkf, nvf);
        }
        kf.scale(qscale);
        const int key = kBlk * b + c;
        // The key's interval and the block's query range read together (the
        // compiler would sink the interval read past the range's wait).
        const int iv = tb.kint[key];
        const int blo = tb.blo[b], bhi = tb.bhi[b];
        asm volatile("" ::"v"(iv), "v"(blo), "v"(bhi));
        const int i0 = uniform(blo) / kBlk;
        const int i1 = (uniform(bhi) + kBlk - 1) / kBlk;
        for (int i = i0; i < i1; ++i) {
          const int qr = kBlk * i + c;
          const int q0 = kBlk * i + 4 * g;
          bool live[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) live[r] = in_interval(q0 + r, iv);
          Slice<Tin, KD> qa, ga;
          qa.load(Qs + qr * WS + KD * g);
          ga.load(Gs + qr * WS + KD * g);
          f4 sv = slice_dot(qa, kf, f4{0.0f, 0.0f, 0.0f, 0.0f});
          const f4 tv = slice_dot(ga, vf, f4{0.0f, 0.0f, 0.0f, 0.0f});
          const f4 l2v = *reinterpret_cast<const f4*>(&tb.l2[q0]);
          const f4 dlv = *reinterpret_cast<const f4*>(&tb.dl[q0]);
          // bf16: the second products' transposed operands are read here,
          // in the registers the first products' operands free, so the reads
          // overlap the softmax instead of one wait per product after it.
          agpt_blk::bf16x4_bits tgv[sizeof(Tin) == 2 ? MT : 1], tqv[sizeof(Tin) == 2 ? MT : 1];
          if constexpr (sizeof(Tin) == 2) {
#pragma unroll
            for (int j = 0; j < MT; ++j) {  // dO^T, Q^T blocks: dims 16j .., queries 16i ..
              tgv[j] = read_tr(Gs, WS, kBlk * i, kBlk * j, lane);
              tqv[j] = read_tr(Qs, WS, kBlk * i, kBlk * j, lane);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          float p[4], ds[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {  // masked: exp2(-inf) = 0, no branch per pair
            p[r] = fast_exp2(live[r] ? __builtin_fmaf(sv[r], sfac, -l2v[r]) : -__builtin_inff());
            ds[r] = p[r] * (tv[r] - dlv[r]) * scale;
          }
          if constexpr (sizeof(Tin) == 2) {
            const uint2 pw = pack_bf16(p), dw = pack_bf16(ds);
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              dv[j] = mfma_a_bf16(tgv[j], pw, dv[j]);
              dk[j] = mfma_a_bf16(tqv[j], dw, dk[j]);
            }
          } else {
#pragma unroll
            for (int j = 0; j < MT; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int row = (q0 + r) * WS + kBlk * j + c;
                dv[j] = mfma16(ld1(Gs + row), p[r], dv[j]);
                dk[j] = mfma16(ld1(Qs + row), ds[r], dk[j]);
              }
          }
        }
        // This lane's share of the key: dims 16j+4g.. of dK (gk) and dV (gv).
        float gk[MT][4], gv[MT][4];
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            gk[j][x] = dk[j][x];
            gv[j][x] = dv[j][x];
          }
        auto slot = [&](int parity, int d) { return cs + ((parity * P + d) * 2) * HD + 4 * g; };
        auto put = [&](float* o, int stride) {  // o: the key's dK row (dims), dV row `stride` floats on
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            store_vec<4>(o + kBlk * j, gk[j]);
            store_vec<4>(o + stride + kBlk * j, gv[j]);
          }
        };
        auto chunk_part = [&](float* base, int d) {
          put(base + (static_cast<int64_t>(chunk) * P + d) * 2 * D + h * HD + 4 * g, D);
        };
        // Final dK/dV of row a at depth dep: + seeds, inverse RoPE of dK.
        auto finish = [&](int64_t a, int dep) {
          const int pos = rope.cos_t ? rope_pos(dep, rope.seq_len) : 0;
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            const int d0 = kBlk * j + 4 * g;
            if (acc_dk) {
              float y[4];
              load_vec<4>(acc_dk + a * D + h * HD + d0, y);
#pragma unroll
              for (int x = 0; x < 4; ++x) gk[j][x] += y[x];
            }
            if (acc_dv) {
              float y[4];
              load_vec<4>(acc_dv + a * D + h * HD + d0, y);
#pragma unroll
              for (int x = 0; x < 4; ++x) gv[j][x] += y[x];
            }
            if (rope.cos_t) agpt_fast::rope_inverse_part<4, HD>(gk[j], rope.cos_t, rope.sin_t, pos, d0);
            store_vec<4>(dK + a * D + h * HD + d0, gk[j]);
            store_vec<4>(dV + a * D + h * HD + d0, gv[j]);
          }
        };
        bool keep = false;  // the lane's key sum continues in the carry registers
        if (key < A) {
          const int d = key;  // prefix entry d = depth d+1
          const int e = tb.pend[d];
          // The sum so far is in the registers when the key had this key
          // slot in the previous tile too: a key of its prefix, or one of its
          // rows that continued a chain from its first row (row r' at slot
          // a_prev + r' = its depth - 1). Else it is in the carry row.
          const int pr = tb.krow[key] - (s - kTile);  // row in the previous tile, < 0: its prefix
          if (!first && (!reg || (pr >= 0 && a_prev + pr != d))) {
            const float* cp = slot(cur, d);
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              float yk[4], yv[4];
              load_vec<4>(cp + kBlk * j, yk);
              load_vec<4>(cp + HD + kBlk * j, yv);
#pragma unroll
              for (int x = 0; x < 4; ++x) {
                gk[j][x] = yk[x] + gk[j][x];
                gv[j][x] = yv[x] + gv[j][x];
              }
            }
          }
          const bool cont = !last && e > s + ntile;  // the next tile of the chunk sees it
          if (cont) {
            if (reg) keep = true;
            else put(slot(cur ^ 1, d), HD);
          } else if (tb.krow[key] < s_first) {
            chunk_part(E, d);  // a key from before the chunk
          } else if (e > s + ntile) {
            chunk_part(F, d);  // the chunk ends, the key's subtree does not
          } else {
            finish(tb.krow[key], d + 1);
          }
        } else if (key < A + ntile) {
          const int r = key - A;
          const int64_t a = static_cast<int64_t>(s) + r;
          if (tb.rend[r] <= s + ntile) finish(a, tb.rdep[r]);
          else if (last) chunk_part(F, tb.rdep[r] - 1);
          else if (reg && tb.rdep[r] - 1 == key) keep = true;  // the next tile's prefix entry in this slot
          else put(slot(cur ^ 1, tb.rdep[r] - 1), HD);  // the next tile's prefix entry at its depth
        }
        if (reg) {
#pragma unroll
          for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int x = 0; x < 4; ++x) {
              dk[j][x] = keep ? gk[j][x] : 0.0f;
              dv[j][x] = keep ? gv[j][x] : 0.0f;
            }
        }
      };
      __builtin_amdgcn_s_setprio(0);  // the key blocks at the base priority
      if (wave < nkb) {
        if constexpr (kCache) fetch_c(wave, 0, nkf, nvf, nmiss);
        else fetch(wave, nkf, nvf);
      }
      if constexpr (NI == kRegIters) {  // every key block of the tile in registers
#pragma unroll
        for (int i = 0; i < NI; ++i)
          if (wave + 4 * i < nkb) key_block(wave + 4 * i, ck[i], cv[i], true, i);
      } else if constexpr (NI > 0) {
        // Deeper plans: the wave's first NI blocks in registers (selected by
        // the block's turn i, a uniform value), the blocks after them through
        // the carry rows. (One call per block, unrolled, spills 192 bytes per
        // lane and ran slower than these selects.)
        for (int b = wave, i = 0; b < nkb; b += 4, ++i) {
          f4 dk[MT], dv[MT];
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            dk[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            dv[j] = dk[j];
#pragma unroll
            for (int x = 0; x < NI; ++x) {
              dk[j] = i == x ? ck[x][j] : dk[j];
              dv[j] = i == x ? cv[x][j] : dv[j];
            }
          }
          key_block(b, dk, dv, i < NI, 0);
#pragma unroll
          for (int x = 0; x < NI; ++x)
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              ck[x][j] = i == x ? dk[j] : ck[x][j];
              cv[x][j] = i == x ? dv[j] : cv[x][j];
            }
        }
      } else {
        for (int b = wave; b < nkb; b += 4) {
          f4 dk[MT], dv[MT];
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            dk[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            dv[j] = dk[j];
          }
          key_block(b, dk, dv, false, 0);
        }
      }
      a_prev = A;
      // the tile's end and the next tile's tables, staging and barriers
      // ahead of the other workgroup's key blocks
      __builtin_amdgcn_s_setprio(3);
      wait_loads();     // the next tile's table inputs are in LDS
      __syncthreads();  // the tile's staged rows, tables and carry rows are done with
    }
    u = uniform(tb.next[par]);
  }
}

}  // namespace agpt_deep
