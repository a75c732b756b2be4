// trie_block.h — block-sparse trie-attention kernels on 16x16 fp32 matrix
// instructions (included by trie_attn.hip after trie_fast.h).
//
// Same persistent streaming scheme as trie_fast.h: a workgroup (256 threads,
// 4 waves) owns one head group of HG heads and a contiguous range of kTile-row
// tiles, keeps the tile context in LDS and prefetches the next tile into
// registers while the current one computes. What differs is the unit of
// work. The tile's attention pattern is a mask over (tile row, key-set slot):
// in DFS preorder the rows that see a key form one interval,
//   prefix key (ancestor of the tile's first row s): rows [0, end - s),
//   tile row c:                                      rows [c, end(c) - s),
// so a 16-row query block and a 16-slot key block either share no pair or
// are handled as one dense 16x16 block with a per-pair interval mask. On the
// C2 corpus a 64-row tile touches ~12.7 such block pairs per head (36% of
// their pairs are live), against ~5x more LDS traffic and instructions per
// live pair for the 4x4 chain-group walk of trie_fast.h.
//
// LDS key set: slots [P - A, P) hold the A prefix rows right-aligned (entry d
// = depth d+1 at slot P - A + d), slots P.. the tile rows; P = max_depth - 1
// rounded up to 16, so key blocks (16 slots) never straddle the prefix/row
// boundary. Slots below P - A are dead (empty interval). Moving to the next
// tile copies each prefix row LDS to LDS, from the current prefix (same
// depth) or from a current tile row; only the first tile of a range (or a
// prefix too long to copy) loads its prefix from memory.
//
// Matrix instruction v_mfma_f32_16x16x4f32: D[16][16] += A[16][4] B[4][16]
// with lane l = 16g + c supplying A[c][g] and B[g][c] and holding D[4g+r][c]
// in register r. The contraction index is permuted freely: step j pairs
// lane group g with dim KD*g + j (KD = HD/4), so every lane reads one
// contiguous KD-slice of a row; for the second product the 4x4 register
// block of D is reused directly as B (key 4g + j at step j).
//
//  query side (forward, dQ): unit = (head, query block i). S^T = K_blk Q_i^T
//    puts query c in lane column c with keys 4g..4g+3 in its registers; the
//    softmax max is reduced over the four lane groups (permlane swaps), and
//    P^T feeds O^T += V^T P^T directly (O^T: dims 4g+r of query c).
//  key side (dK, dV): unit = (head, key block). S = Q_i K_blk^T puts key c in
//    lane column c with queries 4g..4g+3 in registers; P and dS feed
//    dV^T += dO^T P and dK^T += Q^T dS directly.
//
// Units are dealt to the waves in snake order (wave w takes units w, 7-w,
// 8+w, 15-w, ...) after ordering them longest first, which balances the
// waves of a tile without a sort.
#pragma once

namespace agpt_blk {

using namespace agpt;
using agpt_fast::f4;
using agpt_fast::lds_stride;
using agpt_fast::u4;
using agpt_fast::uniform;

constexpr int kTile = 64;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kBlk = 16;               // rows per query block, slots per key block
constexpr float kRescaleLog2 = 8.0f;   // lazy-rescale threshold (log2 units)
constexpr int kCopyPer = 2;            // prefix-copy jobs per thread (else reload)
constexpr int kMaxSlots = kMaxDepth + kTile;
// Stream table flags: lse of the tile rows; δ of the tile rows read from Dl;
// δ = dO·O computed from the fetched O (NT == 3) into the δ table.
constexpr int kLse = 1, kDl = 2, kDeltaO = 4;

// Prefix capacity P: max_depth - 1 rounded up to whole key blocks.
__host__ __device__ constexpr int prefix_cap(int max_depth) {
  return (max_depth - 1 + kBlk - 1) / kBlk * kBlk;
}

// Dynamic LDS: key set K, V [P + kTile][WS], ns staged tile tensors
// [kTile][WS], and with pdl the δ partials [kTile][HG][HD/EPC] fp32.
__host__ __device__ inline size_t block_lds_bytes(int max_depth, int HG, int HD, int elem, int ns, bool pdl) {
  const int ws = HG * HD + 16 / elem;
  size_t b = static_cast<size_t>(2 * (prefix_cap(max_depth) + kTile) + ns * kTile) * ws * elem;
  b = (b + 15) & ~static_cast<size_t>(15);
  if (pdl) b += static_cast<size_t>(kTile) * HG * (HD / (16 / elem)) * sizeof(float);
  return b;
}

// LDS tables of a tile. BT = rows of the lse / δ tables (kTile for the
// backward, 0 for the forward: its workgroup then fits four to a CU).
template <int HG, int BT = kTile>
struct alignas(16) BlockTables {
  alignas(16) int32_t kint[kMaxSlots];  // per key slot: lo | (hi - lo) << 16, rows [lo, hi) see it
  int32_t bhi[kMaxSlots / kBlk];    // per key block: max hi of its slots
  int32_t depth[kTile];
  int32_t tend[kTile];              // absolute subtree end of the tile rows
  int32_t pend[kMaxDepth];          // absolute subtree end of prefix entry d
  int32_t grab;                     // last chunk claimed by the workgroup
  alignas(16) float l2[HG][BT];     // lse * log2(e) of the tile rows (backward)
  alignas(16) float dl[HG][BT];     // δ of the tile rows (backward)
};

__device__ __forceinline__ f4 mfma16(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One lane group's KD consecutive dims of a row (dims KD*g ..), as an
// operand of the first products (S = K·Qᵀ, dO·Vᵀ), whose inputs are the
// caller's tensors. fp32: KD floats, one 4-deep step per dim. bf16: the raw
// halves on the bf16 matrix instructions (one 16-deep step for KD = 4, one
// 32-deep step per 8 dims): lane group g supplies the same dims of both
// operands, and products of bf16 values are exact in fp32, so the scores
// match the 4-deep form up to the order of the sum. The fp32 form scales the
// held operand once (kPre); the bf16 form scales the scores.
template <typename Tin, int KD>
struct Slice;
template <int KD>
struct Slice<float, KD> {
  static constexpr bool kPre = true;
  float v[KD];
  __device__ __forceinline__ void load(const float* p) { load_vec<KD>(p, v); }
  __device__ __forceinline__ void scale(float f) {
#pragma unroll
    for (int j = 0; j < KD; ++j) v[j] *= f;
  }
};
template <int KD>
struct Slice<bf16_t, KD> {
  static_assert(KD == 4 || KD % 8 == 0, "bf16 slices of 4 or a multiple of 8 dims");
  static constexpr bool kPre = false;
  uint32_t w[KD / 2];
  __device__ __forceinline__ void load(const bf16_t* p) {
    if constexpr (KD == 4) {
      const uint2 x = *reinterpret_cast<const uint2*>(p);
      w[0] = x.x;
      w[1] = x.y;
    } else {
#pragma unroll
      for (int i = 0; i < KD / 8; ++i) {
        const uint4 x = *reinterpret_cast<const uint4*>(p + 8 * i);
        w[4 * i] = x.x;
        w[4 * i + 1] = x.y;
        w[4 * i + 2] = x.z;
        w[4 * i + 3] = x.w;
      }
    }
  }
  __device__ __forceinline__ void scale(float) {}
};

template <int KD>
__device__ __forceinline__ f4 slice_dot(const Slice<float, KD>& a, const Slice<float, KD>& b, f4 acc) {
#pragma unroll
  for (int j = 0; j < KD; ++j) acc = mfma16(a.v[j], b.v[j], acc);
  return acc;
}
template <int KD>
__device__ __forceinline__ f4 slice_dot(const Slice<bf16_t, KD>& a, const Slice<bf16_t, KD>& b, f4 acc) {
  typedef __attribute__((ext_vector_type(4))) short s4;
  typedef __attribute__((ext_vector_type(8))) __bf16 b8;
  if constexpr (KD == 4) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, uint2{a.w[0], a.w[1]}),
                                                      __builtin_bit_cast(s4, uint2{b.w[0], b.w[1]}), acc, 0, 0, 0);
  } else {
#pragma unroll
    for (int i = 0; i < KD / 8; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(b8, uint4{a.w[4 * i], a.w[4 * i + 1], a.w[4 * i + 2], a.w[4 * i + 3]}),
          __builtin_bit_cast(b8, uint4{b.w[4 * i], b.w[4 * i + 1], b.w[4 * i + 2], b.w[4 * i + 3]}), acc, 0, 0, 0);
    return acc;
  }
}

// Second products with bf16 inputs, one 16-deep bf16 step: lane (g, c)
// supplies column c of rows 4g .. 4g+3 of a bf16 LDS tile (`col` points at
// row 4g, column c; rows WS apart) and its own four fp32 weights rounded to
// bf16 (pack_bf16), i.e. A[c][4g+i] and B[4g+i][c].
typedef __attribute__((ext_vector_type(4))) short bf16x4_bits;
__device__ __forceinline__ uint2 pack_bf16(const float (&w)[4]) {
  typedef __attribute__((ext_vector_type(2))) float f2;
  typedef __attribute__((ext_vector_type(2))) __bf16 b2;
  return uint2{__builtin_bit_cast(uint32_t, __builtin_convertvector(f2{w[0], w[1]}, b2)),
               __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{w[2], w[3]}, b2))};
}
__device__ __forceinline__ f4 mfma_rows_bf16(const bf16_t* col, int WS, uint2 wb, f4 acc) {
  const uint16_t* v = reinterpret_cast<const uint16_t*>(col);
  const uint32_t a0 = v[0] | (static_cast<uint32_t>(v[WS]) << 16);
  const uint32_t a1 = v[2 * WS] | (static_cast<uint32_t>(v[3 * WS]) << 16);
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_bits, uint2{a0, a1}),
                                                    __builtin_bit_cast(bf16x4_bits, wb), acc, 0, 0, 0);
}

// Reductions over the four lane groups g (lanes c, c+16, c+32, c+48): each
// swap leaves a lane's own value and its partner's (lane ^ 16, lane ^ 32)
// in the two results.
__device__ __forceinline__ float group_max(float x) {
  const unsigned u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned v = __float_as_uint(x);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group_sum(float x) {
  const unsigned u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const unsigned v = __float_as_uint(x);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Reductions over aligned groups of consecutive lanes with DPP lane moves
// (VALU, no LDS round trip). quad_perm [1,0,3,2] = 0xB1 and [2,3,0,1] = 0x4E
// swap within quads; row_ror:n = 0x120 + n rotates within a row of 16.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
template <int kCtrl>
__device__ __forceinline__ int dpp_n(int v) {
  return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xf, 0xf, false);
}
// Sum over each aligned group of W consecutive lanes (W = 1, 2, 4, 8, 16),
// left in every lane of the group. The order of the additions is fixed.
template <int W>
__device__ __forceinline__ float lane_group_sum(float v) {
  if constexpr (W >= 2) v += dpp_f<0xB1>(v);
  if constexpr (W >= 4) v += dpp_f<0x4E>(v);
  if constexpr (W >= 8) {
    // lanes 0-3 of each 8 take lanes 4-7 (row_ror:12), lanes 4-7 take 0-3 (row_ror:4)
    const float a = dpp_f<0x12C>(v), b = dpp_f<0x124>(v);
    v += (threadIdx.x & 4) ? b : a;
  }
  if constexpr (W >= 16) v += dpp_f<0x128>(v);
  return v;
}
// Max over each row of 16 lanes, left in every lane of the row.
__device__ __forceinline__ int row16_max(int v) {
  v = max(v, dpp_n<0x121>(v));
  v = max(v, dpp_n<0x122>(v));
  v = max(v, dpp_n<0x124>(v));
  return max(v, dpp_n<0x128>(v));
}

__device__ __forceinline__ bool in_interval(int q, int iv) {
  return static_cast<unsigned>(q - (iv & 0xffff)) < static_cast<unsigned>(iv >> 16);
}

__device__ __forceinline__ float ld1(const float* p) { return *p; }
__device__ __forceinline__ float ld1(const bf16_t* p) { return to_f32(*p); }

// k-th unit of wave w in snake order.
__device__ __forceinline__ int snake_unit(int k, int w) { return kWaves * k + ((k & 1) ? kWaves - 1 - w : w); }

// ---------------------------------------------------------------------------
// Tile context stream. NT = tile-row tensors fetched: 1 = Q (forward);
// 2 = Q, dO; 3 = Q, dO, O (O is reduced to δ partials, not staged).
// kTabs: kLse / kDl tables of the tile rows.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, int NT, int kTabs, typename PlanT>
struct BStream {
  using Tables = BlockTables<HG, kTabs != 0 ? kTile : 0>;
  // δ partials per 16-byte chunk in LDS (NT == 3 without kDeltaO).
  static constexpr bool kPdl = NT == 3 && (kTabs & kDeltaO) == 0;
  static constexpr int W = HG * HD;
  static constexpr int WS = lds_stride<Tin>(W);
  static constexpr int EPC = 16 / static_cast<int>(sizeof(Tin));  // elements per 16-B chunk
  static constexpr int CPR = W / EPC;                              // chunks per row slice
  static constexpr int CPH = HD / EPC;                             // chunks per head
  static constexpr int ROWJ = kTile * CPR;                         // chunk jobs per row tensor
  static constexpr int KV_PER = (2 * ROWJ + kThreads - 1) / kThreads;
  static constexpr int T_PER = (ROWJ + kThreads - 1) / kThreads;
  static constexpr int NS = NT < 2 ? NT : 2;  // staged tile tensors
  static constexpr int PJ = 2 * CPR;          // copy jobs per prefix entry (K and V)

  const PlanT pl;
  const Tin* K;
  const Tin* V;
  const Tin* TT[NT];
  const float* lse;
  const float* Dl;
  int D, H, P;
  int hg, n_hg;  // head group of the current / the prefetched tile
  Tin* Ks;
  Tin* Vs;
  Tin* Ts;     // [NS][kTile][WS]
  float* pdl;  // [kTile][HG][CPH] δ partials (NT == 3)
  Tables& tb;
  // current tile
  int s, ntile, A, poff;
  // next tile (prefetched)
  int n_s, n_ntile, n_A, n_poff;
  int n_t = -2, n_pend, n_pend_v;  // last prefetched tile, pref_off[n_t + 1] (loaded there)
  u4 kv[KV_PER];
  u4 tt[NT][T_PER];
  int dep, tend_r;
  float lse_r, dl_r;
  float dscale = 1.0f;  // δ = dO·O is stored times this (NT == 3 with kDeltaO)
  int cp_id[kCopyPer];

  __device__ __forceinline__ BStream(const PlanT& pl_, const Tin* K_, const Tin* V_, const Tin* T0,
                                     const Tin* T1, const Tin* T2, const float* lse_, const float* Dl_,
                                     int H_, int hg_, unsigned char* dyn, Tables& tb_)
      : pl(pl_), K(K_), V(V_), lse(lse_), Dl(Dl_), H(H_), hg(hg_), n_hg(hg_), tb(tb_) {
    TT[0] = T0;
    if constexpr (NT > 1) TT[1] = T1;
    if constexpr (NT > 2) TT[2] = T2;
    D = H * HD;
    P = prefix_cap(pl.max_depth);
    Ks = reinterpret_cast<Tin*>(dyn);
    Vs = Ks + (P + kTile) * WS;
    Ts = Vs + (P + kTile) * WS;
    // Offsets from the LDS base (integer casts of the pointer would lose its
    // address space and turn the accesses into flat ones).
    const int tbytes = (2 * (P + kTile) + NS * kTile) * WS * static_cast<int>(sizeof(Tin));
    pdl = reinterpret_cast<float*>(dyn + ((tbytes + 15) & ~15));
    s = 0;
    A = 0;
    // Every staged value stays finite: a matrix step multiplies dead slots
    // and rows past the tile by zero weights, and 0 * NaN would leak.
    const int n16 = static_cast<int>(lds_bytes(pl.max_depth) / 16);
    u4* z = reinterpret_cast<u4*>(dyn);
    for (int j = threadIdx.x; j < n16; j += kThreads) z[j] = u4{0u, 0u, 0u, 0u};
    __syncthreads();
  }

  __host__ __device__ static size_t lds_bytes(int max_depth) {
    return block_lds_bytes(max_depth, HG, HD, sizeof(Tin), NS, kPdl);
  }

  __device__ __forceinline__ const Tin* gsrc(const Tin* base, int64_t row, int c) const {
    return base + row * D + n_hg * W + c * EPC;
  }

  // Issues the loads of tile nt, head group g, into registers (consumed by
  // commit()).
  __device__ __forceinline__ void prefetch(int nt, int g) {
    const int tid = threadIdx.x;
    n_hg = g;
    n_s = nt * kTile;
    n_ntile = min(kTile, static_cast<int>(pl.T - n_s));
    // The prefix offset of tile nt is the end offset of tile nt - 1, already
    // loaded when that tile was prefetched; only a jump (new chunk) waits on
    // a load here. The end offset is first used by commit().
    n_poff = nt == n_t + 1 ? n_pend : pl.pref_off[nt];
    {
      // Loaded as a per-lane value, so that nothing waits for it before
      // commit() makes it uniform again.
      int idx = nt + 1;
      asm volatile("" : "+v"(idx));
      n_pend_v = pl.pref_off[idx];
    }
    n_t = nt;
    // Unconditional loads from in-range addresses (indices past the tile are
    // clamped; commit() ignores those values). Each address is the tile's
    // uniform base plus a 32-bit byte offset of the lane, so the loads take
    // a scalar base and no 64-bit arithmetic per lane.
    const int last = n_ntile - 1;
    const int64_t rb = static_cast<int64_t>(n_s) * D + n_hg * W;  // the tile's slice, in elements
    auto at = [&](const Tin* base, int r, int c) {
      const unsigned off = static_cast<unsigned>(r * D + c * EPC) * static_cast<unsigned>(sizeof(Tin));
      return *reinterpret_cast<const u4*>(reinterpret_cast<const char*>(base + rb) + off);
    };
#pragma unroll
    for (int k = 0; k < KV_PER; ++k) {
      if constexpr (ROWJ % kThreads == 0) {
        // Whole rounds of the workgroup per tensor: K or V is fixed per k.
        const int ten = k * kThreads / ROWJ;  // a constant once the loop is unrolled
        const int j = tid + k * kThreads - ten * ROWJ;
        kv[k] = at(ten ? V : K, min(j / CPR, last), j % CPR);
      } else {
        const int j = min(tid + k * kThreads, 2 * ROWJ - 1);
        const int ten = j / ROWJ;
        const int r = min((j - ten * ROWJ) / CPR, last);
        kv[k] = *reinterpret_cast<const u4*>(gsrc(ten ? V : K, n_s + r, j % CPR));
      }
    }
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int k = 0; k < T_PER; ++k) {
        const int j = min(tid + k * kThreads, ROWJ - 1);
        tt[i][k] = at(TT[i], min(j / CPR, last), j % CPR);
      }
    const int lane = tid & 63;
    const unsigned lr = static_cast<unsigned>(min(lane, last)) * 4u;
    dep = *reinterpret_cast<const int*>(reinterpret_cast<const char*>(pl.depth + n_s) + lr);
    tend_r = *reinterpret_cast<const int*>(reinterpret_cast<const char*>(pl.end + n_s) + lr);
    if constexpr (kTabs != 0) {
      const int i = min(tid, n_ntile * HG - 1);
      const int r = i / HG;
      const unsigned o = static_cast<unsigned>(r * H + (i - r * HG)) * 4u;
      const int64_t o0 = static_cast<int64_t>(n_s) * H + n_hg * HG;
      if constexpr ((kTabs & kLse) != 0) lse_r = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(lse + o0) + o);
      if constexpr ((kTabs & kDl) != 0) dl_r = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(Dl + o0) + o);
    }
#pragma unroll
    for (int k = 0; k < kCopyPer; ++k) {
      const int d = (tid + k * kThreads) / PJ;
      // Entries past the prefix load a valid one; commit() ignores them (no
      // value is used here, so the loads stay in flight until commit()).
      cp_id[k] = pl.prefix[max(min(n_poff + d, pl.n_prefix - 1), 0)];
    }
  }

  // Interval entry of prefix entry d of the next tile (subtree end e).
  __device__ __forceinline__ void set_prefix_entry(int d, int e) {
    const int slot = P - n_A + d;
    const int hi = min(e - n_s, n_ntile);
    tb.pend[d] = e;
    tb.kint[slot] = hi << 16;
    if ((slot & (kBlk - 1)) == 0 || d == 0) tb.bhi[slot / kBlk] = hi;
  }

  // Installs the prefetched tile in LDS. cold: the prefix rows are loaded
  // from memory (first tile of a chunk, or a prefix too long to copy).
  // publish: thread 0 stores `grab` in tb.grab for every thread to read
  // after the call.
  __device__ __forceinline__ void commit(bool cold, bool publish = false, int grab = 0) {
    const int tid = threadIdx.x;
    n_pend = uniform(n_pend_v);
    n_A = n_pend - n_poff;
    cold = cold || n_A * PJ > kCopyPer * kThreads;
    u4 cpv[kCopyPer];
    int cpe[kCopyPer];
#pragma unroll
    for (int k = 0; k < kCopyPer; ++k) {
      // Source of prefix entry d of the next tile: a current tile row (id >=
      // s) or the current prefix entry of the same depth.
      const int j = tid + k * kThreads;
      const int d = j / PJ;
      const int rem = j % PJ;
      const int id = cp_id[k];
      int src = P, e = 0;  // cold or no entry: a dummy read
      if (!cold && d < n_A && id >= s) {
        src = P + (id - s);
        e = tb.tend[id - s];
      } else if (!cold && d < n_A) {  // an ancestor of s (a context row: negative): d < A
        src = P - A + d;
        e = tb.pend[d];
      }
      cpv[k] = *reinterpret_cast<const u4*>((rem < CPR ? Ks : Vs) + src * WS + (rem % CPR) * EPC);
      cpe[k] = e;
    }
    __syncthreads();  // the current tile's context is no longer read
    if (publish && tid == 0) tb.grab = grab;
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
    if constexpr (NT == 3) {  // δ = dO·O: per 16-byte chunk, then per head
#pragma unroll
      for (int k = 0; k < T_PER; ++k) {
        const int j = tid + k * kThreads;
        const int r = j / CPR;
        const float* g = reinterpret_cast<const float*>(&tt[1][k]);
        const float* o = reinterpret_cast<const float*>(&tt[2][k]);
        float v = (g[0] * o[0] + g[1] * o[1]) + (g[2] * o[2] + g[3] * o[3]);
        if constexpr (kPdl) {
          if (j < ROWJ && r < n_ntile) pdl[r * (HG * CPH) + j % CPR] = v;
        } else {
          // The CPH chunks of a head sit in CPH consecutive lanes.
          v = lane_group_sum<CPH>(v);
          if (j < ROWJ && r < n_ntile && (j % CPH) == 0) tb.dl[(j % CPR) / CPH][r] = v * dscale;
        }
      }
    }
    if (!cold) {
#pragma unroll
      for (int k = 0; k < kCopyPer; ++k) {
        const int j = tid + k * kThreads;
        const int d = j / PJ;
        const int rem = j % PJ;
        if (d < n_A) {
          const int dst = P - n_A + d;
          const bool moved = cp_id[k] >= s || A != n_A;  // else it is already in place
          if (moved) *reinterpret_cast<u4*>((rem < CPR ? Ks : Vs) + dst * WS + (rem % CPR) * EPC) = cpv[k];
          if (rem == 0) set_prefix_entry(d, cpe[k]);
        }
      }
    } else {
      for (int j = tid; j < n_A * PJ; j += kThreads) {
        const int d = j / PJ;
        const int rem = j % PJ;
        const int id = pl.prefix[n_poff + d];
        *reinterpret_cast<u4*>((rem < CPR ? Ks : Vs) + (P - n_A + d) * WS + (rem % CPR) * EPC) =
            *reinterpret_cast<const u4*>(gsrc(rem < CPR ? K : V, id, rem % CPR));
        if (rem == 0) set_prefix_entry(d, pl.pref_end[n_poff + d]);
      }
    }
    // Dead slots of the first prefix block, and the tile rows.
    const int dead0 = (P - n_A) & ~(kBlk - 1);
    if (tid < kBlk && dead0 + tid < P - n_A) tb.kint[dead0 + tid] = 0;
    if (tid < kTile) {
      const int r = tid;
      const bool live = r < n_ntile;
      const int hi = live ? min(tend_r - n_s, n_ntile) : r;
      tb.kint[P + r] = r | ((hi - r) << 16);
      tb.depth[r] = dep;
      tb.tend[r] = tend_r;
      // Row block maxima over the 16 lanes of each block (wave 0).
      int m = live ? hi : 0;
      m = row16_max(m);
      if ((r & (kBlk - 1)) == 0) tb.bhi[(P + r) / kBlk] = m;
    }
    if constexpr (kTabs != 0) {
      if (tid < n_ntile * HG) {
        const int r = tid / HG;
        if constexpr ((kTabs & kLse) != 0) tb.l2[tid - r * HG][r] = lse_r * kLog2e;
        if constexpr ((kTabs & kDl) != 0) tb.dl[tid - r * HG][r] = dl_r;
      }
    }
    // Every prefetched register counts as read here on every path (waves
    // past the row tables, the cold path, rows past a short tile): a load
    // left pending would make the next prefetch wait, before reusing its
    // register, for every memory operation issued after it — the stores
    // of the tile in between included.
    asm volatile("" ::"v"(dep), "v"(tend_r));
#pragma unroll
    for (int k = 0; k < kCopyPer; ++k) asm volatile("" ::"v"(cp_id[k]));
#pragma unroll
    for (int k = 0; k < KV_PER; ++k) asm volatile("" ::"v"(kv[k].x));
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int k = 0; k < T_PER; ++k) asm volatile("" ::"v"(tt[i][k].x));
    if constexpr ((kTabs & kLse) != 0) asm volatile("" ::"v"(lse_r));
    if constexpr ((kTabs & kDl) != 0) asm volatile("" ::"v"(dl_r));
    s = n_s;
    ntile = n_ntile;
    A = n_A;
    poff = n_poff;
    hg = n_hg;
    __syncthreads();
  }
};

// ---------------------------------------------------------------------------
// Dynamic tile chunks. Workgroups claim (chunk, head group) pairs from one
// counter per kernel (chunk c = tiles [cK, (c+1)K), the last chunk running
// to the end). A workgroup claims
// its next chunk during the current one, so with three or more tiles per
// chunk the claim is known before the last tile's prefetch; within a chunk
// the prefix moves LDS to LDS, the first tile of a chunk loads it from
// memory. Results do not depend on which workgroup takes a tile.
// ---------------------------------------------------------------------------
template <typename PlanT>
struct ChunkLoop {
  int* ctr;
  int nch, ngr, K, ntiles;
  int t, tend, hg, nxt, nxt_c, nt, gr, phase;
  bool sent, known;  // the next claim is sent / published

  // Claim c is tile chunk c / ngr of head group c % ngr, so the head groups
  // of a chunk run at about the same time and the rows they split are
  // fetched together.
  __device__ __forceinline__ int chunk_of(int c) const { return c / ngr; }
  __device__ __forceinline__ bool valid(int c) const { return chunk_of(c) < nch; }

  __device__ __forceinline__ ChunkLoop(const PlanT& pl, int* ctr_, int ngr_, int c)
      : ctr(ctr_), nch(pl.n_chunks), ngr(ngr_), K(pl.chunk_tiles), ntiles(pl.n_tiles) {
    hg = c % ngr;
    t = valid(c) ? chunk_of(c) * K : ntiles;
    tend = valid(c) ? cend(chunk_of(c)) : ntiles;
    nxt = -1;
    nxt_c = c;
    phase = 0;
    gr = 0;
    sent = known = false;
  }
  __device__ __forceinline__ int cend(int ch) const { return ch == nch - 1 ? ntiles : (ch + 1) * K; }

  template <typename ST>
  __device__ __forceinline__ void learn(ST& st) {
    nxt_c = uniform(st.tb.grab);
    nxt = valid(nxt_c) ? chunk_of(nxt_c) * K : -1;
    known = true;
  }

  // Prefetches the next tile. On the last tile of a chunk whose next claim
  // is not published yet (a chunk of one or two tiles) the claim completes
  // here, with a barrier.
  template <typename ST>
  __device__ __forceinline__ void begin_tile(ST& st) {
    const bool within = t + 1 < tend;
    if (!within && !known) {
      if (!sent && threadIdx.x == 0) gr = atomicAdd(ctr, 1);
      sent = true;
      if (threadIdx.x == 0) st.tb.grab = gr;
      __syncthreads();
      learn(st);
    }
    nt = within ? t + 1 : nxt;
    if (nt >= 0) st.prefetch(nt, within ? hg : nxt_c % ngr);
  }
  // Installs the next tile; false when the workgroup is done. The next claim
  // is sent at the end of a chunk's first tile and published at the end of
  // its second, so its round trip overlaps a whole tile and no wait
  // precedes the atomic.
  template <typename ST>
  __device__ __forceinline__ bool end_tile(ST& st) {
    if (nt < 0) return false;
    const bool cold = t + 1 >= tend;
    const bool pub = phase == 1 && !known;
    if (!sent && threadIdx.x == 0) gr = atomicAdd(ctr, 1);
    sent = true;
    st.commit(cold, pub, gr);
    if (pub) learn(st);
    if (cold) {
      tend = cend(chunk_of(nxt_c));
      hg = nxt_c % ngr;
      nxt = -1;
      phase = 0;
      sent = known = false;
    } else {
      ++phase;
    }
    t = nt;
    return true;
  }
};

// ---------------------------------------------------------------------------
// Forward: O and lse. A unit is a query block with UH heads of the group
// (the mask and the loop are shared by the heads; each head is its own
// chain of matrix steps).
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, int UH, typename PlanT>
__global__ __launch_bounds__(kThreads) void fwd_kernel(PlanT pl, const Tin* __restrict__ Q,
                                                       const Tin* __restrict__ K,
                                                       const Tin* __restrict__ V,
                                                       Tin* __restrict__ O,
                                                       float* __restrict__ lse, int H, float scale) {
  constexpr int KD = HD / 4;   // contraction dims per lane group
  constexpr int MT = HD / 16;  // 16-dim output tiles
  constexpr int NUH = HG / UH;
  using ST = BStream<HD, Tin, HG, 1, 0, PlanT>;
  constexpr int WS = ST::WS;
  __shared__ typename ST::Tables tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  int* ctr = pl.sched + 0;
  if (threadIdx.x == 0) tb.grab = atomicAdd(ctr, 1);
  ST st(pl, K, V, Q, nullptr, nullptr, nullptr, nullptr, H, 0, dyn, tb);
  ChunkLoop<PlanT> cl(pl, ctr, H / HG, uniform(tb.grab));  // the constructor's barrier publishes the claim
  if (cl.t >= cl.ntiles) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const float qscale = scale * kLog2e;
  const int P = st.P;
  st.prefetch(cl.t, cl.hg);
  st.commit(true);
  do {
    cl.begin_tile(st);
    __builtin_amdgcn_s_setprio(0);  // the block pairs at the base priority
    const int nqb = (st.ntile + kBlk - 1) / kBlk;
    const int pb0 = (P - st.A) / kBlk;  // first key block with prefix slots
    const int rb0 = P / kBlk;
    // At most NUH units per wave. The loop is unrolled: a loop that stores
    // but does not load has the compiler drain every memory operation before
    // it, the prefetch of the next tile included.
#pragma unroll
    for (int k = 0; k < NUH; ++k) {
      const int u = snake_unit(k, wave);
      if (u >= nqb * NUH) break;
      const int i = nqb - 1 - u / NUH;  // query block, longest first
      const int h0 = (u % NUH) * UH;    // first head of the unit (in the group)
      const int q = kBlk * i + c;
      Slice<Tin, KD> qf[UH];
      float m[UH], l[UH];
      f4 o[UH][MT];
#pragma unroll
      for (int e = 0; e < UH; ++e) {
        qf[e].load(st.Ts + q * WS + (h0 + e) * HD + KD * g);
        qf[e].scale(qscale);
        m[e] = -__builtin_inff();
        l[e] = 0.0f;
#pragma unroll
        for (int j = 0; j < MT; ++j) o[e][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      // The diagonal block first (it holds every row's own key), then the
      // prefix blocks and the row blocks above the diagonal. Which of them
      // have a live pair is one wave-uniform mask (lane n tests the n-th
      // block), not an LDS round trip at the top of every block.
      const int nb = i + rb0 - pb0 + 1;  // <= (P + kTile) / kBlk <= 20
      const uint32_t bmask = static_cast<uint32_t>(__ballot(
          lane < nb && kBlk * i < tb.bhi[lane == 0 ? rb0 + i : pb0 + min(lane, nb) - 1]));
      for (int n = 0, b = rb0 + i; n < nb; ++n, b = pb0 + n - 1) {
        if (!((bmask >> n) & 1u)) continue;  // no live pair
        const int k0 = kBlk * b;
        // The interval read is issued ahead of the first K read and product
        // (the scheduler would put it after the product and wait for it there).
        const int4 iv = *reinterpret_cast<const int4*>(tb.kint + k0 + 4 * g);
        __builtin_amdgcn_sched_barrier(0);
        const bool live[4] = {in_interval(q, iv.x), in_interval(q, iv.y), in_interval(q, iv.z),
                              in_interval(q, iv.w)};
#pragma unroll
        for (int e = 0; e < UH; ++e) {
          const int hoff = (h0 + e) * HD;
          Slice<Tin, KD> kf;
          kf.load(st.Ks + (k0 + c) * WS + hoff + KD * g);
          f4 sv = slice_dot(kf, qf[e], f4{0.0f, 0.0f, 0.0f, 0.0f});  // key k0+4g+r, query q
          if constexpr (!Slice<Tin, KD>::kPre) sv *= qscale;
          float sc[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[r] = live[r] ? sv[r] : -__builtin_inff();
          // The four-group max of a query passes m + 2^8 exactly when one of
          // its lanes' own maxima does, so the reduction runs only then.
          const float lmx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
          if (__any(lmx > m[e] + kRescaleLog2)) {
            const float mx = group_max(lmx);
            const bool resc = mx > m[e] + kRescaleLog2;
            const float a = resc ? fast_exp2(m[e] - mx) : 1.0f;
            m[e] = resc ? mx : m[e];
            l[e] *= a;
#pragma unroll
            for (int j = 0; j < MT; ++j) o[e][j] *= a;
          }
          float p[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[r] = fast_exp2(sc[r] - m[e]);  // masked: exp2(-inf) = 0
            l[e] += p[r];
          }
          if constexpr (sizeof(Tin) == 2) {
            // bf16 inputs: P rounded to bf16 (O is returned in bf16), one
            // 16-deep step per output tile: V[keys 4g..4g+3][dim c] against
            // this lane's P[query c][keys 4g..4g+3].
            const uint2 pw = pack_bf16(p);
#pragma unroll
            for (int j = 0; j < MT; ++j)
              o[e][j] = mfma_rows_bf16(st.Vs + (k0 + 4 * g) * WS + hoff + kBlk * j + c, WS, pw, o[e][j]);
          } else {
#pragma unroll
            for (int j = 0; j < MT; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                o[e][j] = mfma16(ld1(st.Vs + (k0 + 4 * g + r) * WS + hoff + kBlk * j + c), p[r], o[e][j]);
          }
        }
      }
      if (q < st.ntile) {
        const int64_t row = static_cast<int64_t>(st.s) + q;
#pragma unroll
        for (int e = 0; e < UH; ++e) {
          const float le = group_sum(l[e]);
          const float inv = __builtin_amdgcn_rcpf(le);
          const int h = st.hg * HG + h0 + e;
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            float v[4] = {o[e][j][0] * inv, o[e][j][1] * inv, o[e][j][2] * inv, o[e][j][3] * inv};
            store_vec<4>(O + row * D + h * HD + kBlk * j + 4 * g, v);
          }
          if (g == 0) lse[row * H + h] = (m[e] + fast_log2(le)) * kLn2;
        }
      }
    }
    // the next tile's install and its barriers ahead of the other
    // workgroups' block pairs (as in the backward: 14.18 -> 14.11 ms)
    __builtin_amdgcn_s_setprio(3);
  } while (cl.end_tile(st));
}

// ---------------------------------------------------------------------------
// Backward, query side: δ and dQ. δ = dO·O for fp32 inputs (from the chunk
// partials); for bf16 inputs O is a rounded output, so δ = Σ_j w_j dO·v_j is
// recomputed over the path in fp32 (batched_depth_backward.cr:637-646). δ is
// written to Dl [T, H] for the key side.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, int UH, typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) void bwd_q_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const Tin* __restrict__ O, const float* __restrict__ lse, const Tin* __restrict__ dO,
    float* __restrict__ dQ, float* __restrict__ Dl, RopeT rope, int H, float scale) {
  constexpr int KD = HD / 4;
  constexpr int MT = HD / 16;
  constexpr int NUH = HG / UH;
  constexpr bool kDeltaFromO = sizeof(Tin) == sizeof(float);
  constexpr int NT = kDeltaFromO ? 3 : 2;
  using ST = BStream<HD, Tin, HG, NT, kLse, PlanT>;
  constexpr int WS = ST::WS;
  __shared__ typename ST::Tables tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  int* ctr = pl.sched + 1;
  if (threadIdx.x == 0) tb.grab = atomicAdd(ctr, 1);
  ST st(pl, K, V, Q, dO, O, lse, nullptr, H, 0, dyn, tb);
  ChunkLoop<PlanT> cl(pl, ctr, H / HG, uniform(tb.grab));  // the constructor's barrier publishes the claim
  if (cl.t >= cl.ntiles) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const float qscale = scale * kLog2e;
  const int P = st.P;
  const Tin* Qs = st.Ts;
  const Tin* Gs = st.Ts + kTile * WS;
  st.prefetch(cl.t, cl.hg);
  st.commit(true);
  do {
    cl.begin_tile(st);
    const int nqb = (st.ntile + kBlk - 1) / kBlk;
    const int pb0 = (P - st.A) / kBlk;
    const int rb0 = P / kBlk;
    for (int k = 0;; ++k) {
      const int u = snake_unit(k, wave);
      if (u >= nqb * NUH) break;
      const int i = nqb - 1 - u / NUH;
      const int h0 = (u % NUH) * UH;
      const int q = kBlk * i + c;
      Slice<Tin, KD> qf[UH], gf[UH];
      float l2[UH], dl[UH];
      f4 dq[UH][MT];
#pragma unroll
      for (int e = 0; e < UH; ++e) {
        qf[e].load(Qs + q * WS + (h0 + e) * HD + KD * g);
        gf[e].load(Gs + q * WS + (h0 + e) * HD + KD * g);
        qf[e].scale(qscale);
        l2[e] = tb.l2[h0 + e][q];
#pragma unroll
        for (int j = 0; j < MT; ++j) dq[e][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      // Scores and dO·v of head e against key block k0: register r holds key
      // k0+4g+r against query q.
      auto scores = [&](int e, int k0, f4& sv, f4& tv) {
        const int hoff = (h0 + e) * HD;
        Slice<Tin, KD> kf, vf;
        kf.load(st.Ks + (k0 + c) * WS + hoff + KD * g);
        vf.load(st.Vs + (k0 + c) * WS + hoff + KD * g);
        sv = slice_dot(kf, qf[e], f4{0.0f, 0.0f, 0.0f, 0.0f});
        tv = slice_dot(vf, gf[e], f4{0.0f, 0.0f, 0.0f, 0.0f});
        if constexpr (!Slice<Tin, KD>::kPre) sv *= qscale;
      };
      auto mask = [&](int k0, bool (&live)[4]) {
        const int4 iv = *reinterpret_cast<const int4*>(tb.kint + k0 + 4 * g);
        live[0] = in_interval(q, iv.x);
        live[1] = in_interval(q, iv.y);
        live[2] = in_interval(q, iv.z);
        live[3] = in_interval(q, iv.w);
      };
      const int nblk = i + rb0 - pb0;  // blocks after the diagonal one
      if constexpr (kDeltaFromO) {
#pragma unroll
        for (int e = 0; e < UH; ++e) {
          dl[e] = 0.0f;
          const float* pp = st.pdl + (q * HG + h0 + e) * ST::CPH;
#pragma unroll
          for (int j = 0; j < ST::CPH; ++j) dl[e] += pp[j];
        }
      } else {
        float acc[UH];
#pragma unroll
        for (int e = 0; e < UH; ++e) acc[e] = 0.0f;
        for (int n = 0, b = rb0 + i; n <= nblk; ++n, b = pb0 + n - 1) {
          if (kBlk * i >= uniform(tb.bhi[b])) continue;
          bool live[4];
          mask(kBlk * b, live);
#pragma unroll
          for (int e = 0; e < UH; ++e) {
            f4 sv, tv;
            scores(e, kBlk * b, sv, tv);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[e] += live[r] ? fast_exp2(sv[r] - l2[e]) * tv[r] : 0.0f;
          }
        }
#pragma unroll
        for (int e = 0; e < UH; ++e) dl[e] = group_sum(acc[e]);
      }
      for (int n = 0, b = rb0 + i; n <= nblk; ++n, b = pb0 + n - 1) {
        if (kBlk * i >= uniform(tb.bhi[b])) continue;
        const int k0 = kBlk * b;
        bool live[4];
        mask(k0, live);
#pragma unroll
        for (int e = 0; e < UH; ++e) {
          f4 sv, tv;
          scores(e, k0, sv, tv);
          float ds[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            ds[r] = live[r] ? fast_exp2(sv[r] - l2[e]) * (tv[r] - dl[e]) * scale : 0.0f;
          const int hoff = (h0 + e) * HD;
          if constexpr (sizeof(Tin) == 2) {  // dS rounded to bf16, one 16-deep step per tile
            const uint2 dw = pack_bf16(ds);
#pragma unroll
            for (int j = 0; j < MT; ++j)
              dq[e][j] = mfma_rows_bf16(st.Ks + (k0 + 4 * g) * WS + hoff + kBlk * j + c, WS, dw, dq[e][j]);
          } else {
#pragma unroll
            for (int j = 0; j < MT; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                dq[e][j] = mfma16(ld1(st.Ks + (k0 + 4 * g + r) * WS + hoff + kBlk * j + c), ds[r], dq[e][j]);
          }
        }
      }
      if (q < st.ntile) {
        const int64_t row = static_cast<int64_t>(st.s) + q;
        const int pos = rope.cos_t ? rope_pos(tb.depth[q], rope.seq_len) : 0;
#pragma unroll
        for (int e = 0; e < UH; ++e) {
          const int h = st.hg * HG + h0 + e;
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            float v[4] = {dq[e][j][0], dq[e][j][1], dq[e][j][2], dq[e][j][3]};
            if (rope.cos_t) agpt_fast::rope_inverse_part<4, HD>(v, rope.cos_t, rope.sin_t, pos, kBlk * j + 4 * g);
            store_vec<4>(dQ + row * D + h * HD + kBlk * j + 4 * g, v);
          }
          if (g == 0) Dl[row * H + h] = dl[e];
        }
      }
    }
  } while (cl.end_tile(st));
}

// ---------------------------------------------------------------------------
// Backward, key side: dK / dV of the tile's key set, a unit being a key
// block with UH heads. Prefix keys leave their partial over this tile in
// Pk/Pv (row pref_off[t] + depth-1); tile rows whose subtree ends inside the
// tile are finished here (seed, inverse RoPE); open tile rows leave their
// partial in dK/dV for the reduction kernels.
// ---------------------------------------------------------------------------
template <int HD, typename Tin, int HG, int UH, typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) void bwd_kv_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const float* __restrict__ lse, const float* __restrict__ Dl, const Tin* __restrict__ dO,
    float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ Pk, float* __restrict__ Pv,
    const float* __restrict__ acc_dk, const float* __restrict__ acc_dv, RopeT rope, int H,
    float scale) {
  constexpr int KD = HD / 4;
  constexpr int MT = HD / 16;
  constexpr int NUH = HG / UH;
  using ST = BStream<HD, Tin, HG, 2, kLse | kDl, PlanT>;
  constexpr int WS = ST::WS;
  __shared__ typename ST::Tables tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  int* ctr = pl.sched + 2;
  if (threadIdx.x == 0) tb.grab = atomicAdd(ctr, 1);
  ST st(pl, K, V, Q, dO, nullptr, lse, Dl, H, 0, dyn, tb);
  ChunkLoop<PlanT> cl(pl, ctr, H / HG, uniform(tb.grab));  // the constructor's barrier publishes the claim
  if (cl.t >= cl.ntiles) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const float qscale = scale * kLog2e;
  const int P = st.P;
  const Tin* Qs = st.Ts;
  const Tin* Gs = st.Ts + kTile * WS;
  st.prefetch(cl.t, cl.hg);
  st.commit(true);
  do {
    cl.begin_tile(st);
    const int nrb = (st.ntile + kBlk - 1) / kBlk;
    const int pb0 = (P - st.A) / kBlk;
    const int rb0 = P / kBlk;
    const int nkb = rb0 - pb0 + nrb;  // prefix blocks (shallowest first), then row blocks
    for (int k = 0;; ++k) {
      const int u = snake_unit(k, wave);
      if (u >= nkb * NUH) break;
      const int b = pb0 + u / NUH;
      const int h0 = (u % NUH) * UH;
      const int kslot = kBlk * b + c;  // this lane's key
      Slice<Tin, KD> kf[UH], vf[UH];
      f4 dk[UH][MT], dv[UH][MT];
#pragma unroll
      for (int e = 0; e < UH; ++e) {
        kf[e].load(st.Ks + kslot * WS + (h0 + e) * HD + KD * g);
        vf[e].load(st.Vs + kslot * WS + (h0 + e) * HD + KD * g);
        kf[e].scale(qscale);
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          dk[e][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
          dv[e][j] = dk[e][j];
        }
      }
      const int iv = tb.kint[kslot];
      const int i0 = b < rb0 ? 0 : b - rb0;
      const int i1 = uniform((tb.bhi[b] + kBlk - 1) / kBlk);
      for (int i = i0; i < i1; ++i) {
        const int qr = kBlk * i + c;  // query row this lane supplies
        const int q0 = kBlk * i + 4 * g;
        bool live[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) live[r] = in_interval(q0 + r, iv);
#pragma unroll
        for (int e = 0; e < UH; ++e) {
          const int hoff = (h0 + e) * HD;
          Slice<Tin, KD> qa, ga;
          qa.load(Qs + qr * WS + hoff + KD * g);
          ga.load(Gs + qr * WS + hoff + KD * g);
          f4 sv = slice_dot(qa, kf[e], f4{0.0f, 0.0f, 0.0f, 0.0f});  // sv[r]: query q0+r against key kslot
          const f4 tv = slice_dot(ga, vf[e], f4{0.0f, 0.0f, 0.0f, 0.0f});
          if constexpr (!Slice<Tin, KD>::kPre) sv *= qscale;
          const f4 l2v = *reinterpret_cast<const f4*>(&tb.l2[h0 + e][q0]);
          const f4 dlv = *reinterpret_cast<const f4*>(&tb.dl[h0 + e][q0]);
          float p[4], ds[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[r] = live[r] ? fast_exp2(sv[r] - l2v[r]) : 0.0f;
            ds[r] = live[r] ? p[r] * (tv[r] - dlv[r]) * scale : 0.0f;
          }
          if constexpr (sizeof(Tin) == 2) {  // P and dS rounded to bf16, one 16-deep step per tile
            const uint2 pw = pack_bf16(p), dw = pack_bf16(ds);
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              const int col = q0 * WS + hoff + kBlk * j + c;
              dv[e][j] = mfma_rows_bf16(Gs + col, WS, pw, dv[e][j]);
              dk[e][j] = mfma_rows_bf16(Qs + col, WS, dw, dk[e][j]);
            }
          } else {
#pragma unroll
            for (int j = 0; j < MT; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int row = (q0 + r) * WS + hoff + kBlk * j + c;
                dv[e][j] = mfma16(ld1(Gs + row), p[r], dv[e][j]);
                dk[e][j] = mfma16(ld1(Qs + row), ds[r], dk[e][j]);
              }
          }
        }
      }
      // Emit dims 16j+4g.. of key kslot.
      if (kslot < P) {
        const int d = kslot - (P - st.A);
        if (d >= 0) {
          const int64_t row = static_cast<int64_t>(st.poff) + d;
#pragma unroll
          for (int e = 0; e < UH; ++e) {
            const int hd = st.hg * HG + h0 + e;
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              float a[4] = {dk[e][j][0], dk[e][j][1], dk[e][j][2], dk[e][j][3]};
              float v[4] = {dv[e][j][0], dv[e][j][1], dv[e][j][2], dv[e][j][3]};
              store_vec<4>(Pk + row * D + hd * HD + kBlk * j + 4 * g, a);
              store_vec<4>(Pv + row * D + hd * HD + kBlk * j + 4 * g, v);
            }
          }
        }
      } else {
        const int r = kslot - P;
        if (r < st.ntile) {
          const int64_t a = static_cast<int64_t>(st.s) + r;
          const bool done = tb.tend[r] <= st.s + st.ntile;
          const int pos = rope.cos_t ? rope_pos(tb.depth[r], rope.seq_len) : 0;
#pragma unroll
          for (int e = 0; e < UH; ++e) {
            const int hd = st.hg * HG + h0 + e;
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              const int d0 = kBlk * j + 4 * g;
              float gk[4] = {dk[e][j][0], dk[e][j][1], dk[e][j][2], dk[e][j][3]};
              float gv[4] = {dv[e][j][0], dv[e][j][1], dv[e][j][2], dv[e][j][3]};
              if (done) {
                if (acc_dk) {
                  float y[4];
                  load_vec<4>(acc_dk + a * D + hd * HD + d0, y);
#pragma unroll
                  for (int x = 0; x < 4; ++x) gk[x] += y[x];
                }
                if (acc_dv) {
                  float y[4];
                  load_vec<4>(acc_dv + a * D + hd * HD + d0, y);
#pragma unroll
                  for (int x = 0; x < 4; ++x) gv[x] += y[x];
                }
                if (rope.cos_t) agpt_fast::rope_inverse_part<4, HD>(gk, rope.cos_t, rope.sin_t, pos, d0);
              }
              store_vec<4>(dK + a * D + hd * HD + d0, gk);
              store_vec<4>(dV + a * D + hd * HD + d0, gv);
            }
          }
        }
      }
    }
  } while (cl.end_tile(st));
}

// ---------------------------------------------------------------------------
// Fused backward (fp32 inputs): dQ, dK, dV in one pass over the tiles. A
// unit is a key block of one head (kv orientation: S = Q_i K^T puts key c in
// lane column c). Per block pair (query block i, key block) the scores, P,
// dP and dS are formed once and feed
//   dV^T += dO^T P,   dK^T += Q^T dS    (registers of the unit, emitted at
//                                        its end as in bwd_kv_kernel),
//   dQ_i^T += K^T dS^T                   (dS transposed through a per-wave
//                                        LDS tile; accumulated in the
//                                        wave's own LDS dQ tile).
// Each head of the group has kWaves / HG waves of its own; the units of a
// head (its key blocks) are dealt to them longest first, each to the least
// loaded wave (every wave computes the same assignment). After the units
// the workgroup sums each head's wave tiles of dQ in wave order, then
// applies inverse RoPE: the order of every sum is fixed, so results are
// bitwise reproducible. δ = dO·O comes with the tile (the stream reduces
// the fetched O). Two heads per workgroup (HG = 2) fetch whole 128-byte
// row segments at hd 16, where one head would leave half of every fetched
// line to another workgroup.
// ---------------------------------------------------------------------------
//
// Path carry (kCarry). Within a chunk a workgroup visits consecutive tiles,
// and the keys a tile leaves open (subtree not finished) are exactly the
// prefix of the next tile: the ancestors of its first row, one per depth.
// So instead of one partial per (tile, prefix key) the workgroup keeps the
// dK/dV sums of the current path in LDS, indexed by depth: a prefix key
// that the next tile still sees adds its tile sum there; one that it does
// not see is finished: its total goes to dK/dV (a key first seen in this
// chunk whose subtree ends here), or to the chunk's partial E[chunk][depth]
// (a key from before the chunk), or at the chunk's end to F[chunk][depth]
// (a key of this chunk still open). Open tile rows start their depth's sum.
// The sums live in two copies by tile parity: a tile reads its prefix's
// sums from one and writes the next tile's into the other, so a sum that
// ends and the one that replaces it at the same depth never meet. With the
// carry each wave also keeps its dQ in registers (one 16x16 block per query
// block of the tile), summed across the head's waves through LDS at the end
// of the tile; bwd_carry_kernel then adds F and the later chunks' E in
// chunk order.
// ---------------------------------------------------------------------------
// LDS past the stream. Without the carry: dQ partials [wave][kTile][HD]
// (each wave serves one head) and dS^T tiles [wave][16][20]. With it: the
// dS^T tiles, the path sums [2][P][HG][2 * HD + 4] (dK, dV; padded) and the
// row of each depth [2][P].
__host__ __device__ constexpr int carry_stride(int HD) { return 2 * HD + 4; }
__host__ __device__ constexpr size_t carry_bytes(int max_depth, int HG, int HD) {
  return 2 * static_cast<size_t>(prefix_cap(max_depth)) * (HG * carry_stride(HD) + 1) * sizeof(float);
}
__host__ __device__ inline size_t fused_lds_bytes(int max_depth, int HG, int HD, bool carry) {
  const size_t tr = static_cast<size_t>(kWaves) * kBlk * 20 * sizeof(float);
  return block_lds_bytes(max_depth, HG, HD, sizeof(float), 2, false) + tr +
         (carry ? carry_bytes(max_depth, HG, HD) : static_cast<size_t>(kWaves) * kTile * HD * sizeof(float));
}

template <int HD, typename Tin, int HG, bool kCarry, typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) void bwd_kernel(
    PlanT pl, const Tin* __restrict__ Q, const Tin* __restrict__ K, const Tin* __restrict__ V,
    const Tin* __restrict__ O, const float* __restrict__ lse, const Tin* __restrict__ dO,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ Pk,
    float* __restrict__ Pv, const float* __restrict__ acc_dk, const float* __restrict__ acc_dv,
    RopeT rope, int H, float scale) {
  // With the carry, Pk holds E and Pv holds F: [n_chunks][P][2][D] (dK, dV).

  static_assert(sizeof(Tin) == sizeof(float), "the fused backward takes fp32 inputs (δ = dO·O)");
  static_assert(kWaves % HG == 0, "whole waves per head");
  constexpr int WPH = kWaves / HG;  // waves per head
  constexpr int KD = HD / 4;
  constexpr int MT = HD / 16;
  using ST = BStream<HD, Tin, HG, 3, kLse | kDeltaO, PlanT>;
  constexpr int WS = ST::WS;
  __shared__ typename ST::Tables tb;
  extern __shared__ __align__(16) unsigned char dyn[];
  int* ctr = pl.sched + 1;
  if (threadIdx.x == 0) tb.grab = atomicAdd(ctr, 1);
  ST st(pl, K, V, Q, dO, O, lse, nullptr, H, 0, dyn, tb);
  st.dscale = scale;  // dS = P (dP - δ) scale, with V and δ taken times scale
  ChunkLoop<PlanT> cl(pl, ctr, H / HG, uniform(tb.grab));  // the constructor's barrier publishes the claim
  if (cl.t >= cl.ntiles) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int D = H * HD;
  const float qscale = scale * kLog2e;
  const int P = st.P;
  const Tin* Qs = st.Ts;
  const Tin* Gs = st.Ts + kTile * WS;
  constexpr int NQB = kTile / kBlk;  // query blocks of a tile
  constexpr int CS = carry_stride(HD);
  float* scr = reinterpret_cast<float*>(dyn + ST::lds_bytes(pl.max_depth));
  float* dqs = scr;                                                         // [wave][kTile][HD] (no carry)
  float* tr = scr + (kCarry ? 0 : kWaves * kTile * HD) + wave * (kBlk * 20);  // this wave's dS^T tile
  float* cry = scr + kWaves * kBlk * 20;                 // [2][P][HG][CS] path sums (carry)
  int* cid = reinterpret_cast<int*>(cry + 2 * P * HG * CS);  // [2][P] row of each depth; -1: from before the chunk
  // Staged Q and dO, free once a tile's units are done, carry the dQ sums
  // across waves: two [NQB][MT][64] f4 slots.
  static_assert(2 * NQB * MT * 64 * 4 <= 2 * kTile * WS, "dQ exchange fits the staged tile");
  const int hh = wave / WPH;  // this wave's head of the group
  const int wl = wave % WPH;  // and its place among that head's waves
  st.prefetch(cl.t, cl.hg);
  st.commit(true);
  bool more;
  do {
    cl.begin_tile(st);
    const int nrb = (st.ntile + kBlk - 1) / kBlk;
    const int pb0 = (P - st.A) / kBlk;
    const int rb0 = P / kBlk;
    const int npu = rb0 - pb0;       // prefix units of a head
    const int nu = npu + nrb;        // units of a head: key blocks, prefix first
    // Chunk of the tile and its place in it (the last chunk runs to the end).
    const int chunk = min(cl.t / cl.K, cl.nch - 1);
    const bool first = cl.t == chunk * cl.K;
    const bool last = cl.t + 1 == cl.tend;
    const int cur = cl.t & 1;  // path sums of this tile's prefix; the next tile's are in cur ^ 1
    // This wave's dQ starts at zero: registers with the carry, else its LDS tile.
    float* mydq = dqs + wave * kTile * HD;
    f4 dqr[NQB][MT];
#pragma unroll
    for (int x = 0; x < NQB; ++x)
#pragma unroll
      for (int j = 0; j < MT; ++j) dqr[x][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (!kCarry)
      for (int x = lane; x < kTile * HD / 4; x += 64) reinterpret_cast<f4*>(mydq)[x] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    int load0 = 0, load1 = 0, load2 = 0, load3 = 0;
    // The units' query-block ends, read once: lane u holds unit u's (nu <=
    // (P + kTile) / kBlk <= 20), taken out with a lane read per unit instead
    // of an LDS round trip per unit in every wave.
    const int bh = tb.bhi[pb0 + min(lane, nu - 1)];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): bh is in before the loop
    __builtin_amdgcn_s_setprio(0);  // the block pairs at the base priority
    for (int u = 0; u < nu; ++u) {
      const int b = pb0 + u;
      const int i0 = b < rb0 ? 0 : b - rb0;
      const int i1 = (__builtin_amdgcn_readlane(bh, u) + kBlk - 1) / kBlk;
      // Least loaded wave of the head (lowest index on ties) takes the unit.
      const int cost = i1 - i0;
      int w = 0;
      if constexpr (WPH == 4) {
        int lmin = load0;
        if (load1 < lmin) { w = 1; lmin = load1; }
        if (load2 < lmin) { w = 2; lmin = load2; }
        if (load3 < lmin) { w = 3; lmin = load3; }
        if (w == 0) load0 += cost;
        else if (w == 1) load1 += cost;
        else if (w == 2) load2 += cost;
        else load3 += cost;
      } else if constexpr (WPH == 2) {
        w = load1 < load0 ? 1 : 0;
        if (w == 0) load0 += cost;
        else load1 += cost;
      }
      if (w != wl) continue;
      const int hoff = hh * HD;
      const int kslot = kBlk * b + c;  // this lane's key
      float kf[KD], vf[KD], kt[MT][4];
      load_vec<KD>(st.Ks + kslot * WS + hoff + KD * g, kf);
      load_vec<KD>(st.Vs + kslot * WS + hoff + KD * g, vf);
#pragma unroll
      for (int j = 0; j < KD; ++j) {
        kf[j] *= qscale;
        vf[j] *= scale;
      }
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) kt[t][r] = ld1(st.Ks + (kBlk * b + 4 * g + r) * WS + hoff + kBlk * t + c);
      const int iv = tb.kint[kslot];
      f4 dk[MT], dv[MT];
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        dk[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        dv[j] = dk[j];
      }
      // Block pair (query block i, this key block): S, P, dP, dS once; dV, dK
      // in registers; dS^T back in dst for the dQ product (the dV, dK
      // products sit between its LDS write and read).
      auto pair = [&](const int i, float (&dst)[4]) {
        const int qr = kBlk * i + c;  // query row this lane supplies
        const int q0 = kBlk * i + 4 * g;
        // Every LDS read of the pair is issued before its first product and
        // before the dS^T store (which the reads could not pass), so their
        // latency hides behind the S products.
        float qa[KD], ga[KD], gcol[MT][4], qcol[MT][4];
        load_vec<KD>(Qs + qr * WS + hoff + KD * g, qa);
        load_vec<KD>(Gs + qr * WS + hoff + KD * g, ga);
        const f4 l2v = *reinterpret_cast<const f4*>(&tb.l2[hh][q0]);
        const f4 dlv = *reinterpret_cast<const f4*>(&tb.dl[hh][q0]);
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = (q0 + r) * WS + hoff + kBlk * j + c;
            gcol[j][r] = ld1(Gs + row);
            qcol[j][r] = ld1(Qs + row);
          }
        __builtin_amdgcn_sched_barrier(0);  // (the scheduler would sink them past the S products)
        f4 sv = f4{0.0f, 0.0f, 0.0f, 0.0f}, tv = sv;
#pragma unroll
        for (int j = 0; j < KD; ++j) {
          sv = mfma16(qa[j], kf[j], sv);  // sv[r]: query q0+r against key kslot
          tv = mfma16(ga[j], vf[j], tv);
        }
        float p[4], ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool live = in_interval(q0 + r, iv);
          p[r] = live ? fast_exp2(sv[r] - l2v[r]) : 0.0f;
          ds[r] = p[r] * (tv[r] - dlv[r]);  // tv, dlv carry the scale; zero where p is
        }
        // dS^T for the dQ product: write key c's four queries, read back
        // query c's four keys (LDS operations of a wave complete in order).
        *reinterpret_cast<f4*>(tr + c * 20 + 4 * g) = f4{ds[0], ds[1], ds[2], ds[3]};
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            dv[j] = mfma16(gcol[j][r], p[r], dv[j]);
            dk[j] = mfma16(qcol[j][r], ds[r], dk[j]);
          }
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = tr[(4 * g + r) * 20 + c];
      };
      // lane: dims 16j+4g.. of query row kBlk * i + c
      if constexpr (kCarry) {
        // Unrolled over the tile's query blocks (uniform guards), so each
        // block pair is straight-line code with its own dQ registers.
#pragma unroll
        for (int i = 0; i < NQB; ++i) {
          if (i < i0 || i >= i1) continue;
          float dst[4];
          pair(i, dst);
#pragma unroll
          for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) dqr[i][j] = mfma16(kt[j][r], dst[r], dqr[i][j]);
        }
      } else {
        for (int i = i0; i < i1; ++i) {
          float dst[4];
          pair(i, dst);
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            f4* dqp = reinterpret_cast<f4*>(mydq + (kBlk * i + c) * HD + kBlk * j + 4 * g);
            f4 acc = *dqp;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc = mfma16(kt[j][r], dst[r], acc);
            *dqp = acc;
          }
        }
      }
      // Emit dims 16j+4g.. of key kslot.
      const int hd = st.hg * HG + hh;
      float gk[MT][4], gv[MT][4];
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          gk[j][x] = dk[j][x];
          gv[j][x] = dv[j][x];
        }
      // Final dK/dV of row a at depth dep: + seeds, inverse RoPE of dK.
      auto finish = [&](int64_t a, int dep) {
        const int pos = rope.cos_t ? rope_pos(dep, rope.seq_len) : 0;
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const int d0 = kBlk * j + 4 * g;
          if (acc_dk) {
            float y[4];
            load_vec<4>(acc_dk + a * D + hd * HD + d0, y);
#pragma unroll
            for (int x = 0; x < 4; ++x) gk[j][x] += y[x];
          }
          if (acc_dv) {
            float y[4];
            load_vec<4>(acc_dv + a * D + hd * HD + d0, y);
#pragma unroll
            for (int x = 0; x < 4; ++x) gv[j][x] += y[x];
          }
          if (rope.cos_t) agpt_fast::rope_inverse_part<4, HD>(gk[j], rope.cos_t, rope.sin_t, pos, d0);
          store_vec<4>(dK + a * D + hd * HD + d0, gk[j]);
          store_vec<4>(dV + a * D + hd * HD + d0, gv[j]);
        }
      };
      // A chunk partial (E or F) of depth entry d.
      auto chunk_part = [&](float* base, int d) {
        float* o = base + (static_cast<int64_t>(chunk) * P + d) * 2 * D + hd * HD + 4 * g;
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          store_vec<4>(o + kBlk * j, gk[j]);
          store_vec<4>(o + D + kBlk * j, gv[j]);
        }
      };
      if (kslot < P) {
        const int d = kslot - (P - st.A);
        if (d >= 0) {
          if constexpr (kCarry) {
            const int e = tb.pend[d];
            const bool cont = !last && e > st.s + st.ntile;  // the next tile of the chunk sees it
            const float* cp = cry + ((cur * P + d) * HG + hh) * CS + 4 * g;
            float* np = cry + (((cur ^ 1) * P + d) * HG + hh) * CS + 4 * g;
            const int id = first ? -1 : cid[cur * P + d];
            if (!first) {
#pragma unroll
              for (int j = 0; j < MT; ++j) {
                const f4 ck = *reinterpret_cast<const f4*>(cp + kBlk * j);
                const f4 cv = *reinterpret_cast<const f4*>(cp + HD + kBlk * j);
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                  gk[j][x] = ck[x] + gk[j][x];
                  gv[j][x] = cv[x] + gv[j][x];
                }
              }
            }
            if (cont) {
#pragma unroll
              for (int j = 0; j < MT; ++j) {
                store_vec<4>(np + kBlk * j, gk[j]);
                store_vec<4>(np + HD + kBlk * j, gv[j]);
              }
              if (hh == 0 && g == 0) cid[(cur ^ 1) * P + d] = id;
            } else if (id < 0) {
              chunk_part(Pk, d);  // E: a key from before the chunk
            } else if (e > st.s + st.ntile) {
              chunk_part(Pv, d);  // F: the chunk ends, the key's subtree does not
            } else {
              finish(id, d + 1);
            }
          } else {
            const int64_t row = static_cast<int64_t>(st.poff) + d;
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              store_vec<4>(Pk + row * D + hd * HD + kBlk * j + 4 * g, gk[j]);
              store_vec<4>(Pv + row * D + hd * HD + kBlk * j + 4 * g, gv[j]);
            }
          }
        }
      } else {
        const int r = kslot - P;
        if (r < st.ntile) {
          const int64_t a = static_cast<int64_t>(st.s) + r;
          if (tb.tend[r] <= st.s + st.ntile) {
            finish(a, tb.depth[r]);
          } else if constexpr (kCarry) {
            const int d = tb.depth[r] - 1;  // the row's depth entry in the next tile's prefix
            if (last) {
              chunk_part(Pv, d);
            } else {
              float* np = cry + (((cur ^ 1) * P + d) * HG + hh) * CS + 4 * g;
#pragma unroll
              for (int j = 0; j < MT; ++j) {
                store_vec<4>(np + kBlk * j, gk[j]);
                store_vec<4>(np + HD + kBlk * j, gv[j]);
              }
              if (hh == 0 && g == 0) cid[(cur ^ 1) * P + d] = static_cast<int>(a);
            }
          } else {
            // Open row: its partial over this tile, finished by the reduction.
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              store_vec<4>(dK + a * D + hd * HD + kBlk * j + 4 * g, gk[j]);
              store_vec<4>(dV + a * D + hd * HD + kBlk * j + 4 * g, gv[j]);
            }
          }
        }
      }
    }
    // dQ is held in registers while the next tile is installed and stored
    // after it: the install waits for the prefetched rows, and the memory
    // counter retires operations in issue order, so a store issued before it
    // would be waited for too.
    if constexpr (kCarry) {
      // The head's wave sums, added in the fixed order ((w0 + w1) + (w2 + w3)).
      // The tile's end (the dQ exchange, the next tile's install and its
      // barriers) at a higher wave priority than the block pairs: a wave
      // that reaches it gets its LDS traffic and barrier out ahead of the
      // other workgroup's matrix work, so its workgroup waits less at the
      // barriers (trie_bwd 33.48 -> 32.83 ms; level 1 gave 32.87).
      __builtin_amdgcn_s_setprio(3);
      __syncthreads();  // every unit is done: the staged Q and dO are free
      f4* xs = reinterpret_cast<f4*>(st.Ts);
      auto slot = [&](int k, int x, int j) { return xs + ((k * NQB + x) * MT + j) * 64 + lane; };
      if constexpr (WPH == 2) {
        if (wl == 1)
#pragma unroll
          for (int x = 0; x < NQB; ++x)
#pragma unroll
            for (int j = 0; j < MT; ++j) *slot(hh, x, j) = dqr[x][j];
        __syncthreads();
        if (wl == 0)
#pragma unroll
          for (int x = 0; x < NQB; ++x)
#pragma unroll
            for (int j = 0; j < MT; ++j) dqr[x][j] += *slot(hh, x, j);
      } else if constexpr (WPH == 4) {
        if (wl & 1)
#pragma unroll
          for (int x = 0; x < NQB; ++x)
#pragma unroll
            for (int j = 0; j < MT; ++j) *slot(wl >> 1, x, j) = dqr[x][j];
        __syncthreads();
        if ((wl & 1) == 0) {
#pragma unroll
          for (int x = 0; x < NQB; ++x)
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              dqr[x][j] += *slot(wl >> 1, x, j);
              if (wl == 2) *slot(1, x, j) = dqr[x][j];
            }
        }
        __syncthreads();
        if (wl == 0)
#pragma unroll
          for (int x = 0; x < NQB; ++x)
#pragma unroll
            for (int j = 0; j < MT; ++j) dqr[x][j] += *slot(1, x, j);
      }
      const int64_t s0 = st.s;
      const int nt0 = st.ntile;
      const int col = (st.hg * HG + hh) * HD + 4 * g;
      float qv[NQB][MT][4];
#pragma unroll
      for (int x = 0; x < NQB; ++x)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
#pragma unroll
          for (int r = 0; r < 4; ++r) qv[x][j][r] = dqr[x][j][r];
          const int q = kBlk * x + c;
          if (wl == 0 && rope.cos_t && q < nt0)
            agpt_fast::rope_inverse_part<4, HD>(qv[x][j], rope.cos_t, rope.sin_t, rope_pos(tb.depth[q], rope.seq_len),
                                                kBlk * j + 4 * g);
        }
      more = cl.end_tile(st);
      if (wl == 0)
#pragma unroll
        for (int x = 0; x < NQB; ++x) {
          const int q = kBlk * x + c;
          if (q < nt0)
#pragma unroll
            for (int j = 0; j < MT; ++j) store_vec<4>(dQ + (s0 + q) * D + col + kBlk * j, qv[x][j]);
        }
      continue;
    }
    // The waves' dQ tiles of each head, summed in wave order.
    __syncthreads();
    constexpr int kQuads = HG * kTile * HD / 4;  // 4 consecutive dims of a row of a head
    static_assert(kQuads % kThreads == 0, "whole dQ quads per thread");
    constexpr int kPer = kQuads / kThreads;
    float qv[kPer][4];
    int64_t qo[kPer];  // element offset of the quad in dQ; -1: row past the tile
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int x = threadIdx.x + k * kThreads;
      const int e = x / (kTile * HD / 4);
      const int rem = x - e * (kTile * HD / 4);
      const int q = rem / (HD / 4);
      const int d0 = (rem - q * (HD / 4)) * 4;
      f4 sum = *reinterpret_cast<const f4*>(dqs + (e * WPH * kTile + q) * HD + d0);
#pragma unroll
      for (int w = 1; w < WPH; ++w) sum += *reinterpret_cast<const f4*>(dqs + ((e * WPH + w) * kTile + q) * HD + d0);
#pragma unroll
      for (int r = 0; r < 4; ++r) qv[k][r] = sum[r];
      if (rope.cos_t && q < st.ntile)
        agpt_fast::rope_inverse_part<4, HD>(qv[k], rope.cos_t, rope.sin_t, rope_pos(tb.depth[q], rope.seq_len), d0);
      qo[k] = q < st.ntile ? (static_cast<int64_t>(st.s) + q) * D + (st.hg * HG + e) * HD + d0 : -1;
    }
    more = cl.end_tile(st);
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (qo[k] >= 0) store_vec<4>(dQ + qo[k], qv[k]);
  } while (more);
}

// ---------------------------------------------------------------------------
// Carry reduction: one workgroup per chunk C but the last. The keys first
// seen in chunk C and still open at its end are the prefix entries d of the
// next chunk's first tile with row >= the chunk's first row; each one's
// total is F[C][d] + Σ E[C'][d] over the later chunks C' whose first row
// lies in its subtree (those are exactly the chunks it reaches, and E[C'][d]
// is its sum over C'), in chunk order; then seeds and inverse RoPE.
// E, F: [n_chunks][P][2][D] (dK, dV).
// ---------------------------------------------------------------------------
template <int HD, typename PlanT, typename RopeT>
__global__ __launch_bounds__(256) void bwd_carry_kernel(PlanT pl, const float* __restrict__ E,
                                                        const float* __restrict__ F, float* __restrict__ dK,
                                                        float* __restrict__ dV, const float* __restrict__ acc_dk,
                                                        const float* __restrict__ acc_dv, RopeT rope, int H) {
  const int C = blockIdx.x;
  const int K = pl.chunk_tiles;
  const int64_t rows_per_chunk = static_cast<int64_t>(K) * kTile;
  const int64_t sC = C * rows_per_chunk;
  const int t1 = (C + 1) * K;
  const int off = pl.pref_off[t1];
  const int A = pl.pref_off[t1 + 1] - off;
  const int P = prefix_cap(pl.max_depth);
  const int D = H * HD;
  const int Q = D / 2;  // 4-float jobs of a row: dK then dV
  for (int j = threadIdx.x; j < A * Q; j += blockDim.x) {
    const int d = j / Q;
    const int q = j - d * Q;
    const int64_t a = pl.prefix[off + d];
    if (a < sC) continue;  // first seen before chunk C: summed by its own chunk's job
    const int tv = q / (D / 4);
    const int col = (q - tv * (D / 4)) * 4;
    const int64_t ea = pl.end[a];
    float v[4];
    load_vec<4>(F + ((static_cast<int64_t>(C) * P + d) * 2 + tv) * D + col, v);
    // Chunks c2 > C with c2's first row inside the subtree; eight loads in
    // flight at a time, added in chunk order.
    const int c_end = static_cast<int>(min(static_cast<int64_t>(pl.n_chunks), (ea + rows_per_chunk - 1) / rows_per_chunk));
    const float* e0 = E + (static_cast<int64_t>(d) * 2 + tv) * D + col;
    const int64_t cstride = static_cast<int64_t>(P) * 2 * D;
    int c2 = C + 1;
    for (; c2 + 8 <= c_end; c2 += 8) {
      float y[8][4];
#pragma unroll
      for (int u = 0; u < 8; ++u) load_vec<4>(e0 + (c2 + u) * cstride, y[u]);
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int x = 0; x < 4; ++x) v[x] += y[u][x];
    }
    for (; c2 < c_end; ++c2) {
      float y[4];
      load_vec<4>(e0 + c2 * cstride, y);
#pragma unroll
      for (int x = 0; x < 4; ++x) v[x] += y[x];
    }
    const float* acc = tv ? acc_dv : acc_dk;
    if (acc) {
      float y[4];
      load_vec<4>(acc + a * D + col, y);
#pragma unroll
      for (int x = 0; x < 4; ++x) v[x] += y[x];
    }
    if (tv == 0 && rope.cos_t)
      agpt_fast::rope_inverse_part<4, HD>(v, rope.cos_t, rope.sin_t, rope_pos(d + 1, rope.seq_len), col % HD);
    store_vec<4>((tv ? dV : dK) + a * D + col, v);
  }
}

}  // namespace agpt_blk
