// varlen_attn.hip — drop-ins for the reference's packed varlen attention
// externs (agpt_train.cu:73-86, 3120-3132), fp32, gfx950.
//
// These keep the reference's packed layout, where every node / radix node
// carries its own copy of its ancestors' K/V rows, so callers such as
// batched_depth_forward.cr:767 and agpt_train.cu:4740/4988 can switch by
// renaming. The trie-native path (trie_attn.hip) avoids that duplication.
//
// Forward and node-level backward: a wave per query and group of heads,
// its lanes over head-slice dims, heads and packed rows (VLanes), so a
// query's contiguous packed rows are read in whole, coalesced rows; an
// online softmax per lane, merged across lanes, and the saved weights
// (weights_out, which the reference's backward reads) normalized in a second
// pass. Backward from saved weights, with the reference's Float64
// softmax-backward dot (batched_depth_backward.cr:637-651). The L-query
// backward accumulates
// each packed row over the radix node's queries in a fixed order inside one
// workgroup: no atomics.

#include "common.h"
#include "../../include/agpt_attn.h"

#include <cstdarg>
#include <cstdio>
#include <string>

using namespace agpt;

namespace {

constexpr int kMaxPackedLen = 4096;  // LDS bound of the L-query backward
typedef float f4 __attribute__((ext_vector_type(4)));

int vset_error(int code, const char* msg) { return agpt_internal_set_error(code, msg); }

__device__ __forceinline__ int visible_len(int qi, const int* q2n, const int* qoff,
                                           const int* kv_len, int max_len, int* node_out) {
  int node = q2n ? q2n[qi] : qi;
  int len = kv_len[node];
  if (q2n) {
    const int L = qoff[node + 1] - qoff[node];
    len = len - L + (qi - qoff[node]) + 1;
  }
  *node_out = node;
  return len < 0 ? 0 : (len > max_len ? max_len : len);
}

// Lane layout of the forward and node-level backward: a wave takes one
// query and a group of HW of its heads (HW a power of two). Lane
// L = dsub + NS (hl + HW pg): sub-lane dsub holds dims DS dsub .. of the head
// slice (NS = HD / 16 sub-lanes at head_dim 32 and 64, else one), hl is the
// head in the group and pg the lane's key group: it takes packed rows
// p = pg, pg + PG, .. (PG = 64 / (NS HW) groups). For one p the lanes of a
// wave read HW whole head slices of PG consecutive packed rows, and the rows
// of a query are contiguous in the packed layout, so the reads coalesce.
template <int HD>
struct VLanes {
  static constexpr int NS = HD > 16 ? HD / 16 : 1;
  static constexpr int DS = HD / NS;
  int hw, pgs, slots;  // heads per wave, key groups, waves per query
  __host__ __device__ VLanes(int H) {
    hw = 1;
    while (hw * 2 <= H && hw * 2 * NS <= 64) hw *= 2;
    pgs = 64 / (NS * hw);
    slots = (H + hw - 1) / hw;
  }
};

// Sum (or max) over the lanes that share (dsub, hl): a butterfly over the
// key-group bits of the lane index.
template <int NS>
__device__ __forceinline__ float pg_sum(float x, int hw, int pgs) {
  for (int m = NS * hw; m < NS * hw * pgs; m <<= 1) x += __shfl_xor(x, m);
  return x;
}
template <int NS>
__device__ __forceinline__ double pg_sum_d(double x, int hw, int pgs) {
  for (int m = NS * hw; m < NS * hw * pgs; m <<= 1) x += __shfl_xor(x, m);
  return x;
}
template <int NS>
__device__ __forceinline__ float pg_max(float x, int hw, int pgs) {
  for (int m = NS * hw; m < NS * hw * pgs; m <<= 1) x = fmaxf(x, __shfl_xor(x, m));
  return x;
}
// Sum over the NS sub-lanes of one head slice.
template <int NS>
__device__ __forceinline__ float sub_sum(float x) {
#pragma unroll
  for (int m = 1; m < NS; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

// Forward of one query (node, or L-query slot) and HW heads per wave: each
// lane keeps an online softmax over its key group (running max m, sum l and
// the weighted V sum), writing raw scores to the weights; the key groups
// merge by log-sum-exp, and a second pass over the lane's keys turns the
// raw scores into the normalized weights the backward reads.
template <int HD>
__global__ __launch_bounds__(256) void varlen_fwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const int* __restrict__ kv_off, const int* __restrict__ kv_len, const int* __restrict__ q2n,
    const int* __restrict__ qoff, float* __restrict__ out, float* __restrict__ weights, int n_q,
    int H, int max_len, float scale) {
  using LN = VLanes<HD>;
  constexpr int NS = LN::NS, DS = LN::DS;
  const LN ln(H);
  const int item = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= n_q * ln.slots) return;  // uniform per wave
  const int qi = item / ln.slots;
  const int lane = threadIdx.x & 63;
  const int dsub = lane % NS, hl = (lane / NS) % ln.hw, pg = lane / (NS * ln.hw);
  const int h = (item - qi * ln.slots) * ln.hw + hl;
  const bool act = h < H && pg < ln.pgs;
  const int hh = act ? h : 0;
  int node;
  const int len = visible_len(qi, q2n, qoff, kv_len, max_len, &node);
  const int64_t off = kv_off[node];
  float qq[DS], acc[DS];
  load_vec<DS>(q + (static_cast<int64_t>(qi) * H + hh) * HD + DS * dsub, qq);
#pragma unroll
  for (int i = 0; i < DS; ++i) acc[i] = 0.0f;
  float* w = weights + (static_cast<int64_t>(qi) * H + hh) * max_len;
  float m = -INFINITY, l = 0.0f;
  const int np = act ? (len - pg + ln.pgs - 1) / ln.pgs : 0;  // this lane's keys
  const int np_max = (len + ln.pgs - 1) / ln.pgs;               // the wave's trip count
  for (int i = 0; i < np_max; ++i) {
    const int p = pg + i * ln.pgs;
    const bool on = i < np;
    const int64_t row = (off + (on ? p : 0)) * H + hh;
    float kk[DS], vv[DS];
    load_vec<DS>(k + row * HD + DS * dsub, kk);
    load_vec<DS>(v + row * HD + DS * dsub, vv);
    float sc = 0.0f;
#pragma unroll
    for (int x = 0; x < DS; ++x) sc += qq[x] * kk[x];
    sc = sub_sum<NS>(sc) * scale;
    if (on && dsub == 0) w[p] = sc;
    const float s2 = on ? sc * kLog2e : -INFINITY;
    const float mn = fmaxf(m, s2);
    const float corr = mn == -INFINITY ? 1.0f : fast_exp2(m - mn);
    const float e = on ? fast_exp2(s2 - mn) : 0.0f;
    l = l * corr + e;
#pragma unroll
    for (int x = 0; x < DS; ++x) acc[x] = acc[x] * corr + e * vv[x];
    m = mn;
  }
  // merge the key groups
  const float mt = pg_max<NS>(m, ln.hw, ln.pgs);
  const float cf = m == -INFINITY ? 0.0f : fast_exp2(m - mt);
  const float lt = pg_sum<NS>(l * cf, ln.hw, ln.pgs);
#pragma unroll
  for (int x = 0; x < DS; ++x) acc[x] = pg_sum<NS>(acc[x] * cf, ln.hw, ln.pgs);
  const float inv = len > 0 ? 1.0f / lt : 0.0f;
  if (act && pg == 0) {
    float o[DS];
#pragma unroll
    for (int x = 0; x < DS; ++x) o[x] = acc[x] * inv;
    store_vec<DS>(out + (static_cast<int64_t>(qi) * H + h) * HD + DS * dsub, o);
  }
  if (act && dsub == 0)
    for (int i = 0; i < np; ++i) {
      const int p = pg + i * ln.pgs;
      w[p] = fast_exp2(w[p] * kLog2e - mt) * inv;
    }
}

// Node-level backward: every packed row belongs to exactly one node, so the
// lanes of (node, head) own its rows and write them. δ = Σ_p w_p (dO·v_p)
// in float64 as in the reference (batched_depth_backward.cr:637-651), then
// dS, dQ (summed over the key groups), and the rows' dK = dS q, dV = w dO.
template <int HD>
__global__ __launch_bounds__(256) void varlen_bwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ weights, const float* __restrict__ d_out,
    const int* __restrict__ kv_off, const int* __restrict__ kv_len, float* __restrict__ dq,
    float* __restrict__ dk, float* __restrict__ dv, int n_nodes, int H, int max_len, float scale) {
  using LN = VLanes<HD>;
  constexpr int NS = LN::NS, DS = LN::DS;
  const LN ln(H);
  const int item = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= n_nodes * ln.slots) return;  // uniform per wave
  const int i = item / ln.slots;
  const int lane = threadIdx.x & 63;
  const int dsub = lane % NS, hl = (lane / NS) % ln.hw, pg = lane / (NS * ln.hw);
  const int h = (item - i * ln.slots) * ln.hw + hl;
  const bool act = h < H && pg < ln.pgs;
  const int hh = act ? h : 0;
  int node;
  const int len = visible_len(i, nullptr, nullptr, kv_len, max_len, &node);
  const int64_t off = kv_off[node];
  float g[DS], qq[DS], dqa[DS];
  load_vec<DS>(d_out + (static_cast<int64_t>(i) * H + hh) * HD + DS * dsub, g);
  load_vec<DS>(q + (static_cast<int64_t>(i) * H + hh) * HD + DS * dsub, qq);
#pragma unroll
  for (int x = 0; x < DS; ++x) dqa[x] = 0.0f;
  const float* w = weights + (static_cast<int64_t>(i) * H + hh) * max_len;
  const int np = act ? (len - pg + ln.pgs - 1) / ln.pgs : 0;
  const int np_max = (len + ln.pgs - 1) / ln.pgs;  // uniform per wave
  // dO·v of the lane's first kCache keys stays in registers between the two
  // passes (the second then reads no V); later keys recompute it.
  constexpr int kCache = 8;
  float dwc[kCache];
  auto dw_of = [&](int p, bool on) {
    float vv[DS];
    load_vec<DS>(v + ((off + (on ? p : 0)) * H + hh) * HD + DS * dsub, vv);
    float dw = 0.0f;
#pragma unroll
    for (int x = 0; x < DS; ++x) dw += g[x] * vv[x];
    return sub_sum<NS>(dw);
  };
  double dot = 0.0;
#pragma unroll
  for (int t = 0; t < kCache; ++t) {
    if (t >= np_max) break;
    const int p = pg + t * ln.pgs;
    const bool on = t < np;
    dwc[t] = dw_of(p, on);
    if (on) dot += static_cast<double>(dwc[t] * w[p]);
  }
  for (int t = kCache; t < np_max; ++t) {
    const int p = pg + t * ln.pgs;
    const bool on = t < np;
    const float dw = dw_of(p, on);
    if (on) dot += static_cast<double>(dw * w[p]);
  }
  dot = pg_sum_d<NS>(dot, ln.hw, ln.pgs);
  auto emit = [&](int p, bool on, float dw) {
    const int64_t row = (off + (on ? p : 0)) * H + hh;
    float kk[DS];
    load_vec<DS>(k + row * HD + DS * dsub, kk);
    const float wp = on ? w[p] : 0.0f;
    const float ds = static_cast<float>(static_cast<double>(wp) * (static_cast<double>(dw) - dot) *
                                        static_cast<double>(scale));
    float rk[DS], rv[DS];
#pragma unroll
    for (int x = 0; x < DS; ++x) {
      dqa[x] += ds * kk[x];
      rk[x] = ds * qq[x];
      rv[x] = wp * g[x];
    }
    if (on) {
      store_vec<DS>(dk + row * HD + DS * dsub, rk);
      store_vec<DS>(dv + row * HD + DS * dsub, rv);
    }
  };
#pragma unroll
  for (int t = 0; t < kCache; ++t) {
    if (t >= np_max) break;
    emit(pg + t * ln.pgs, t < np, dwc[t]);
  }
  for (int t = kCache; t < np_max; ++t) {
    const int p = pg + t * ln.pgs;
    const bool on = t < np;
    emit(p, on, dw_of(p, on));
  }
#pragma unroll
  for (int x = 0; x < DS; ++x) dqa[x] = pg_sum<NS>(dqa[x], ln.hw, ln.pgs);
  if (act && pg == 0) store_vec<DS>(dq + (static_cast<int64_t>(i) * H + h) * HD + DS * dsub, dqa);
}

// L-query backward: one 64-lane workgroup per (radix node, head), launched
// per query slot and kept only at the node's first query. Lanes first take
// the node's queries (δ_j into LDS, dQ), then the node's packed rows (each
// row sums its queries in order j = 0..L-1 and adds into dk_full/dv_full).
template <int HD>
__global__ __launch_bounds__(64) void varlen_L_bwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ weights, const float* __restrict__ d_out,
    const int* __restrict__ q2n, const int* __restrict__ qoff, const int* __restrict__ kv_off,
    const int* __restrict__ kv_len, float* __restrict__ dq, float* __restrict__ dk,
    float* __restrict__ dv, int H, int max_len, float scale) {
  extern __shared__ double delta[];
  const int t0 = blockIdx.x;
  const int h = blockIdx.y;
  const int node = q2n[t0];
  if (qoff[node] != t0) return;  // uniform across the workgroup
  const int L = qoff[node + 1] - t0;
  if (L < 1 || L > max_len) return;  // inconsistent tables: LDS holds max_len entries
  const int64_t off = kv_off[node];
  int len = kv_len[node];
  if (len > max_len) len = max_len;
  const float* wbase = weights;
  for (int j = threadIdx.x; j < L; j += blockDim.x) {
    const int t = t0 + j;
    int vis = len - L + j + 1;
    if (vis < 0) vis = 0;
    float g[HD], dqa[HD];
    load_vec<HD>(d_out + (static_cast<int64_t>(t) * H + h) * HD, g);
#pragma unroll
    for (int x = 0; x < HD; ++x) dqa[x] = 0.0f;
    const float* w = wbase + (static_cast<int64_t>(t) * H + h) * max_len;
    double dot = 0.0;
    for (int p = 0; p < vis; ++p) {
      float vv[HD];
      load_vec<HD>(v + ((off + p) * H + h) * HD, vv);
      float dw = 0.0f;
#pragma unroll
      for (int x = 0; x < HD; ++x) dw += g[x] * vv[x];
      dot += static_cast<double>(dw * w[p]);
    }
    for (int p = 0; p < vis; ++p) {
      float vv[HD], kk[HD];
      load_vec<HD>(v + ((off + p) * H + h) * HD, vv);
      load_vec<HD>(k + ((off + p) * H + h) * HD, kk);
      float dw = 0.0f;
#pragma unroll
      for (int x = 0; x < HD; ++x) dw += g[x] * vv[x];
      const float ds = static_cast<float>(static_cast<double>(w[p]) * (static_cast<double>(dw) - dot) *
                                          static_cast<double>(scale));
#pragma unroll
      for (int x = 0; x < HD; ++x) dqa[x] += ds * kk[x];
    }
    delta[j] = dot;
    store_vec<HD>(dq + (static_cast<int64_t>(t) * H + h) * HD, dqa);
  }
  __syncthreads();
  const int first_row_all = len - L;  // rows < this are seen by every query
  for (int p = threadIdx.x; p < len; p += blockDim.x) {
    float vv[HD], dka[HD], dva[HD];
    load_vec<HD>(v + ((off + p) * H + h) * HD, vv);
#pragma unroll
    for (int x = 0; x < HD; ++x) {
      dka[x] = 0.0f;
      dva[x] = 0.0f;
    }
    const int j0 = p - first_row_all > 0 ? p - first_row_all : 0;
    for (int j = j0; j < L; ++j) {
      const int t = t0 + j;
      float g[HD], qq[HD];
      load_vec<HD>(d_out + (static_cast<int64_t>(t) * H + h) * HD, g);
      load_vec<HD>(q + (static_cast<int64_t>(t) * H + h) * HD, qq);
      float dw = 0.0f;
#pragma unroll
      for (int x = 0; x < HD; ++x) dw += g[x] * vv[x];
      const float wp = wbase[(static_cast<int64_t>(t) * H + h) * max_len + p];
      const float ds = static_cast<float>(static_cast<double>(wp) * (static_cast<double>(dw) - delta[j]) *
                                          static_cast<double>(scale));
#pragma unroll
      for (int x = 0; x < HD; ++x) {
        dka[x] += ds * qq[x];
        dva[x] += wp * g[x];
      }
    }
    float* rk = dk + ((off + p) * H + h) * HD;
    float* rv = dv + ((off + p) * H + h) * HD;
    float ok[HD], ov[HD];
    load_vec<HD>(rk, ok);
    load_vec<HD>(rv, ov);
#pragma unroll
    for (int x = 0; x < HD; ++x) {
      ok[x] += dka[x];
      ov[x] += dva[x];
    }
    store_vec<HD>(rk, ok);
    store_vec<HD>(rv, ov);
  }
}

// L-query kernels over radix nodes, on 16x16 fp32 matrix instructions. A
// wave owns the radix nodes whose first query lies in its block of 64
// queries (one ballot finds them; a node's queries may run past the block),
// so no launch slot is spent on a query that is not a node's first, and
// takes each node one head at a time in 16x16 blocks of (query, packed row).
// Query j of a node with L queries and len packed rows sees rows
// p <= len - L + j (agpt_train.cu:3106-3117).
//
// v_mfma_f32_16x16x4f32: D[16][16] += A[16][4] B[4][16]; lane l = 16g + c
// supplies A[c][g], B[g][c] and holds D[4g + r][c] in register r. For a
// contraction over head dims, step j pairs lane group g with dim KD g + j
// (KD = HD / 4: each lane reads one contiguous slice of a row); over the 16
// rows or queries of a block, step j pairs group g with index 4g + j, which
// is the D layout, so a product's registers feed the next one directly.
constexpr int kLqMaxDelta = 1024;  // queries per node in the backward's per-wave δ table (LDS)

// Bit mask of the lanes whose query t = base + lane is its radix node's first.
__device__ __forceinline__ uint64_t node_starts(const int* __restrict__ q2n, const int* __restrict__ qoff,
                                                int64_t base, int T_q) {
  const int64_t t = base + (threadIdx.x & 63);
  bool first = false;
  if (t < T_q) first = qoff[q2n[t]] == t;
  return __ballot(first);
}

__device__ __forceinline__ f4 lq_mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// Max / sum over the four lane groups (lanes c, c+16, c+32, c+48).
__device__ __forceinline__ float lq_gmax(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float lq_gsum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}
__device__ __forceinline__ double lq_gsum_d(double x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// S^T = X_b Y_i^T of one 16x16 block: X rows (packed rows) are the A side,
// Y rows (queries) the B side; this lane supplies KD dims (from KD g) of its
// X row at xrow and holds its Y row's slice y. s[r]: packed row 4g + r
// against query c.
template <int HD>
__device__ __forceinline__ f4 lq_rows_dot(const float* __restrict__ xrow, const float (&y)[HD / 4], int g) {
  constexpr int KD = HD / 4;
  float x[KD];
  load_vec<KD>(xrow + KD * g, x);
  f4 acc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < KD; ++j) acc = lq_mfma(x[j], y[j], acc);
  return acc;
}
// Weights of rows p0 .. p0+3 of one query's row (entries from vis on read
// as 0): one 16-byte load when the rows are 16-byte aligned (max_len a
// multiple of 4, p0 a multiple of 4), else one load per visible entry.
__device__ __forceinline__ void lq_weights4(const float* __restrict__ wrow, int p0, bool vec, int vis,
                                            float (&w)[4]) {
  if (vec && p0 + 4 <= vis) {
    const f4 x = *reinterpret_cast<const f4*>(wrow + p0);
#pragma unroll
    for (int r = 0; r < 4; ++r) w[r] = x[r];
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) w[r] = p0 + r < vis ? wrow[p0 + r] : 0.0f;
  }
}

// Score blocks a first pass keeps in registers for the second (rows beyond
// 16 * kLqCache are recomputed).
constexpr int kLqCache = 4;

// Forward. A wave takes one head of the nodes that start in its query
// block. Per (node, query block i): a first pass over the visible packed-row
// blocks takes each query's maximum and sum (S^T blocks: query c in lane
// column c, rows in registers), a second recomputes S^T, writes the
// normalized weights (visible entries only) and adds O^T += V^T P^T.
template <int HD>
__global__ __launch_bounds__(256) void varlen_Lq_fwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const int* __restrict__ q2n, const int* __restrict__ qoff, const int* __restrict__ kv_off,
    const int* __restrict__ kv_len, float* __restrict__ out, float* __restrict__ weights, int T_q, int H,
    int max_len, float scale) {
  constexpr int MT = HD / 16;
  // wave = (block of 64 queries, head)
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t base = wid / H * 64;
  const int h = static_cast<int>(wid - wid / H * H);
  if (base >= T_q) return;  // uniform per wave
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  uint64_t starts = node_starts(q2n, qoff, base, T_q);
  const float qs = scale * kLog2e;
  const int RS = H * HD;         // row stride of q / k / v / out
  const int WS = H * max_len;    // query stride of the weights
  const bool wvec = (max_len & 3) == 0;  // weight rows 16-byte aligned
  while (starts) {
    const int64_t t0 = base + __builtin_ctzll(starts);
    starts &= starts - 1;
    const int node = q2n[t0];
    const int L = qoff[node + 1] - static_cast<int>(t0);
    const int len = min(kv_len[node], max_len);
    if (L < 1 || L > max_len || len < 1) continue;  // inconsistent tables
    const int64_t off = kv_off[node];
    const float* qh = q + (t0 * H + h) * HD;  // query j of the node at qh + j RS
    float* oh = out + (t0 * H + h) * HD;
    float* wh = weights + (t0 * H + h) * max_len;
    const float* kh = k + (off * H + h) * HD;  // packed row p at kh + p RS
    const float* vh = v + (off * H + h) * HD;
    const int shift = len - L;  // query j sees rows p <= shift + j
    for (int i = 0; i < L; i += 16) {
      const int jq = i + c;  // this lane's query (column)
      const bool qok = jq < L;
      float qy[HD / 4];
      load_vec<HD / 4>(qh + (qok ? jq : 0) * RS + (HD / 4) * g, qy);
      const int pend = min(len, shift + i + 16);  // rows any query of the block sees
      float m = -INFINITY, l = 0.0f;
      f4 sc[kLqCache];
#pragma unroll
      for (int x = 0; x < kLqCache; ++x) sc[x] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int b = 0; b < pend; b += 16) {
        const f4 sv0 = lq_rows_dot<HD>(kh + min(b + c, len - 1) * RS, qy, g);
#pragma unroll
        for (int x = 0; x < kLqCache; ++x)
          if (b == 16 * x) sc[x] = sv0;
        float sv[4], bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = b + 4 * g + r;
          sv[r] = (qok && p < len && p <= shift + jq) ? sv0[r] * qs : -INFINITY;
          bm = fmaxf(bm, sv[r]);
        }
        const float mn = fmaxf(m, lq_gmax(bm));
        float e = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) e += sv[r] == -INFINITY ? 0.0f : fast_exp2(sv[r] - mn);
        l = (m == -INFINITY ? 0.0f : l * fast_exp2(m - mn)) + lq_gsum(e);
        m = mn;
      }
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
      f4 o[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) o[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      float* wrow = wh + static_cast<int64_t>(qok ? jq : 0) * WS;
      for (int b = 0; b < pend; b += 16) {
        // V^T operand first: lane (g, c) supplies V[row b + 4g + j][dim 16t + c]
        float vt[MT][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int t = 0; t < MT; ++t) vt[t][j] = vh[min(b + 4 * g + j, len - 1) * RS + 16 * t + c];
        f4 sv = sc[0];
#pragma unroll
        for (int x = 1; x < kLqCache; ++x)
          if (b == 16 * x) sv = sc[x];
        if (b >= 16 * kLqCache) sv = lq_rows_dot<HD>(kh + min(b + c, len - 1) * RS, qy, g);
        float pw[4];
        const int vis = qok ? min(len, shift + jq + 1) : 0;  // this query's visible rows
#pragma unroll
        for (int r = 0; r < 4; ++r) pw[r] = b + 4 * g + r < vis ? fast_exp2(sv[r] * qs - m) * inv : 0.0f;
        if (wvec && b + 4 * g + 4 <= vis) {
          *reinterpret_cast<f4*>(wrow + b + 4 * g) = f4{pw[0], pw[1], pw[2], pw[3]};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (b + 4 * g + r < vis) wrow[b + 4 * g + r] = pw[r];
        }
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j) o[t] = lq_mfma(vt[t][j], pw[j], o[t]);
      }
      // O^T[dim 16t + 4g + r][query c]
      if (qok)
#pragma unroll
        for (int t = 0; t < MT; ++t) *reinterpret_cast<f4*>(oh + jq * RS + 16 * t + 4 * g) = o[t];
    }
  }
}

// Backward from the saved weights; a wave takes one head of the nodes that
// start in its query block. Query side, per query block: dW^T = V dO^T
// blocks and the weights give δ_j = Σ_p w_jp dW_jp, accumulated in float64
// (batched_depth_backward.cr:637-651) and kept in the wave's LDS table; a
// second pass forms dS^T = w (dW - δ) scale (float64, rounded once) and
// dQ^T += K^T dS^T. Key side, per packed-row block: dW blocks in the other
// orientation (row c in lane column c), dS with the table's δ, dV^T +=
// dO^T P and dK^T += Q^T dS over the node's query blocks in order, added
// into dk_full / dv_full — each row of a node has one owner lane, so there
// are no atomics.
template <int HD>
__global__ __launch_bounds__(256) void varlen_Lq_bwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ weights, const float* __restrict__ d_out, const int* __restrict__ q2n,
    const int* __restrict__ qoff, const int* __restrict__ kv_off, const int* __restrict__ kv_len,
    float* __restrict__ dq, float* __restrict__ dk, float* __restrict__ dv, int T_q, int H, int max_len,
    float scale) {
  constexpr int MT = HD / 16;
  extern __shared__ double lq_delta[];
  double* delta = lq_delta + (threadIdx.x >> 6) * max_len;
  // wave = (block of 64 queries, head)
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t base = wid / H * 64;
  const int h = static_cast<int>(wid - wid / H * H);
  if (base >= T_q) return;  // uniform per wave
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  uint64_t starts = node_starts(q2n, qoff, base, T_q);
  const double dscale = static_cast<double>(scale);
  const int RS = H * HD;       // row stride of q / k / v / d_out / dq / dk / dv
  const int WS = H * max_len;  // query stride of the weights
  const bool wvec = (max_len & 3) == 0;  // weight rows 16-byte aligned
  while (starts) {
    const int64_t t0 = base + __builtin_ctzll(starts);
    starts &= starts - 1;
    const int node = q2n[t0];
    const int L = qoff[node + 1] - static_cast<int>(t0);
    const int len = min(kv_len[node], max_len);
    if (L < 1 || L > max_len || len < 1) continue;  // inconsistent tables: δ holds max_len queries
    const int64_t off = kv_off[node];
    const float* qh = q + (t0 * H + h) * HD;  // query j of the node at + j RS
    const float* gh = d_out + (t0 * H + h) * HD;
    float* dqh = dq + (t0 * H + h) * HD;
    const float* wh = weights + (t0 * H + h) * max_len;
    const float* kh = k + (off * H + h) * HD;  // packed row p at + p RS
    const float* vh = v + (off * H + h) * HD;
    float* dkh = dk + (off * H + h) * HD;
    float* dvh = dv + (off * H + h) * HD;
    const int shift = len - L;
    // ---- query side: δ and dQ
    for (int i = 0; i < L; i += 16) {
      const int jq = i + c;
      const bool qok = jq < L;
      float gy[HD / 4];
      load_vec<HD / 4>(gh + (qok ? jq : 0) * RS + (HD / 4) * g, gy);
      const float* wrow = wh + static_cast<int64_t>(qok ? jq : 0) * WS;
      const int pend = min(len, shift + i + 16);
      double dot = 0.0;
      for (int b = 0; b < pend; b += 16) {
        const f4 dw = lq_rows_dot<HD>(vh + min(b + c, len - 1) * RS, gy, g);
        float wp[4];
        lq_weights4(wrow, b + 4 * g, wvec, qok ? min(len, shift + jq + 1) : 0, wp);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (qok && b + 4 * g + r < len && b + 4 * g + r <= shift + jq) dot += static_cast<double>(dw[r] * wp[r]);
      }
      dot = lq_gsum_d(dot);
      if (qok && g == 0) delta[jq] = dot;
      f4 dqa[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) dqa[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int b = 0; b < pend; b += 16) {
        // K^T operand: lane (g, c) supplies K[row b + 4g + j][dim 16t + c]
        float kt[MT][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int t = 0; t < MT; ++t) kt[t][j] = kh[min(b + 4 * g + j, len - 1) * RS + 16 * t + c];
        const f4 dw = lq_rows_dot<HD>(vh + min(b + c, len - 1) * RS, gy, g);
        float wp[4], ds[4];
        lq_weights4(wrow, b + 4 * g, wvec, qok ? min(len, shift + jq + 1) : 0, wp);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ds[r] = static_cast<float>(static_cast<double>(wp[r]) * (static_cast<double>(dw[r]) - dot) * dscale);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j) dqa[t] = lq_mfma(kt[t][j], ds[j], dqa[t]);
      }
      if (qok)
#pragma unroll
        for (int t = 0; t < MT; ++t) *reinterpret_cast<f4*>(dqh + jq * RS + 16 * t + 4 * g) = dqa[t];
    }
    // the δ table is read across lanes below
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- key side: dK, dV of the node's packed rows
    for (int b = 0; b < len; b += 16) {
      const int p = b + c;  // this lane's packed row (column)
      const bool pok = p < len;
      float vy[HD / 4];
      load_vec<HD / 4>(vh + (pok ? p : 0) * RS + (HD / 4) * g, vy);
      f4 dka[MT], dva[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        dka[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        dva[t] = dka[t];
      }
      // the block's rows are seen from query max(0, b - shift) on
      for (int i = max(0, b - shift) / 16 * 16; i < L; i += 16) {
        // dO^T, Q^T operands: lane (g, c) supplies row i + 4g + j at dim 16t + c
        float gt[MT][4], qt[MT][4], wv[4];
        double dl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int jj = i + 4 * g + j;
          const int jc = min(jj, L - 1);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            gt[t][j] = gh[jc * RS + 16 * t + c];
            qt[t][j] = qh[jc * RS + 16 * t + c];
          }
          const bool live = pok && jj < L && p <= shift + jj;
          wv[j] = live ? wh[static_cast<int64_t>(jc) * WS + p] : 0.0f;
          dl[j] = live ? delta[jc] : 0.0;
        }
        const f4 dw = lq_rows_dot<HD>(gh + min(i + c, L - 1) * RS, vy, g);
        float ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ds[r] = static_cast<float>(static_cast<double>(wv[r]) * (static_cast<double>(dw[r]) - dl[r]) * dscale);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            dva[t] = lq_mfma(gt[t][j], wv[j], dva[t]);
            dka[t] = lq_mfma(qt[t][j], ds[j], dka[t]);
          }
      }
      // dK^T[dim 16t + 4g + r][row c]: add into the caller's rows
      if (pok)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          f4* pk = reinterpret_cast<f4*>(dkh + p * RS + 16 * t + 4 * g);
          f4* pv = reinterpret_cast<f4*>(dvh + p * RS + 16 * t + 4 * g);
          *pk = *pk + dka[t];
          *pv = *pv + dva[t];
        }
    }
    // the next node's query side rewrites the δ table
    __builtin_amdgcn_wave_barrier();
  }
}

template <typename Fn>
int dispatch(int hd, Fn&& fn) {
  switch (hd) {
    case 4: fn(std::integral_constant<int, 4>{}); return AGPT_OK;
    case 8: fn(std::integral_constant<int, 8>{}); return AGPT_OK;
    case 16: fn(std::integral_constant<int, 16>{}); return AGPT_OK;
    case 32: fn(std::integral_constant<int, 32>{}); return AGPT_OK;
    case 64: fn(std::integral_constant<int, 64>{}); return AGPT_OK;
    default: return vset_error(AGPT_ERR_UNSUPPORTED, "varlen: head_dim not built (4, 8, 16, 32, 64)");
  }
}

bool bad_dims(int n, int H, int max_len) { return n < 0 || H < 1 || max_len < 1; }

int finish_launch() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return vset_error(AGPT_ERR_DEVICE, hipGetErrorString(e));
  return AGPT_OK;
}

}  // namespace

extern "C" int agpt_varlen_attention(const float* q, const float* k, const float* v,
                                     const int* kv_offsets, const int* kv_lengths, float* output,
                                     float* weights_out, int n_nodes, int n_heads, int head_dim,
                                     int max_len, float scale, void* stream) {
  if (bad_dims(n_nodes, n_heads, max_len)) return vset_error(AGPT_ERR_INVALID_ARG, "varlen: bad sizes");
  if (n_nodes == 0) return AGPT_OK;
  if (!q || !k || !v || !kv_offsets || !kv_lengths || !output || !weights_out)
    return vset_error(AGPT_ERR_INVALID_ARG, "varlen: null pointer");
  const int rc = dispatch(head_dim, [&](auto c) {
    constexpr int HD = decltype(c)::value;
    const int64_t items = static_cast<int64_t>(n_nodes) * VLanes<HD>(n_heads).slots;  // one wave each
    hipLaunchKernelGGL((varlen_fwd_kernel<HD>), dim3(static_cast<unsigned>((items + 3) / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), q, k, v, kv_offsets, kv_lengths, nullptr,
                       nullptr, output, weights_out, n_nodes, n_heads, max_len, scale);
  });
  return rc != AGPT_OK ? rc : finish_launch();
}

extern "C" int agpt_varlen_attention_backward(const float* q, const float* k, const float* v,
                                              const float* attn_weights, const float* d_out,
                                              const int* kv_offsets, const int* kv_lengths,
                                              float* dq, float* dk_full, float* dv_full,
                                              int n_nodes, int n_heads, int head_dim, int max_len,
                                              float scale, void* stream) {
  if (bad_dims(n_nodes, n_heads, max_len)) return vset_error(AGPT_ERR_INVALID_ARG, "varlen: bad sizes");
  if (n_nodes == 0) return AGPT_OK;
  if (!q || !k || !v || !attn_weights || !d_out || !kv_offsets || !kv_lengths || !dq || !dk_full || !dv_full)
    return vset_error(AGPT_ERR_INVALID_ARG, "varlen: null pointer");
  const int rc = dispatch(head_dim, [&](auto c) {
    constexpr int HD = decltype(c)::value;
    const int64_t items = static_cast<int64_t>(n_nodes) * VLanes<HD>(n_heads).slots;  // one wave each
    hipLaunchKernelGGL((varlen_bwd_kernel<HD>), dim3(static_cast<unsigned>((items + 3) / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), q, k, v, attn_weights, d_out, kv_offsets,
                       kv_lengths, dq, dk_full, dv_full, n_nodes, n_heads, max_len, scale);
  });
  return rc != AGPT_OK ? rc : finish_launch();
}

extern "C" int agpt_unpack_batched_attn_output(const float* packed, float* unpacked, int n_nodes,
                                               int n_heads, int head_dim, void* stream) {
  if (n_nodes < 0 || n_heads < 1 || head_dim < 1) return vset_error(AGPT_ERR_INVALID_ARG, "unpack: bad sizes");
  if (n_nodes == 0) return AGPT_OK;
  if (!packed || !unpacked) return vset_error(AGPT_ERR_INVALID_ARG, "unpack: null pointer");
  const size_t bytes = static_cast<size_t>(n_nodes) * n_heads * head_dim * sizeof(float);
  if (packed != unpacked) {
    const hipError_t e = hipMemcpyAsync(unpacked, packed, bytes, hipMemcpyDeviceToDevice,
                                        static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return vset_error(AGPT_ERR_DEVICE, hipGetErrorString(e));
  }
  return AGPT_OK;
}

extern "C" int agpt_varlen_attention_L_queries(const float* q, const float* k, const float* v,
                                               const int* query_to_node, const int* query_offsets,
                                               const int* kv_offsets, const int* kv_lengths,
                                               float* output, float* weights_out, int T_q,
                                               int n_heads, int head_dim, int max_kv_len,
                                               float scale, void* stream) {
  if (bad_dims(T_q, n_heads, max_kv_len)) return vset_error(AGPT_ERR_INVALID_ARG, "varlen_L: bad sizes");
  if (T_q == 0) return AGPT_OK;
  if (!q || !k || !v || !query_to_node || !query_offsets || !kv_offsets || !kv_lengths || !output ||
      !weights_out)
    return vset_error(AGPT_ERR_INVALID_ARG, "varlen_L: null pointer");
  const int rc = dispatch(head_dim, [&](auto c) {
    constexpr int HD = decltype(c)::value;
    if constexpr (HD % 16 == 0) {
      const int64_t waves = (static_cast<int64_t>(T_q) + 63) / 64 * n_heads;  // (block of 64 queries, head)
      hipLaunchKernelGGL((varlen_Lq_fwd_kernel<HD>), dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0,
                         static_cast<hipStream_t>(stream), q, k, v, query_to_node, query_offsets, kv_offsets,
                         kv_lengths, output, weights_out, T_q, n_heads, max_kv_len, scale);
    } else {  // head dims 4 and 8: a wave per (query, head group)
      const int64_t items = static_cast<int64_t>(T_q) * VLanes<HD>(n_heads).slots;
      hipLaunchKernelGGL((varlen_fwd_kernel<HD>), dim3(static_cast<unsigned>((items + 3) / 4)), dim3(256), 0,
                         static_cast<hipStream_t>(stream), q, k, v, kv_offsets, kv_lengths, query_to_node,
                         query_offsets, output, weights_out, T_q, n_heads, max_kv_len, scale);
    }
  });
  return rc != AGPT_OK ? rc : finish_launch();
}

extern "C" int agpt_varlen_attention_L_queries_backward(
    const float* q, const float* k, const float* v, const float* attn_weights, const float* d_out,
    const int* query_to_node, const int* query_offsets, const int* kv_offsets,
    const int* kv_lengths, float* dq, float* dk_full, float* dv_full, int T_q, int n_heads,
    int head_dim, int max_kv_len, float scale, void* stream) {
  if (bad_dims(T_q, n_heads, max_kv_len)) return vset_error(AGPT_ERR_INVALID_ARG, "varlen_L: bad sizes");
  if (max_kv_len > kMaxPackedLen)
    return vset_error(AGPT_ERR_UNSUPPORTED, "varlen_L backward: max_kv_len above 4096");
  if (T_q == 0) return AGPT_OK;
  if (!q || !k || !v || !attn_weights || !d_out || !query_to_node || !query_offsets || !kv_offsets ||
      !kv_lengths || !dq || !dk_full || !dv_full)
    return vset_error(AGPT_ERR_INVALID_ARG, "varlen_L: null pointer");
  const int rc = dispatch(head_dim, [&](auto c) {
    constexpr int HD = decltype(c)::value;
    if (HD % 16 == 0 && max_kv_len <= kLqMaxDelta) {
      const int64_t waves = (static_cast<int64_t>(T_q) + 63) / 64 * n_heads;  // (block of 64 queries, head)
      hipLaunchKernelGGL((varlen_Lq_bwd_kernel<HD % 16 == 0 ? HD : 16>), dim3(static_cast<unsigned>((waves + 3) / 4)),
                         dim3(256), sizeof(double) * 4 * max_kv_len, static_cast<hipStream_t>(stream), q, k, v,
                         attn_weights, d_out, query_to_node, query_offsets, kv_offsets, kv_lengths, dq, dk_full,
                         dv_full, T_q, n_heads, max_kv_len, scale);
    } else {  // head dims 4 and 8, or a δ table past the wave's LDS share: a workgroup per (radix node, head)
      hipLaunchKernelGGL((varlen_L_bwd_kernel<HD>), dim3(T_q, n_heads), dim3(64),
                         sizeof(double) * max_kv_len, static_cast<hipStream_t>(stream), q, k, v,
                         attn_weights, d_out, query_to_node, query_offsets, kv_offsets, kv_lengths, dq,
                         dk_full, dv_full, n_heads, max_kv_len, scale);
    }
  });
  return rc != AGPT_OK ? rc : finish_launch();
}
