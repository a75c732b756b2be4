// agpt_loss.hip — the per-query AGPT loss over radix queries (gfx950), the
// drop-in for launch_agpt_loss_per_query (agpt_train.cu:2199-2216, kernel
// :2069-2194), plus the host-side corpus-mass weights (agpt_train.cu:4608-4637).
//
// Each query row q of logits [T_q, V] gets p = softmax(row) and:
//   intermediate (q+1 < end of its radix node's queries, or an endpoint under
//   ce_only with a next query): target = token_ids[q+1],
//     loss = -log(p_t + 1e-10), grad = p - onehot(t), both times
//     intermediate_weight (x mass_weights[q]);
//   endpoint: the node's next-token counts c (CSR by radix id), total N,
//     loss = -sum_e (c_e/N) log(p_tok_e + 1e-10), grad = p - c/N, both times
//     (1 + lambda H/log V) (x mass_weights[q]); an endpoint without counts
//     gets loss 0 and grad = p.
//
// Layout: LPR lanes own one row (4 for V <= 32, 8 for V <= 128, 16 for
// V <= 512, else 64) of the rows staged in LDS. The row is read once and
// written once: the loss is HBM-bound at 8V bytes per query. The count entries of an endpoint are applied one at a time in
// their stored order (as the reference's single thread does), so repeated
// tokens and the loss sum come out in the same order.

#include "common.h"
#include "../../include/agpt_loss.h"

#include <cfloat>
#include <cmath>
#include <algorithm>
#include <cstdio>

namespace {

using agpt::fast_exp2;
using agpt::kLog2e;

constexpr int kThreads = 256;

// Row reductions by DPP lane moves (no LDS round trip). Sums pair lane i
// with its mirror (16-lane row, 8-lane half, quad, pair; a 4-lane row starts
// at the quad): each step adds two values that are equal-by-symmetry sums,
// so every lane of the row ends with the same bits. Across the four rows of a wave (LPR = 64) the row totals
// are combined by lane-half swaps, again commutative pairs.
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
template <int kCtrl>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xf, 0xf, false);
}
constexpr int kRowMirror = 0x140, kRowHalfMirror = 0x141, kQuadRev = 0x1B, kQuadSwap = 0xB1;

template <int LPR, typename T>
__device__ __forceinline__ T row_sum(T v) {
  if constexpr (LPR >= 16) v += dpp<kRowMirror>(v);
  if constexpr (LPR >= 8) v += dpp<kRowHalfMirror>(v);
  v += dpp<kQuadRev>(v);
  return v + dpp<kQuadSwap>(v);
}
template <int LPR>
__device__ __forceinline__ float row_max(float v) {
  if constexpr (LPR >= 16) v = fmaxf(v, dpp<kRowMirror>(v));
  if constexpr (LPR >= 8) v = fmaxf(v, dpp<kRowHalfMirror>(v));
  v = fmaxf(v, dpp<kQuadRev>(v));
  return fmaxf(v, dpp<kQuadSwap>(v));
}
// Lane-half swaps: each result pair holds the lane's own value and its
// partner's (lane ^ 16, then lane ^ 32), in an order that depends on the lane.
__device__ __forceinline__ float cross_rows_max(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned w = __float_as_uint(v);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float cross_rows_sum(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const unsigned w = __float_as_uint(v);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ int cross_rows_sum(int v) {
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = static_cast<int>(a[0]) + static_cast<int>(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return static_cast<int>(b[0]) + static_cast<int>(b[1]);
}
template <int LPR>
__device__ __forceinline__ float group_max(float v) {
  v = row_max<LPR>(v);
  if constexpr (LPR == 64) v = cross_rows_max(v);
  return v;
}
template <int LPR, typename T>
__device__ __forceinline__ T group_sum(T v) {
  v = row_sum<LPR>(v);
  if constexpr (LPR == 64) v = cross_rows_sum(v);
  return v;
}

// Columns of a row over its LPR lanes: rows of 4 or 8 lanes give each lane
// VPL consecutive columns; wider rows interleave them (lane c: c, c + LPR,
// ...), which keeps the LDS reads of rows whose length is a multiple of 64
// off a shared bank.
template <int LPR, int VPL>
struct Cols {
  static constexpr bool kSlice = LPR <= 8;
  static __device__ __forceinline__ int col(int c, int i) { return kSlice ? c * VPL + i : c + LPR * i; }
  static __device__ __forceinline__ int owner(int j) { return kSlice ? j / VPL : j % LPR; }
  static __device__ __forceinline__ int slot(int j) { return kSlice ? j % VPL : j / LPR; }
};

// Value of column j of the row held by this lane's group (j uniform over the
// group).
template <int LPR, int VPL>
__device__ __forceinline__ float row_value(const float (&x)[VPL], int base, int j) {
  const int slot = Cols<LPR, VPL>::slot(j);
  float v = x[0];
#pragma unroll
  for (int i = 1; i < VPL; ++i) v = slot == i ? x[i] : v;
  return __shfl(v, base + Cols<LPR, VPL>::owner(j), 64);
}
template <int VPL>
__device__ __forceinline__ void sub_at(float (&x)[VPL], int slot, bool own, float d) {
#pragma unroll
  for (int i = 0; i < VPL; ++i)
    if (own && slot == i) x[i] -= d;
}

// A workgroup takes a run of RB consecutive rows (RB * V <= kChunk floats):
// the run is one contiguous byte range, read and written with aligned
// 16-byte vector accesses through LDS, whatever V. The next run's bytes and
// first-level tables are requested before the current run is worked on, so
// they arrive during its arithmetic and stores.
constexpr int kChunk = 8192;  // floats staged per workgroup (32 KiB: four workgroups per CU)
constexpr int kMaxRows = 256;

struct RowTabs {
  int end[kMaxRows], tgt[kMaxRows], cs[kMaxRows], ce[kMaxRows];
  float mw[kMaxRows];
};

// Global floats [f0, f1) (f1 - f0 <= kChunk) in 16-byte pieces on
// 16-byte-aligned addresses: piece k of thread t starts at a0 + 4 (t + k
// kThreads); the two partial pieces at the ends are read element by element.
constexpr int kMoveIters = kChunk / (4 * kThreads) + 1;  // +1: the run need not start aligned

__device__ __forceinline__ int64_t piece0(const float* g, int64_t f0) {
  const int mis = static_cast<int>((reinterpret_cast<uintptr_t>(g) >> 2) & 3);
  return f0 - ((f0 + mis) & 3);
}

__device__ __forceinline__ void load_run(const float* __restrict__ g, float4 (&v)[kMoveIters], int64_t f0,
                                         int64_t f1) {
  const int64_t a0 = piece0(g, f0);
#pragma unroll
  for (int k = 0; k < kMoveIters; ++k) {
    const int64_t i = a0 + 4 * (threadIdx.x + k * kThreads);
    if (i >= f0 && i + 4 <= f1) {
      v[k] = *reinterpret_cast<const float4*>(g + i);
    } else {
      v[k].x = i >= f0 && i < f1 ? g[i] : 0.0f;
      v[k].y = i + 1 >= f0 && i + 1 < f1 ? g[i + 1] : 0.0f;
      v[k].z = i + 2 >= f0 && i + 2 < f1 ? g[i + 2] : 0.0f;
      v[k].w = i + 3 >= f0 && i + 3 < f1 ? g[i + 3] : 0.0f;
    }
  }
}

__device__ __forceinline__ void run_to_lds(const float* g, const float4 (&v)[kMoveIters], float* __restrict__ l,
                                           int64_t f0, int64_t f1) {
  const int64_t a0 = piece0(g, f0);
#pragma unroll
  for (int k = 0; k < kMoveIters; ++k) {
    const int64_t i = a0 + 4 * (threadIdx.x + k * kThreads);
    const float e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (i + t >= f0 && i + t < f1) l[i + t - f0] = e[t];
  }
}

__device__ __forceinline__ void store_run(float* __restrict__ g, const float* __restrict__ l, int64_t f0,
                                          int64_t f1) {
  const int64_t a0 = piece0(g, f0);
#pragma unroll
  for (int k = 0; k < kMoveIters; ++k) {
    const int64_t i = a0 + 4 * (threadIdx.x + k * kThreads);
    if (i >= f1) continue;
    const float* d = l + (i - f0);
    if (i >= f0 && i + 4 <= f1) {
      *reinterpret_cast<float4*>(g + i) = float4{d[0], d[1], d[2], d[3]};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i + e >= f0 && i + e < f1) g[i + e] = d[e];
    }
  }
}

template <int LPR, int VPL>
__global__ __launch_bounds__(kThreads) void loss_kernel(
    const float* __restrict__ logits, const int* __restrict__ q2n, const int* __restrict__ qoff,
    const int* __restrict__ radix_ids, const int* __restrict__ token_ids,
    const int* __restrict__ coff, const int* __restrict__ ctok, const int* __restrict__ cval,
    const float* __restrict__ mass, float* __restrict__ d_logits, float* __restrict__ loss_out,
    int T_q, int V, int RB, float lambda, float inter_w, int ce_only) {
  __shared__ float buf[kChunk];
  __shared__ RowTabs tab;
  const int lane = threadIdx.x & 63;
  const int c = lane % LPR;
  const int base = lane - c;  // first lane of this row's group
  const int grp = threadIdx.x / LPR;
  constexpr int kGroups = kThreads / LPR;
  const float logV = logf(static_cast<float>(V));
  const int64_t step = static_cast<int64_t>(gridDim.x) * RB;
  int64_t r0 = static_cast<int64_t>(blockIdx.x) * RB;
  if (r0 >= T_q) return;
  float4 v[kMoveIters];
  int ni = 0, tg = -1;  // this thread's row of the run: node, next token
  float mwv = 1.0f;
  auto fetch = [&](int64_t r) {  // the run at r: bytes and first-level tables
    const int n = static_cast<int>(min(static_cast<int64_t>(RB), T_q - r));
    load_run(logits, v, r * V, (r + n) * V);
    if (static_cast<int>(threadIdx.x) < n) {
      const int64_t q = r + threadIdx.x;
      ni = q2n[q];
      tg = q + 1 < T_q ? token_ids[q + 1] : -1;
      mwv = mass != nullptr ? mass[q] : 1.0f;
    }
  };
  int ne = 0, rid = 0;  // second-level tables of this thread's row: node end, radix id
  auto fetch2 = [&](int64_t r) {
    if (static_cast<int64_t>(threadIdx.x) < min(static_cast<int64_t>(RB), T_q - r)) {
      ne = qoff[ni + 1];
      rid = radix_ids[ni];
    }
  };
  fetch(r0);
  fetch2(r0);
  for (;;) {
    const int n = static_cast<int>(min(static_cast<int64_t>(RB), T_q - r0));
    // The run's moves between HBM and LDS and their barriers at a higher
    // wave priority than the rows' arithmetic, so a workgroup moving its run
    // gets ahead of the others' rows and waits less at its barriers.
    __builtin_amdgcn_s_setprio(3);
    if (static_cast<int>(threadIdx.x) < n) {
      tab.tgt[threadIdx.x] = tg;
      tab.mw[threadIdx.x] = mwv;
      tab.end[threadIdx.x] = ne;
      tab.cs[threadIdx.x] = coff[rid];
      tab.ce[threadIdx.x] = coff[rid + 1];
    }
    run_to_lds(logits, v, buf, r0 * V, (r0 + n) * V);
    __syncthreads();
    const int64_t next = r0 + step;
    if (next < T_q) fetch(next);
    __builtin_amdgcn_s_setprio(0);
    for (int r = grp; r < n; r += kGroups) {
      const int64_t q = r0 + r;
      float* row = buf + r * V;
      float x[VPL];
      float mx = -FLT_MAX;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int j = Cols<LPR, VPL>::col(c, i);
        x[i] = j < V ? row[j] : -FLT_MAX;
        mx = fmaxf(mx, x[i]);
      }
      mx = group_max<LPR>(mx);
      // e^(x - max) as 2^(x log2e - max log2e): one multiply-add and the
      // hardware exp2 (relative error ~1e-6 over the softmax's range).
      const float ml = mx * kLog2e;
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int j = Cols<LPR, VPL>::col(c, i);
        x[i] = j < V ? fast_exp2(fmaf(x[i], kLog2e, -ml)) : 0.0f;
        s += x[i];
      }
      s = group_sum<LPR>(s);
      const float inv = 1.0f / s;
#pragma unroll
      for (int i = 0; i < VPL; ++i) x[i] *= inv;

      const bool endpoint = q + 1 == tab.end[r];
      const bool ce_inter = ce_only && endpoint && q + 1 < T_q;
      float loss = 0.0f, w = 1.0f;
      if (endpoint && !ce_inter) {
        const int start = tab.cs[r], end = tab.ce[r];
        if (start < end) {
          int tot = 0;
          for (int e = start + c; e < end; e += LPR) tot += cval[e];
          const float total = static_cast<float>(group_sum<LPR>(tot));
          float weight = 1.0f;
          if (lambda > 0.0f && end - start > 1) {
            float H = 0.0f;
            for (int e0 = start; e0 < end; e0 += LPR) {
              const int mine = e0 + c < end ? cval[e0 + c] : 0;
              const int m = min(LPR, end - e0);
              for (int t = 0; t < m; ++t) {
                const float qe = static_cast<float>(__shfl(mine, base + t, 64)) / total;
                if (qe > 0.0f) H -= qe * logf(qe);
              }
            }
            weight = 1.0f + lambda * (H / logV);
          }
          if (mass != nullptr) weight *= tab.mw[r];
          for (int e0 = start; e0 < end; e0 += LPR) {
            const bool have = e0 + c < end;
            const int mt = have ? ctok[e0 + c] : 0, mv = have ? cval[e0 + c] : 0;
            const int m = min(LPR, end - e0);
            for (int t = 0; t < m; ++t) {
              const int tok = __shfl(mt, base + t, 64);
              const float f = static_cast<float>(__shfl(mv, base + t, 64)) / total;
              if (tok < 0 || tok >= V) continue;  // outside the row: nothing to read or move
              const float p = row_value<LPR, VPL>(x, base, tok);
              loss -= f * logf(p + 1e-10f);
              sub_at<VPL>(x, Cols<LPR, VPL>::slot(tok), c == Cols<LPR, VPL>::owner(tok), f);
            }
          }
          w = weight;
        }
      } else {
        // q + 1 < T_q for every intermediate query of a well-formed batch.
        const int t = tab.tgt[r];
        if (t >= 0 && t < V) {
          const float p = row_value<LPR, VPL>(x, base, t);
          loss = -logf(p + 1e-10f);
          sub_at<VPL>(x, Cols<LPR, VPL>::slot(t), c == Cols<LPR, VPL>::owner(t), 1.0f);
        }
        w = inter_w;
        if (mass != nullptr) w *= tab.mw[r];
      }
      if (w != 1.0f) {
        loss *= w;
#pragma unroll
        for (int i = 0; i < VPL; ++i) x[i] *= w;
      }
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int j = Cols<LPR, VPL>::col(c, i);
        if (j < V) row[j] = x[i];
      }
      if (c == 0) loss_out[q] = loss;
    }
    if (next < T_q) fetch2(next);  // its first level arrived during the rows above
    __builtin_amdgcn_s_setprio(3);
    __syncthreads();
    store_run(d_logits, buf, r0 * V, (r0 + n) * V);
    if (next >= T_q) break;
    __syncthreads();  // the next run overwrites buf and tab
    r0 = next;
  }
}

// Workgroups: one per run, at most as many as are resident at once (every
// workgroup walks the same number of runs, so a second wave of workgroups
// would double the time).
template <typename K>
int grid_for(K kernel, int64_t runs) {
  int dev = 0, cus = 256, per_cu = 0;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int64_t cap = static_cast<int64_t>(cus) * per_cu;
  return static_cast<int>(runs < cap ? (runs > 0 ? runs : 1) : cap);
}

template <int LPR, int VPL>
void launch(const float* logits, const int* q2n, const int* qoff, const int* rids, const int* toks,
            const int* coff, const int* ctok, const int* cval, const float* mass, float* dl,
            float* lo, int T_q, int V, float lambda, float iw, int ce, hipStream_t st) {
  const int RB = std::min(kMaxRows, kChunk / V);
  const int64_t runs = (static_cast<int64_t>(T_q) + RB - 1) / RB;
  auto fn = loss_kernel<LPR, VPL>;
  hipLaunchKernelGGL(fn, dim3(grid_for(fn, runs)), dim3(kThreads), 0, st, logits, q2n,
                     qoff, rids, toks, coff, ctok, cval, mass, dl, lo, T_q, V, RB, lambda, iw, ce);
}

// Lanes per row: 4 up to 32 columns, 8 up to 128, 16 up to 512, a wave up
// to 1024; VPL columns per lane.
template <typename... A>
bool dispatch(int V, A... a) {
  if (V <= 16) launch<4, 4>(a...);
  else if (V <= 32) launch<4, 8>(a...);
  else if (V <= 40) launch<8, 5>(a...);
  else if (V <= 48) launch<8, 6>(a...);
  else if (V <= 64) launch<8, 8>(a...);
  else if (V <= 72) launch<8, 9>(a...);
  else if (V <= 80) launch<8, 10>(a...);
  else if (V <= 96) launch<8, 12>(a...);
  else if (V <= 128) launch<8, 16>(a...);
  else if (V <= 192) launch<16, 12>(a...);
  else if (V <= 256) launch<16, 16>(a...);
  else if (V <= 384) launch<16, 24>(a...);
  else if (V <= 512) launch<16, 32>(a...);
  else if (V <= 1024) launch<64, 16>(a...);
  else return false;
  return true;
}

}  // namespace

extern "C" int agpt_loss_per_query(const float* logits, const int* query_to_node,
                                   const int* query_offsets, const int* radix_ids,
                                   const int* token_ids, const int* counts_offset,
                                   const int* counts_tok, const int* counts_val,
                                   const float* mass_weights, float* d_logits, float* loss_out,
                                   int T_q, int V, float entropy_lambda, float intermediate_weight,
                                   int ce_only, void* stream) {
  if (T_q < 0 || V < 1)
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_loss_per_query: T_q < 0 or V < 1");
  if (T_q == 0) return AGPT_OK;
  if (!logits || !query_to_node || !query_offsets || !radix_ids || !token_ids || !counts_offset ||
      !counts_tok || !counts_val || !d_logits || !loss_out)
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_loss_per_query: null pointer");
  if (static_cast<int64_t>(T_q) * V > (static_cast<int64_t>(1) << 40))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_loss_per_query: T_q * V too large");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (!dispatch(V, logits, query_to_node, query_offsets, radix_ids, token_ids, counts_offset, counts_tok,
                counts_val, mass_weights, d_logits, loss_out, T_q, V, entropy_lambda, intermediate_weight,
                ce_only, st))
    return agpt_internal_set_error(AGPT_ERR_UNSUPPORTED, "agpt_loss_per_query: V > 1024 is not built");
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char msg[160];
    snprintf(msg, sizeof(msg), "agpt_loss_per_query: launch failed: %s", hipGetErrorString(e));
    return agpt_internal_set_error(AGPT_ERR_DEVICE, msg);
  }
  return AGPT_OK;
}

extern "C" int agpt_loss_mass_weights(const int* radix_ids, const int* edge_mass, const int* edge_lens,
                                      const int* query_offsets, int n_nodes, int T_q, int mode,
                                      float* out) {
  if (n_nodes < 0 || T_q < 0 || mode < AGPT_MASS_OFF || mode > AGPT_MASS_LINEAR)
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_loss_mass_weights: bad size or mode");
  if (n_nodes > 0 && (!radix_ids || !edge_mass || !edge_lens || !query_offsets || !out))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_loss_mass_weights: null pointer");
  // Per radix node w = f(edge_mass) (log1p / sqrt / identity / 1), normalised by the
  // query-weighted mean sum_i w_i L_i / T_q (agpt_train.cu:4608-4633).
  double total = 0.0;
  for (int i = 0; i < n_nodes; ++i) {
    const int r = radix_ids[i];
    const float m = static_cast<float>(edge_mass[r]);
    const float w = mode == AGPT_MASS_LOG ? logf(1.0f + m) : mode == AGPT_MASS_SQRT ? sqrtf(m)
                    : mode == AGPT_MASS_LINEAR ? m : 1.0f;
    total += static_cast<double>(w) * edge_lens[r];
  }
  float mean = T_q > 0 ? static_cast<float>(total / T_q) : 1.0f;
  if (mean <= 0.0f) mean = 1.0f;
  for (int i = 0; i < n_nodes; ++i) {
    const int r = radix_ids[i];
    const float m = static_cast<float>(edge_mass[r]);
    const float w = mode == AGPT_MASS_LOG ? logf(1.0f + m) : mode == AGPT_MASS_SQRT ? sqrtf(m)
                    : mode == AGPT_MASS_LINEAR ? m : 1.0f;
    const int a = query_offsets[i], b = query_offsets[i + 1];
    if (a < 0 || b > T_q || a > b)
      return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_loss_mass_weights: query_offsets out of range");
    for (int k = a; k < b; ++k) out[k] = w / mean;
  }
  return AGPT_OK;
}
