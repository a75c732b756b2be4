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
// Layout: LPR lanes own one row (LPR = 16 for V <= 128, else 64), lane c of
// the row holding columns c, c + LPR, ...; a wave covers 64/LPR rows at once
// and walks the rows grid-strided. The row is read once and written once:
// the loss is HBM-bound at 8V bytes per query. The count entries of an
// endpoint are applied one at a time in their stored order (as the
// reference's single thread does), so repeated tokens and the loss sum come
// out in the same order.

#include "common.h"
#include "../../include/agpt_loss.h"

#include <cfloat>
#include <cmath>
#include <cstdio>

namespace {

constexpr int kThreads = 256;

template <int LPR>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int LPR>
__device__ __forceinline__ int group_isum(int v) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Value of column j of the row held by this lane's group (j uniform over the
// group): the owner lane is base + j % LPR, the register j / LPR.
template <int LPR, int VPL>
__device__ __forceinline__ float row_value(const float (&x)[VPL], int base, int j) {
  const int slot = j / LPR;
  float v = x[0];
#pragma unroll
  for (int i = 1; i < VPL; ++i) v = slot == i ? x[i] : v;
  return __shfl(v, base + j % LPR, 64);
}
template <int VPL>
__device__ __forceinline__ void sub_at(float (&x)[VPL], int slot, bool own, float d) {
#pragma unroll
  for (int i = 0; i < VPL; ++i)
    if (own && slot == i) x[i] -= d;
}

template <int LPR, int VPL>
__global__ __launch_bounds__(kThreads) void loss_kernel(
    const float* __restrict__ logits, const int* __restrict__ q2n, const int* __restrict__ qoff,
    const int* __restrict__ radix_ids, const int* __restrict__ token_ids,
    const int* __restrict__ coff, const int* __restrict__ ctok, const int* __restrict__ cval,
    const float* __restrict__ mass, float* __restrict__ d_logits, float* __restrict__ loss_out,
    int T_q, int V, float lambda, float inter_w, int ce_only) {
  constexpr int RPW = 64 / LPR;  // rows per wave
  const int lane = threadIdx.x & 63;
  const int c = lane % LPR;
  const int base = lane - c;  // first lane of this row's group
  const int64_t stride = static_cast<int64_t>(gridDim.x) * (kThreads / 64) * RPW;
  const float logV = logf(static_cast<float>(V));
  for (int64_t q0 = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6)) * RPW;
       q0 < T_q; q0 += stride) {
    const int64_t q = q0 + lane / LPR;
    const bool row = q < T_q;
    const float* in = logits + q * V;
    float x[VPL];
    float mx = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = c + LPR * i;
      x[i] = row && j < V ? in[j] : -FLT_MAX;
      mx = fmaxf(mx, x[i]);
    }
    int n_idx = 0, node_end = 0;
    if (row) {
      n_idx = q2n[q];
      node_end = qoff[n_idx + 1];
    }
    mx = group_max<LPR>(mx);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = c + LPR * i;
      x[i] = j < V ? expf(x[i] - mx) : 0.0f;
      s += x[i];
    }
    s = group_sum<LPR>(s);
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < VPL; ++i) x[i] *= inv;

    const bool endpoint = q + 1 == node_end;
    const bool ce_inter = ce_only && endpoint && q + 1 < T_q;
    float loss = 0.0f, w = 1.0f;
    if (row && endpoint && !ce_inter) {
      const int rid = radix_ids[n_idx];
      const int start = coff[rid], end = coff[rid + 1];
      if (start < end) {
        int tot = 0;
        for (int e = start + c; e < end; e += LPR) tot += cval[e];
        const float total = static_cast<float>(group_isum<LPR>(tot));
        float weight = 1.0f;
        if (lambda > 0.0f && end - start > 1) {
          float H = 0.0f;
          for (int e0 = start; e0 < end; e0 += LPR) {
            const int mine = e0 + c < end ? cval[e0 + c] : 0;
            const int n = min(LPR, end - e0);
            for (int k = 0; k < n; ++k) {
              const float qe = static_cast<float>(__shfl(mine, base + k, 64)) / total;
              if (qe > 0.0f) H -= qe * logf(qe);
            }
          }
          weight = 1.0f + lambda * (H / logV);
        }
        if (mass != nullptr) weight *= mass[q];
        for (int e0 = start; e0 < end; e0 += LPR) {
          const bool have = e0 + c < end;
          const int mt = have ? ctok[e0 + c] : 0, mv = have ? cval[e0 + c] : 0;
          const int n = min(LPR, end - e0);
          for (int k = 0; k < n; ++k) {
            const int tok = __shfl(mt, base + k, 64);
            const float f = static_cast<float>(__shfl(mv, base + k, 64)) / total;
            if (tok < 0 || tok >= V) continue;  // outside the row: nothing to read or move
            const float p = row_value<LPR, VPL>(x, base, tok);
            loss -= f * logf(p + 1e-10f);
            sub_at<VPL>(x, tok / LPR, c == tok % LPR, f);
          }
        }
        w = weight;
      }
    } else if (row) {
      // q + 1 < T_q for every intermediate query of a well-formed batch.
      const int t = q + 1 < T_q ? token_ids[q + 1] : -1;
      if (t >= 0 && t < V) {
        const float p = row_value<LPR, VPL>(x, base, t);
        loss = -logf(p + 1e-10f);
        sub_at<VPL>(x, t / LPR, c == t % LPR, 1.0f);
      }
      w = inter_w;
      if (mass != nullptr) w *= mass[q];
    }
    if (w != 1.0f) {
      loss *= w;
#pragma unroll
      for (int i = 0; i < VPL; ++i) x[i] *= w;
    }
    if (row) {
      float* out = d_logits + q * V;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int j = c + LPR * i;
        if (j < V) out[j] = x[i];
      }
      if (c == 0) loss_out[q] = loss;
    }
  }
}

int grid_for(int64_t groups) {
  int dev = 0, cus = 256;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t cap = static_cast<int64_t>(cus) * 16;
  const int64_t need = (groups + kThreads / 64 - 1) / (kThreads / 64);
  return static_cast<int>(need < cap ? (need > 0 ? need : 1) : cap);
}

template <int LPR, int VPL>
void launch(const float* logits, const int* q2n, const int* qoff, const int* rids, const int* toks,
            const int* coff, const int* ctok, const int* cval, const float* mass, float* dl,
            float* lo, int T_q, int V, float lambda, float iw, int ce, hipStream_t st) {
  const int64_t groups = (static_cast<int64_t>(T_q) + 64 / LPR - 1) / (64 / LPR);
  hipLaunchKernelGGL((loss_kernel<LPR, VPL>), dim3(grid_for(groups)), dim3(kThreads), 0, st, logits,
                     q2n, qoff, rids, toks, coff, ctok, cval, mass, dl, lo, T_q, V, lambda, iw, ce);
}

// Rows of up to 128 columns: 16 lanes per row, VPL = ceil(V / 16).
// Wider rows: a wave per row, VPL = ceil(V / 64) rounded up to 4, 8 or 16.
template <typename... A>
bool dispatch(int V, A... a) {
  if (V <= 16) launch<16, 1>(a...);
  else if (V <= 32) launch<16, 2>(a...);
  else if (V <= 48) launch<16, 3>(a...);
  else if (V <= 64) launch<16, 4>(a...);
  else if (V <= 80) launch<16, 5>(a...);
  else if (V <= 96) launch<16, 6>(a...);
  else if (V <= 128) launch<16, 8>(a...);
  else if (V <= 256) launch<64, 4>(a...);
  else if (V <= 512) launch<64, 8>(a...);
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
