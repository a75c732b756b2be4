// varlen_attn.hip — drop-ins for the reference's packed varlen attention
// externs (agpt_train.cu:73-86, 3120-3132), fp32, gfx950.
//
// These keep the reference's packed layout, where every node / radix node
// carries its own copy of its ancestors' K/V rows, so callers such as
// batched_depth_forward.cr:767 and agpt_train.cu:4740/4988 can switch by
// renaming. The trie-native path (trie_attn.hip) avoids that duplication.
//
// Forward: thread per (query, head); scores are staged in weights_out (the
// saved weights the reference's backward reads), softmax, P·V.
// Backward from saved weights, with the reference's Float64 softmax-backward
// dot (batched_depth_backward.cr:637-651). The L-query backward accumulates
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

template <int HD>
__global__ __launch_bounds__(256) void varlen_fwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const int* __restrict__ kv_off, const int* __restrict__ kv_len, const int* __restrict__ q2n,
    const int* __restrict__ qoff, float* __restrict__ out, float* __restrict__ weights, int n_q,
    int H, int max_len, float scale) {
  const int item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= n_q * H) return;
  const int qi = item / H, h = item - (item / H) * H;
  int node;
  const int len = visible_len(qi, q2n, qoff, kv_len, max_len, &node);
  const int64_t off = kv_off[node];
  float qq[HD], acc[HD];
  load_vec<HD>(q + (static_cast<int64_t>(qi) * H + h) * HD, qq);
#pragma unroll
  for (int i = 0; i < HD; ++i) acc[i] = 0.0f;
  float* w = weights + (static_cast<int64_t>(qi) * H + h) * max_len;
  float m = -INFINITY;
  for (int p = 0; p < len; ++p) {
    float kk[HD];
    load_vec<HD>(k + ((off + p) * H + h) * HD, kk);
    float sc = 0.0f;
#pragma unroll
    for (int i = 0; i < HD; ++i) sc += qq[i] * kk[i];
    sc *= scale;
    w[p] = sc;
    m = fmaxf(m, sc);
  }
  float sum = 0.0f;
  for (int p = 0; p < len; ++p) {
    const float ex = fast_exp2((w[p] - m) * kLog2e);
    w[p] = ex;
    sum += ex;
  }
  const float inv = len > 0 ? 1.0f / sum : 0.0f;
  for (int p = 0; p < len; ++p) {
    const float wp = w[p] * inv;
    w[p] = wp;
    float vv[HD];
    load_vec<HD>(v + ((off + p) * H + h) * HD, vv);
#pragma unroll
    for (int i = 0; i < HD; ++i) acc[i] += wp * vv[i];
  }
  store_vec<HD>(out + (static_cast<int64_t>(qi) * H + h) * HD, acc);
}

// Node-level backward: every packed row belongs to exactly one node, so the
// thread of (node, head) owns its rows and writes them.
template <int HD>
__global__ __launch_bounds__(256) void varlen_bwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ weights, const float* __restrict__ d_out,
    const int* __restrict__ kv_off, const int* __restrict__ kv_len, float* __restrict__ dq,
    float* __restrict__ dk, float* __restrict__ dv, int n_nodes, int H, int max_len, float scale) {
  const int item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= n_nodes * H) return;
  const int i = item / H, h = item - (item / H) * H;
  int node;
  const int len = visible_len(i, nullptr, nullptr, kv_len, max_len, &node);
  const int64_t off = kv_off[node];
  float g[HD], qq[HD], dqa[HD];
  load_vec<HD>(d_out + (static_cast<int64_t>(i) * H + h) * HD, g);
  load_vec<HD>(q + (static_cast<int64_t>(i) * H + h) * HD, qq);
#pragma unroll
  for (int j = 0; j < HD; ++j) dqa[j] = 0.0f;
  const float* w = weights + (static_cast<int64_t>(i) * H + h) * max_len;
  double dot = 0.0;
  for (int p = 0; p < len; ++p) {
    float vv[HD];
    load_vec<HD>(v + ((off + p) * H + h) * HD, vv);
    float dw = 0.0f;
#pragma unroll
    for (int j = 0; j < HD; ++j) dw += g[j] * vv[j];
    dot += static_cast<double>(dw * w[p]);
  }
  for (int p = 0; p < len; ++p) {
    float vv[HD], kk[HD];
    load_vec<HD>(v + ((off + p) * H + h) * HD, vv);
    load_vec<HD>(k + ((off + p) * H + h) * HD, kk);
    float dw = 0.0f;
#pragma unroll
    for (int j = 0; j < HD; ++j) dw += g[j] * vv[j];
    const float wp = w[p];
    const float ds = static_cast<float>(static_cast<double>(wp) * (static_cast<double>(dw) - dot) *
                                        static_cast<double>(scale));
    float rk[HD], rv[HD];
#pragma unroll
    for (int j = 0; j < HD; ++j) {
      dqa[j] += ds * kk[j];
      rk[j] = ds * qq[j];
      rv[j] = wp * g[j];
    }
    store_vec<HD>(dk + ((off + p) * H + h) * HD, rk);
    store_vec<HD>(dv + ((off + p) * H + h) * HD, rv);
  }
  store_vec<HD>(dq + (static_cast<int64_t>(i) * H + h) * HD, dqa);
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
  const int items = n_nodes * n_heads;
  const int rc = dispatch(head_dim, [&](auto c) {
    constexpr int HD = decltype(c)::value;
    hipLaunchKernelGGL((varlen_fwd_kernel<HD>), dim3((items + 255) / 256), dim3(256), 0,
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
  const int items = n_nodes * n_heads;
  const int rc = dispatch(head_dim, [&](auto c) {
    constexpr int HD = decltype(c)::value;
    hipLaunchKernelGGL((varlen_bwd_kernel<HD>), dim3((items + 255) / 256), dim3(256), 0,
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
  const int items = T_q * n_heads;
  const int rc = dispatch(head_dim, [&](auto c) {
    constexpr int HD = decltype(c)::value;
    hipLaunchKernelGGL((varlen_fwd_kernel<HD>), dim3((items + 255) / 256), dim3(256), 0,
                       static_cast<hipStream_t>(stream), q, k, v, kv_offsets, kv_lengths, query_to_node,
                       query_offsets, output, weights_out, T_q, n_heads, max_kv_len, scale);
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
    hipLaunchKernelGGL((varlen_L_bwd_kernel<HD>), dim3(T_q, n_heads), dim3(64),
                       sizeof(double) * max_kv_len, static_cast<hipStream_t>(stream), q, k, v,
                       attn_weights, d_out, query_to_node, query_offsets, kv_offsets, kv_lengths, dq,
                       dk_full, dv_full, n_heads, max_kv_len, scale);
  });
  return rc != AGPT_OK ? rc : finish_launch();
}
