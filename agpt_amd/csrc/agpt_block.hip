// agpt_block.hip — the projection epilogue (bias + RoPE, in place) and the
// RMSProp update around the trie-attention path (gfx950).
//
// Both are streaming kernels (HBM-bound): the epilogue reads and writes each
// element once (8 bytes per element, + the tables from L2), RMSProp reads
// params, grads and the square average and writes two of them (20 bytes per
// parameter). Threads take 4 consecutive floats (16-byte accesses) and walk
// the array grid-strided.

#include "common.h"
#include "../../include/agpt_block.h"

#include <cmath>
#include <cstdio>
#include <type_traits>

namespace {

constexpr int kThreads = 256;

int grid_for(int64_t items) {
  int dev = 0, cus = 256;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t cap = static_cast<int64_t>(cus) * 8;
  const int64_t need = (items + kThreads - 1) / kThreads;
  return static_cast<int>(need < cap ? (need > 0 ? need : 1) : cap);
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return AGPT_OK;
  char msg[160];
  snprintf(msg, sizeof(msg), "%s: launch failed: %s", what, hipGetErrorString(e));
  return agpt_internal_set_error(AGPT_ERR_DEVICE, msg);
}

// Each thread owns quads (4 consecutive columns: two rotation pairs of one
// head, since head_dim % 4 == 0).
__global__ __launch_bounds__(kThreads) void bias_rope_kernel(float* __restrict__ x, const float* __restrict__ bias,
                                                             const int32_t* __restrict__ pos,
                                                             const float* __restrict__ cos_t,
                                                             const float* __restrict__ sin_t, int seq, int64_t T,
                                                             int D, int hd) {
  const int qpr = D / 4;  // quads per row
  const int64_t n = T * qpr;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t t = i / qpr;
    const int col = static_cast<int>(i - t * qpr) * 4;
    float4 v = *reinterpret_cast<const float4*>(x + t * D + col);
    if (bias != nullptr) {
      const float4 b = *reinterpret_cast<const float4*>(bias + col);
      v.x += b.x;
      v.y += b.y;
      v.z += b.z;
      v.w += b.w;
    }
    if (cos_t != nullptr) {
      int p = pos[t];
      p = p < 0 ? 0 : (p > seq - 1 ? seq - 1 : p);
      const int j = col % hd;  // pairs (j, j+1), (j+2, j+3)
      const float c0 = cos_t[static_cast<int64_t>(p) * hd + j], s0 = sin_t[static_cast<int64_t>(p) * hd + j];
      const float c1 = cos_t[static_cast<int64_t>(p) * hd + j + 2], s1 = sin_t[static_cast<int64_t>(p) * hd + j + 2];
      const float x0 = v.x, x1 = v.y, x2 = v.z, x3 = v.w;
      v.x = x0 * c0 - x1 * s0;
      v.y = x0 * s0 + x1 * c0;
      v.z = x2 * c1 - x3 * s1;
      v.w = x2 * s1 + x3 * c1;
    }
    *reinterpret_cast<float4*>(x + t * D + col) = v;
  }
}

// The [T, 3D] projection (q | k | v column blocks) split into contiguous
// [T, D] outputs: bias added to all three, RoPE on q and k.
__global__ __launch_bounds__(kThreads) void bias_rope_split_kernel(
    const float* __restrict__ x, const float* __restrict__ bias, const int32_t* __restrict__ pos,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int seq, int64_t T, int D, int hd,
    float* __restrict__ q, float* __restrict__ k, float* __restrict__ v) {
  const int qpr = 3 * D / 4;  // quads per input row
  const int64_t n = T * qpr;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t t = i / qpr;
    const int col3 = static_cast<int>(i - t * qpr) * 4;
    const int part = col3 / D, col = col3 - part * D;
    float4 w = *reinterpret_cast<const float4*>(x + t * 3 * D + col3);
    if (bias != nullptr) {
      const float4 b = *reinterpret_cast<const float4*>(bias + col3);
      w.x += b.x;
      w.y += b.y;
      w.z += b.z;
      w.w += b.w;
    }
    if (part < 2 && cos_t != nullptr) {
      int p = pos[t];
      p = p < 0 ? 0 : (p > seq - 1 ? seq - 1 : p);
      const int j = col % hd;
      const float c0 = cos_t[static_cast<int64_t>(p) * hd + j], s0 = sin_t[static_cast<int64_t>(p) * hd + j];
      const float c1 = cos_t[static_cast<int64_t>(p) * hd + j + 2], s1 = sin_t[static_cast<int64_t>(p) * hd + j + 2];
      const float x0 = w.x, x1 = w.y, x2 = w.z, x3 = w.w;
      w.x = x0 * c0 - x1 * s0;
      w.y = x0 * s0 + x1 * c0;
      w.z = x2 * c1 - x3 * s1;
      w.w = x2 * s1 + x3 * c1;
    }
    float* out = part == 0 ? q : (part == 1 ? k : v);
    *reinterpret_cast<float4*>(out + t * D + col) = w;
  }
}

__device__ __forceinline__ void rms_one(float& p, float g, float& s, float lr, float beta, float eps) {
  s = beta * s + (1.0f - beta) * (g * g);
  p -= lr * (g / (sqrtf(s) + eps));
}

__global__ __launch_bounds__(kThreads) void rmsprop_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                           float* __restrict__ s, float lr, float beta, float eps,
                                                           int64_t n) {
  const int64_t n4 = n / 4;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride) {
    float4 pv = reinterpret_cast<float4*>(p)[i];
    const float4 gv = reinterpret_cast<const float4*>(g)[i];
    float4 sv = reinterpret_cast<float4*>(s)[i];
    rms_one(pv.x, gv.x, sv.x, lr, beta, eps);
    rms_one(pv.y, gv.y, sv.y, lr, beta, eps);
    rms_one(pv.z, gv.z, sv.z, lr, beta, eps);
    rms_one(pv.w, gv.w, sv.w, lr, beta, eps);
    reinterpret_cast<float4*>(p)[i] = pv;
    reinterpret_cast<float4*>(s)[i] = sv;
  }
  // The n % 4 tail, one element per thread of the first workgroup.
  const int64_t k = n4 * 4 + threadIdx.x;
  if (blockIdx.x == 0 && k < n) {
    float pv = p[k], sv = s[k];
    rms_one(pv, g[k], sv, lr, beta, eps);
    p[k] = pv;
    s[k] = sv;
  }
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

// ---- RMSNorm / LayerNorm over rows of D = 16 * VPL floats -------------------
// 16 lanes own a row; lane c holds columns 64k + 4c + e (k < VPL/4, e < 4), so
// each 16-byte load of the 16 lanes covers 256 contiguous bytes. Row sums are
// DPP butterflies (row mirror, half mirror, quad reverse, pair swap), which
// leave the same bits in all 16 lanes. A wave works 4 rows at once.
template <int kCtrl>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dppf<0x140>(v);
  v += dppf<0x141>(v);
  v += dppf<0x1B>(v);
  return v + dppf<0xB1>(v);
}

constexpr int kNormBlocks = 1024;  // workgroups of the row kernels (and weight-gradient partials)

template <int VPL>
__device__ __forceinline__ void load_cols(const float* __restrict__ row, int c, float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / 4; ++k) {
    const float4 q = *reinterpret_cast<const float4*>(row + 64 * k + 4 * c);
    v[4 * k] = q.x;
    v[4 * k + 1] = q.y;
    v[4 * k + 2] = q.z;
    v[4 * k + 3] = q.w;
  }
}
template <int VPL>
__device__ __forceinline__ void store_cols(float* __restrict__ row, int c, const float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / 4; ++k)
    *reinterpret_cast<float4*>(row + 64 * k + 4 * c) = float4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
}

// y = (x - mean) * rstd * w + b (LayerNorm) or x * rstd * w (RMSNorm, b
// NULL), rstd = 1 / sqrt(var + eps) with var the mean of squares (of the
// centred row for LayerNorm). mean (LayerNorm) and rstd per row are saved.
template <int VPL, bool kLN>
__global__ __launch_bounds__(kThreads) void norm_fwd_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                            const float* __restrict__ b, float* __restrict__ y,
                                                            float* __restrict__ mean, float* __restrict__ rstd,
                                                            int64_t T, float eps) {
  constexpr int D = 16 * VPL;
  const int lane = threadIdx.x & 63, c = lane & 15;
  float wv[VPL], bv[VPL];
  load_cols<VPL>(w, c, wv);
  if constexpr (kLN) load_cols<VPL>(b, c, bv);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * (kThreads / 16);
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * (kThreads / 16) + (threadIdx.x >> 4); t < T; t += stride) {
    float v[VPL];
    load_cols<VPL>(x + t * D, c, v);
    float mu = 0.0f;
    if constexpr (kLN) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) s += v[i];
      mu = row16_sum(s) / static_cast<float>(D);
    }
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const float d = v[i] - mu;
      q += d * d;
    }
    const float r = 1.0f / sqrtf(row16_sum(q) / static_cast<float>(D) + eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      v[i] = (v[i] - mu) * r * wv[i];
      if constexpr (kLN) v[i] += bv[i];
    }
    store_cols<VPL>(y + t * D, c, v);
    if (c == 0) {
      rstd[t] = r;
      if constexpr (kLN) mean[t] = mu;
    }
  }
}

// dx = rstd (g - mean(g) - xh mean(g xh)) with g = dy w, xh the normalised
// row (RMSNorm: no mean(g) term); per-workgroup partials of dw = sum dy xh
// and db = sum dy, summed in a fixed order over the workgroup's rows. kRes:
// dx also adds dres (the gradient the residual stream brings to x).
template <int VPL, bool kLN, bool kRes>
__global__ __launch_bounds__(kThreads) void norm_bwd_kernel(const float* __restrict__ dy,
                                                            const float* __restrict__ dres,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ mean,
                                                            const float* __restrict__ rstd, float* __restrict__ dx,
                                                            float* __restrict__ part, int64_t T) {
  constexpr int D = 16 * VPL;
  constexpr int G = kThreads / 16;  // row groups per workgroup
  __shared__ float red[G][D];
  const int lane = threadIdx.x & 63, c = lane & 15, grp = threadIdx.x >> 4;
  float wv[VPL], dwa[VPL], dba[VPL];
  load_cols<VPL>(w, c, wv);
#pragma unroll
  for (int i = 0; i < VPL; ++i) dwa[i] = dba[i] = 0.0f;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * G;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * G + grp; t < T; t += stride) {
    float gy[VPL], xv[VPL];
    load_cols<VPL>(dy + t * D, c, gy);
    load_cols<VPL>(x + t * D, c, xv);
    const float mu = kLN ? mean[t] : 0.0f, r = rstd[t];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      xv[i] = (xv[i] - mu) * r;  // xh
      const float g = gy[i] * wv[i];
      s1 += g;
      s2 += g * xv[i];
      dwa[i] += gy[i] * xv[i];
      dba[i] += gy[i];
    }
    s2 = row16_sum(s2) / static_cast<float>(D);
    s1 = kLN ? row16_sum(s1) / static_cast<float>(D) : 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) gy[i] = r * (gy[i] * wv[i] - s1 - xv[i] * s2);
    if constexpr (kRes) {
      float rv[VPL];
      load_cols<VPL>(dres + t * D, c, rv);
#pragma unroll
      for (int i = 0; i < VPL; ++i) gy[i] += rv[i];
    }
    store_cols<VPL>(dx + t * D, c, gy);
  }
  // the workgroup's G row groups, added in group order
#pragma unroll
  for (int k = 0; k < VPL / 4; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[grp][64 * k + 4 * c + e] = dwa[4 * k + e];
  __syncthreads();
  for (int j = threadIdx.x; j < D; j += kThreads) {
    float a = 0.0f;
    for (int q = 0; q < G; ++q) a += red[q][j];
    part[static_cast<int64_t>(blockIdx.x) * D + j] = a;
  }
  if constexpr (kLN) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < VPL / 4; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[grp][64 * k + 4 * c + e] = dba[4 * k + e];
    __syncthreads();
    for (int j = threadIdx.x; j < D; j += kThreads) {
      float a = 0.0f;
      for (int q = 0; q < G; ++q) a += red[q][j];
      part[static_cast<int64_t>(gridDim.x + blockIdx.x) * D + j] = a;
    }
  }
}

// out[j] = sum over n partial rows of part[., j], in row order.
// out[j] = sum over q of part[q][j], D a multiple of 64. One workgroup per 64
// columns: 16 lanes x float4 across the columns, 16 row slots down the rows
// (slot s sums rows s, s+16, ...), then slot 0 folds the 16 slot sums in
// order, so the result does not depend on timing.
constexpr int kColSlots = kThreads / 16;
__global__ __launch_bounds__(kThreads) void col_sum_kernel(const float* __restrict__ part, int n, int D,
                                                           float* __restrict__ out) {
  __shared__ float4 red[kColSlots][16];
  const int c4 = threadIdx.x & 15, slot = threadIdx.x >> 4;
  const float4* p = reinterpret_cast<const float4*>(part) + blockIdx.x * 16 + c4;
  const int D4 = D / 4;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (int q = slot; q < n; q += kColSlots) {
    const float4 v = p[static_cast<int64_t>(q) * D4];
    a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w;
  }
  red[slot][c4] = a;
  __syncthreads();
  if (slot == 0) {
    for (int t = 1; t < kColSlots; ++t) {
      const float4 v = red[t][c4];
      a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w;
    }
    reinterpret_cast<float4*>(out)[blockIdx.x * 16 + c4] = a;
  }
}

// dh = dy where h > 0, else 0 (the ReLU's backward through its output h);
// per-workgroup partials of db = sum over rows of dh, in a fixed order. dh
// may alias dy (each thread reads a row's slice before it writes it).
template <int VPL>
__global__ __launch_bounds__(kThreads) void relu_bwd_kernel(const float* dy, const float* __restrict__ h, float* dh,
                                                            float* __restrict__ part, int64_t T) {
  constexpr int D = 16 * VPL;
  constexpr int G = kThreads / 16;  // row groups per workgroup
  __shared__ float red[G][D];
  const int c = threadIdx.x & 15, grp = threadIdx.x >> 4;
  float dba[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) dba[i] = 0.0f;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * G;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * G + grp; t < T; t += stride) {
    float gy[VPL], hv[VPL];
    load_cols<VPL>(dy + t * D, c, gy);
    load_cols<VPL>(h + t * D, c, hv);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      gy[i] = hv[i] > 0.0f ? gy[i] : 0.0f;
      dba[i] += gy[i];
    }
    store_cols<VPL>(dh + t * D, c, gy);
  }
#pragma unroll
  for (int k = 0; k < VPL / 4; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[grp][64 * k + 4 * c + e] = dba[4 * k + e];
  __syncthreads();
  for (int j = threadIdx.x; j < D; j += kThreads) {
    float a = 0.0f;
    for (int q = 0; q < G; ++q) a += red[q][j];
    part[static_cast<int64_t>(blockIdx.x) * D + j] = a;
  }
}

template <typename Fn>
bool with_vpl(int D, Fn&& fn) {
  switch (D) {
    case 64: fn(std::integral_constant<int, 4>{}); return true;
    case 128: fn(std::integral_constant<int, 8>{}); return true;
    case 256: fn(std::integral_constant<int, 16>{}); return true;
    case 512: fn(std::integral_constant<int, 32>{}); return true;
    default: return false;
  }
}

}  // namespace

extern "C" int64_t agpt_norm_workspace_floats(int d_model) { return 2 * static_cast<int64_t>(kNormBlocks) * d_model; }

extern "C" int agpt_norm_fwd(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
                             int64_t T, int d_model, float eps, void* stream) {
  if (T < 0) return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_norm_fwd: T < 0");
  if (T == 0) return AGPT_OK;
  if (!x || !w || !y || !rstd || (b && !mean))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_norm_fwd: null pointer");
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || (b && !aligned16(b)))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_norm_fwd: x, w, b, y must be 16-byte aligned");
  const int64_t need = (T + kThreads / 16 - 1) / (kThreads / 16);
  const int grid = static_cast<int>(need < kNormBlocks ? need : kNormBlocks);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = with_vpl(d_model, [&](auto vc) {
    constexpr int VPL = decltype(vc)::value;
    if (b) hipLaunchKernelGGL((norm_fwd_kernel<VPL, true>), dim3(grid), dim3(kThreads), 0, st, x, w, b, y, mean, rstd, T, eps);
    else hipLaunchKernelGGL((norm_fwd_kernel<VPL, false>), dim3(grid), dim3(kThreads), 0, st, x, w, b, y, mean, rstd, T, eps);
  });
  if (!ok) return agpt_internal_set_error(AGPT_ERR_UNSUPPORTED, "agpt_norm_fwd: d_model must be 64, 128, 256 or 512");
  return launch_status("agpt_norm_fwd");
}

extern "C" int agpt_norm_bwd(const float* dy, const float* dres, const float* x, const float* w, const float* mean, const float* rstd,
                             float* dx, float* dw, float* db, float* workspace, int64_t workspace_floats, int64_t T,
                             int d_model, void* stream) {
  if (T < 0) return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_norm_bwd: T < 0");
  if (!dy || !x || !w || !rstd || !dx || !dw || !workspace || (db && !mean))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_norm_bwd: null pointer");
  if (workspace_floats < agpt_norm_workspace_floats(d_model))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_norm_bwd: workspace smaller than agpt_norm_workspace_floats");
  if (!aligned16(dy) || (dres && !aligned16(dres)) || !aligned16(x) || !aligned16(w) || !aligned16(dx) || !aligned16(dw) ||
      (db && !aligned16(db)) || !aligned16(workspace))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG,
                                   "agpt_norm_bwd: dy, dres, x, w, dx, dw, db and workspace must be 16-byte aligned");
  const int64_t need = (T + kThreads / 16 - 1) / (kThreads / 16);
  const int grid = static_cast<int>(need < 1 ? 1 : (need < kNormBlocks ? need : kNormBlocks));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = with_vpl(d_model, [&](auto vc) {
    constexpr int VPL = decltype(vc)::value;
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), 0, st, dy, dres, x, w, mean, rstd, dx, workspace, T);
    };
    if (db) dres ? go(norm_bwd_kernel<VPL, true, true>) : go(norm_bwd_kernel<VPL, true, false>);
    else dres ? go(norm_bwd_kernel<VPL, false, true>) : go(norm_bwd_kernel<VPL, false, false>);
  });
  if (!ok) return agpt_internal_set_error(AGPT_ERR_UNSUPPORTED, "agpt_norm_bwd: d_model must be 64, 128, 256 or 512");
  const int cgrid = d_model / 64;
  hipLaunchKernelGGL(col_sum_kernel, dim3(cgrid), dim3(kThreads), 0, st, workspace, grid, d_model, dw);
  if (db)
    hipLaunchKernelGGL(col_sum_kernel, dim3(cgrid), dim3(kThreads), 0, st,
                       workspace + static_cast<int64_t>(grid) * d_model, grid, d_model, db);
  return launch_status("agpt_norm_bwd");
}

extern "C" int agpt_relu_bwd(const float* dy, const float* h, float* dh, float* db, float* workspace,
                             int64_t workspace_floats, int64_t T, int width, void* stream) {
  if (T < 0) return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_relu_bwd: T < 0");
  if (!dy || !h || !dh || !db || !workspace)
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_relu_bwd: null pointer");
  if (workspace_floats < agpt_norm_workspace_floats(width))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_relu_bwd: workspace smaller than agpt_norm_workspace_floats");
  if (!aligned16(dy) || !aligned16(h) || !aligned16(dh) || !aligned16(db) || !aligned16(workspace))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_relu_bwd: dy, h, dh, db and workspace must be 16-byte aligned");
  const int64_t need = (T + kThreads / 16 - 1) / (kThreads / 16);
  const int grid = static_cast<int>(need < 1 ? 1 : (need < kNormBlocks ? need : kNormBlocks));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = with_vpl(width, [&](auto vc) {
    constexpr int VPL = decltype(vc)::value;
    hipLaunchKernelGGL((relu_bwd_kernel<VPL>), dim3(grid), dim3(kThreads), 0, st, dy, h, dh, workspace, T);
  });
  if (!ok) return agpt_internal_set_error(AGPT_ERR_UNSUPPORTED, "agpt_relu_bwd: width must be 64, 128, 256 or 512");
  hipLaunchKernelGGL(col_sum_kernel, dim3(width / 64), dim3(kThreads), 0, st, workspace, grid, width, db);
  return launch_status("agpt_relu_bwd");
}

extern "C" int agpt_bias_rope(float* x, const float* bias, const int32_t* positions, const float* cos_t,
                              const float* sin_t, int rope_seq_len, int64_t T, int n_heads, int head_dim,
                              void* stream) {
  if (T < 0 || n_heads < 1 || head_dim < 4 || head_dim % 4 != 0)
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_bias_rope: T < 0, n_heads < 1 or head_dim not a multiple of 4");
  if (T == 0) return AGPT_OK;
  if (!x || (cos_t && (!sin_t || !positions || rope_seq_len < 1)))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_bias_rope: null pointer or rope_seq_len < 1");
  if (!aligned16(x) || (bias && !aligned16(bias)))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_bias_rope: x and bias must be 16-byte aligned");
  const int D = n_heads * head_dim;
  hipLaunchKernelGGL(bias_rope_kernel, dim3(grid_for(T * (D / 4))), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), x, bias, positions, cos_t, sin_t, rope_seq_len, T, D,
                     head_dim);
  return launch_status("agpt_bias_rope");
}

extern "C" int agpt_bias_rope_split(const float* qkv, const float* bias, const int32_t* positions,
                                    const float* cos_t, const float* sin_t, int rope_seq_len, int64_t T,
                                    int n_heads, int head_dim, float* q, float* k, float* v, void* stream) {
  if (T < 0 || n_heads < 1 || head_dim < 4 || head_dim % 4 != 0)
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG,
                                   "agpt_bias_rope_split: T < 0, n_heads < 1 or head_dim not a multiple of 4");
  if (T == 0) return AGPT_OK;
  if (!qkv || !q || !k || !v || (cos_t && (!sin_t || !positions || rope_seq_len < 1)))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_bias_rope_split: null pointer or rope_seq_len < 1");
  if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) || !aligned16(v) || (bias && !aligned16(bias)))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_bias_rope_split: buffers must be 16-byte aligned");
  const int D = n_heads * head_dim;
  hipLaunchKernelGGL(bias_rope_split_kernel, dim3(grid_for(T * (3 * D / 4))), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), qkv, bias, positions, cos_t, sin_t, rope_seq_len, T, D,
                     head_dim, q, k, v);
  return launch_status("agpt_bias_rope_split");
}

extern "C" int agpt_rmsprop(float* params, const float* grads, float* sq_avg, float lr, float beta, float eps,
                            int64_t n, void* stream) {
  if (n < 0) return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_rmsprop: n < 0");
  if (n == 0) return AGPT_OK;
  if (!params || !grads || !sq_avg)
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_rmsprop: null pointer");
  if (!aligned16(params) || !aligned16(grads) || !aligned16(sq_avg))
    return agpt_internal_set_error(AGPT_ERR_INVALID_ARG, "agpt_rmsprop: buffers must be 16-byte aligned");
  hipLaunchKernelGGL(rmsprop_kernel, dim3(grid_for(n / 4 + 1)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     params, grads, sq_avg, lr, beta, eps, n);
  return launch_status("agpt_rmsprop");
}
