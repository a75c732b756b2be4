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

}  // namespace

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
