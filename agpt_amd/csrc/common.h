// common.h — device helpers shared by the gfx950 trie-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Records `msg` as the calling thread's last error and returns `code`
// (defined in trie_attn.hip, shared by every entry point of the library).
int agpt_internal_set_error(int code, const char* msg);

namespace agpt {

// Largest tile: a tile is a contiguous DFS-preorder range of node-tokens.
constexpr int kMaxTileRows = 256;
// Deepest supported node (keys per query).
constexpr int kMaxDepth = 256;
// Widest supported head count (LDS tables are sized for it).
constexpr int kMaxHeads = 16;
// Tiles folded into one first-level partial sum of the dK/dV reduction.
constexpr int kChunkTiles = 32;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}

__device__ __forceinline__ void from_f32(float x, float* dst) { *dst = x; }
__device__ __forceinline__ void from_f32(float x, bf16_t* dst) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u) {  // inf / nan: truncate, keep nan quiet
    dst->bits = static_cast<uint16_t>((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
    return;
  }
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  dst->bits = static_cast<uint16_t>(u >> 16);
}

// Loads HD consecutive elements (16-byte aligned for fp32 HD%4==0,
// 8/16-byte aligned for bf16) into fp32 registers.
template <int HD>
__device__ __forceinline__ void load_vec(const float* __restrict__ p, float (&x)[HD]) {
  static_assert(HD % 4 == 0, "head_dim must be a multiple of 4");
#pragma unroll
  for (int i = 0; i < HD; i += 4) {
    const float4 v = *reinterpret_cast<const float4*>(p + i);
    x[i] = v.x;
    x[i + 1] = v.y;
    x[i + 2] = v.z;
    x[i + 3] = v.w;
  }
}

template <int HD>
__device__ __forceinline__ void load_vec(const bf16_t* __restrict__ p, float (&x)[HD]) {
  static_assert(HD % 4 == 0, "head_dim must be a multiple of 4");
  if constexpr (HD % 8 == 0) {
#pragma unroll
    for (int i = 0; i < HD; i += 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(p + i);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x[i + 2 * k] = __uint_as_float(w[k] << 16);
        x[i + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < HD; i += 4) {
      const uint2 v = *reinterpret_cast<const uint2*>(p + i);
      x[i] = __uint_as_float(v.x << 16);
      x[i + 1] = __uint_as_float(v.x & 0xffff0000u);
      x[i + 2] = __uint_as_float(v.y << 16);
      x[i + 3] = __uint_as_float(v.y & 0xffff0000u);
    }
  }
}

template <int HD>
__device__ __forceinline__ void store_vec(float* __restrict__ p, const float (&x)[HD]) {
#pragma unroll
  for (int i = 0; i < HD; i += 4)
    *reinterpret_cast<float4*>(p + i) = make_float4(x[i], x[i + 1], x[i + 2], x[i + 3]);
}

// Two floats rounded to nearest-even bf16 by one v_cvt_pk_bf16_f32 (NaN
// stays NaN), the first in the low half.
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  typedef __attribute__((ext_vector_type(2))) float f2;
  typedef __attribute__((ext_vector_type(2))) __bf16 b2;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, b2));
}

// bf16 stores: groups of four as one 8-byte store (p 8-byte aligned when
// HD % 4 == 0, as every caller's row and head offsets are).
template <int HD>
__device__ __forceinline__ void store_vec(bf16_t* __restrict__ p, const float (&x)[HD]) {
  if constexpr (HD % 4 == 0) {
#pragma unroll
    for (int i = 0; i < HD; i += 4)
      *reinterpret_cast<uint2*>(p + i) = uint2{pack2_bf16(x[i], x[i + 1]), pack2_bf16(x[i + 2], x[i + 3])};
  } else {
#pragma unroll
    for (int i = 0; i < HD; ++i) from_f32(x[i], p + i);
  }
}

// Inverse RoPE on one head slice (batched_depth_backward.cr:738-748): the
// transpose of the rotation at `pos`; tables are [seq, HD] with entry
// [pos, 2i] used for the pair (2i, 2i+1).
template <int HD>
__device__ __forceinline__ void rope_inverse(float (&x)[HD], const float* __restrict__ cos_t,
                                             const float* __restrict__ sin_t, int pos) {
#pragma unroll
  for (int i = 0; i < HD / 2; ++i) {
    const float c = cos_t[pos * HD + 2 * i];
    const float s = sin_t[pos * HD + 2 * i];
    const float x0 = x[2 * i], x1 = x[2 * i + 1];
    x[2 * i] = x0 * c + x1 * s;
    x[2 * i + 1] = -x0 * s + x1 * c;
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

}  // namespace agpt
