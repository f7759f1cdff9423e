// Row segments of 8 key features through buffer resources, shared by the key filter's forward
// (keys.hip) and backward (keys_backward.h) kernels.
#pragma once
#include "common.h"

namespace vsp {
namespace {

constexpr float kKeyFloor = 1e-6f;  // normalize_keys' floor (vesper/recurrence.py:31)

// One row segment of 8 features through a buffer resource: the raw load (kept packed until used),
// its float32 view, and the store of 8 float32 values in TZ.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
template <typename TZ> struct Row8;
template <> struct Row8<float> {
  struct Raw {
    u32x4 a, b;
  };
  static constexpr int kRun = 8;  // tokens per wave: 8 rows of 32 bytes in flight per lane
  __device__ __forceinline__ static Raw load(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
    return Raw{__builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0), __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16u, soff, 0)};
  }
  // two loads of which at most one was in range (the other read zeros), joined bitwise: exact
  __device__ __forceinline__ static Raw join(const Raw& x, const Raw& y) { return Raw{x.a | y.a, x.b | y.b}; }
  __device__ __forceinline__ static void unpack(const Raw& r, float (&x)[8]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = __uint_as_float(r.a[e]);
      x[4 + e] = __uint_as_float(r.b[e]);
    }
  }
  __device__ __forceinline__ static void store(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff, const float (&x)[8]) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{x[0], x[1], x[2], x[3]}), r, voff, soff, 0);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{x[4], x[5], x[6], x[7]}), r, voff + 16u, soff, 0);
  }
};
template <typename H8> struct Row8Half {
  using Raw = u32x4;
  static constexpr int kRun = 16;  // tokens per wave: 16 rows of 16 bytes in flight per lane
  __device__ __forceinline__ static Raw load(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  }
  __device__ __forceinline__ static Raw join(const Raw& x, const Raw& y) { return x | y; }
  __device__ __forceinline__ static void unpack(const Raw& r, float (&x)[8]) {
    const H8 h = __builtin_bit_cast(H8, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)h[e];
  }
  __device__ __forceinline__ static void store(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff, const float (&x)[8]) {
    H8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (decltype(h[0] + 0))x[e];
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, h), r, voff, soff, 0);
  }
};
template <> struct Row8<__bf16> : Row8Half<bf16x8> {};
template <> struct Row8<_Float16> : Row8Half<f16x8> {};

}  // namespace
}  // namespace vsp
