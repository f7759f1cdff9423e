// MFMA operand helpers shared by the window attention kernels (window_attn.hip: forward;
// window_attn_backward.hip: gradients).
#pragma once
#include "common.h"

namespace vsp {
namespace {

template <typename T> struct Mma;
template <> struct Mma<__bf16> {
  using V8 = bf16x8;
  using V4 = bf16x4;
  __device__ __forceinline__ static f32x4 run(V8 a, V8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<_Float16> {
  using V8 = f16x8;
  using V4 = f16x4;
  __device__ __forceinline__ static f32x4 run(V8 a, V8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ typename Mma<T>::V4 read_tr(const T* p) {
  return read_tr16<typename Mma<T>::V4>(p);
}

// IEEE maximum (NaN-propagating): v_maximum3_f32 / v_maximum_f32, which need no operand
// canonicalisation, unlike fmaxf's v_max_f32
__device__ __forceinline__ float fmax_ieee(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lane groups of one query)
__device__ __forceinline__ float max_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmax_ieee(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax_ieee(__uint_as_float(c[0]), __uint_as_float(c[1]));
}

}  // namespace
}  // namespace vsp
