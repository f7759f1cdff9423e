// The rotary embedding's arithmetic on one pair, shared by the rotary kernel and the decode step's
// fused attention projection (which rotates q and k as it stores them), so both give the same bits.
//
// Reference: vesper/attention.py:178-217 (`rotary`): the angle p * base^(-2j/dk) in float64, its cos
// and sin cast to the activations' dtype, and x1 cos - x2 sin, x1 sin + x2 cos evaluated in that
// dtype (each product and the sum rounded to it, as torch evaluates it).
#pragma once

#include "common.h"

namespace vsp {

// double to T through float, as torch casts a float64 tensor to a 16-bit one (two roundings). The
// float is pinned in a register first: otherwise the two conversions are folded into one direct
// (singly rounded) double-to-half conversion, which differs where the float lands exactly on a
// half-way point between two 16-bit values.
template <typename T>
__device__ __forceinline__ T rot_from_f64(double v) {
  float f = (float)v;
  if constexpr (sizeof(T) == 4) {
    return f;
  } else {
    asm volatile("" : "+v"(f));
    return (T)f;
  }
}

// (x1, x2) turned by the angle whose cos and sin (already in T) are c and s: x1 c - x2 s and
// x1 s + x2 c with every operation rounded to T (no contraction into FMAs)
template <typename T>
__device__ __forceinline__ void rot_pair(T x1_, T x2_, T c, T s, T& y1, T& y2) {
#pragma clang fp contract(off)
  const float x1 = to_f32(x1_), x2 = to_f32(x2_), cf = to_f32(c), sf = to_f32(s);
  const float a = to_f32(from_f32<T>(x1 * cf)), b = to_f32(from_f32<T>(x2 * sf));
  const float e = to_f32(from_f32<T>(x1 * sf)), f = to_f32(from_f32<T>(x2 * cf));
  y1 = from_f32<T>(a - b);
  y2 = from_f32<T>(e + f);
}

}  // namespace vsp
