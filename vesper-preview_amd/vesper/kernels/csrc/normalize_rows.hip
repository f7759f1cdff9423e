// normalize_keys on rows of any width (reference vesper/recurrence.py:91-115) on CDNA4 (gfx950),
// with its gradient. The key kernels (keys.hip) normalize heads up to 512 wide inside the key
// filter; this is the standalone row form for any width, up to the reference's own 65536-wide
// rows (tests/test_recurrence_review.py:61-64).
//
// Per row: s = u / max(max_j |u_j|, 1e-6) (a correctly rounded division: reciprocal refined by one
// Newton step on the FMA residual, so the peak component scales to exactly 1), then
// y = s / sqrt(max(sum_j s_j^2, 1)) in float32, returned in the input's dtype. Under autograd the
// peak is a constant (recurrence.py:103-105): with n2 = sum s^2 and g the output's gradient,
//   dx = (g / d - s (s . g) / d^3) / peak   where n2 >= 1 (d = sqrt(n2)),
//   dx = g / peak                             where the norm is floored at one (n2 < 1)
// (torch's clamp passes the gradient at n2 == 1, where both forms agree on d = 1 but the first
// keeps its s (s . g) term, as here).
// One wave per row, lanes striding over it: HBM-bound streaming (the row is read twice, three
// times for the gradient, mostly from L2 for wide rows), wave reductions by DPP and lane swaps in
// a fixed order, so results repeat bitwise.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr float kFloor = 1e-6f;  // normalize_keys' floor (vesper/recurrence.py:31)

__device__ __forceinline__ float scaled(float u, float peak, float inv_peak) {
  const float s0 = u * inv_peak;
  return __builtin_fmaf(__builtin_fmaf(-s0, peak, u), inv_peak, s0);
}

template <typename T>
__device__ __forceinline__ float row_peak(const T* x, int width, int l) {
  float peak = 0.f;
  for (int e = l; e < width; e += 64) peak = __builtin_fmaxf(peak, fabsf(to_f32(x[e])));
  return __builtin_fmaxf(group_max<64>(peak), kFloor);
}

template <typename T>
__global__ __launch_bounds__(256) void normalize_rows_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows,
                                                             int width) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const int l = threadIdx.x & 63;
  const T* xr = x + row * width;
  T* yr = y + row * width;
  const float peak = row_peak(xr, width, l), inv_peak = __builtin_amdgcn_rcpf(peak);
  float ss = 0.f;
  for (int e = l; e < width; e += 64) {
    const float s = scaled(to_f32(xr[e]), peak, inv_peak);
    ss = __builtin_fmaf(s, s, ss);
  }
  const float inv_den = __builtin_amdgcn_rsqf(__builtin_fmaxf(group_sum<64>(ss), 1.f));
  for (int e = l; e < width; e += 64) yr[e] = from_f32<T>(scaled(to_f32(xr[e]), peak, inv_peak) * inv_den);
}

template <typename T>
__global__ __launch_bounds__(256) void normalize_rows_backward_kernel(const T* __restrict__ x, const T* __restrict__ gy,
                                                                      T* __restrict__ gx, int64_t rows, int width) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int l = threadIdx.x & 63;
  const T* xr = x + row * width;
  const T* gr = gy + row * width;
  T* out = gx + row * width;
  const float peak = row_peak(xr, width, l), inv_peak = __builtin_amdgcn_rcpf(peak);
  float ss = 0.f, sg = 0.f;
  for (int e = l; e < width; e += 64) {
    const float s = scaled(to_f32(xr[e]), peak, inv_peak);
    ss = __builtin_fmaf(s, s, ss);
    sg = __builtin_fmaf(s, to_f32(gr[e]), sg);
  }
  const float n2 = group_sum<64>(ss), dot = group_sum<64>(sg);
  const bool floored = n2 < 1.f;
  const float inv_den = floored ? 1.f : __builtin_amdgcn_rsqf(n2);
  const float c = floored ? 0.f : dot * inv_den * inv_den * inv_den;
  for (int e = l; e < width; e += 64) {
    const float s = scaled(to_f32(xr[e]), peak, inv_peak);
    out[e] = from_f32<T>((to_f32(gr[e]) * inv_den - s * c) * inv_peak);
  }
}

template <typename T>
int normalize_rows(const T* x, T* y, int64_t rows, int width, void* stream, const char* who) {
  if (rows < 0 || width < 0) return fail(ERR_ARG, "%s: bad sizes rows=%lld width=%d", who, (long long)rows, width);
  if (rows == 0 || width == 0) return OK;
  if (!x || !y) return fail(ERR_ARG, "%s: null pointer", who);
  if ((rows + 3) / 4 > 0x7FFFFFFF) return fail(ERR_UNSUPPORTED, "%s: %lld rows", who, (long long)rows);
  hipLaunchKernelGGL(normalize_rows_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), x, y, rows, width);
  return check_launch(who);
}

template <typename T>
int normalize_rows_backward(const T* x, const T* gy, T* gx, int64_t rows, int width, void* stream, const char* who) {
  if (rows < 0 || width < 0) return fail(ERR_ARG, "%s: bad sizes rows=%lld width=%d", who, (long long)rows, width);
  if (rows == 0 || width == 0) return OK;
  if (!x || !gy || !gx) return fail(ERR_ARG, "%s: null pointer", who);
  if ((rows + 3) / 4 > 0x7FFFFFFF) return fail(ERR_UNSUPPORTED, "%s: %lld rows", who, (long long)rows);
  hipLaunchKernelGGL(normalize_rows_backward_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), x, gy, gx, rows, width);
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_normalize_keys_bf16(const void* x, void* y, int64_t rows, int width, void* stream) {
  return vsp::normalize_rows(static_cast<const __bf16*>(x), static_cast<__bf16*>(y), rows, width, stream,
                             "vsp_normalize_keys_bf16");
}
extern "C" int vsp_normalize_keys_f16(const void* x, void* y, int64_t rows, int width, void* stream) {
  return vsp::normalize_rows(static_cast<const _Float16*>(x), static_cast<_Float16*>(y), rows, width, stream,
                             "vsp_normalize_keys_f16");
}
extern "C" int vsp_normalize_keys_f32(const float* x, float* y, int64_t rows, int width, void* stream) {
  return vsp::normalize_rows(x, y, rows, width, stream, "vsp_normalize_keys_f32");
}
extern "C" int vsp_normalize_keys_backward_bf16(const void* x, const void* grad_y, void* grad_x, int64_t rows,
                                                int width, void* stream) {
  return vsp::normalize_rows_backward(static_cast<const __bf16*>(x), static_cast<const __bf16*>(grad_y),
                                      static_cast<__bf16*>(grad_x), rows, width, stream,
                                      "vsp_normalize_keys_backward_bf16");
}
extern "C" int vsp_normalize_keys_backward_f16(const void* x, const void* grad_y, void* grad_x, int64_t rows,
                                               int width, void* stream) {
  return vsp::normalize_rows_backward(static_cast<const _Float16*>(x), static_cast<const _Float16*>(grad_y),
                                      static_cast<_Float16*>(grad_x), rows, width, stream,
                                      "vsp_normalize_keys_backward_f16");
}
extern "C" int vsp_normalize_keys_backward_f32(const float* x, const float* grad_y, float* grad_x, int64_t rows,
                                               int width, void* stream) {
  return vsp::normalize_rows_backward(x, grad_y, grad_x, rows, width, stream, "vsp_normalize_keys_backward_f32");
}
