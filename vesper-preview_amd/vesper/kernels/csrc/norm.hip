// The column's sublayer pre-normalization on CDNA4 (gfx950): RMSNorm of float32 rows to bf16.
//
// Reference: vesper/column.py:146-188 (`RMSNorm.forward`): y = x / sqrt(mean(x^2) + 1e-6) * g,
// computed scale-safely: each row is first divided by its peak magnitude floored at 1e-3, and the
// root is taken of mean(s^2) + 1e-6 / scale^2, in float32. The looped column runs it on its float32
// residual stream before each sublayer's projections, whose bf16 operand this kernel writes
// directly (one launch in place of the norm's elementwise chain and the cast).
//
// With a residual (vsp_add_rms_norm_bf16) the row normalized is x + r (r in bf16, added in float32
// as the column's residual add does), and that sum is written to sum_out too: the add, its
// separate pass over memory and the norm's re-read become one launch.
//
// One wave per row: a lane holds the row's 8-float segments lane, lane + 64, ... (16-byte loads),
// the peak and the sum of squares are wave reductions (DPP and lane swaps), the division by the
// peak is a reciprocal refined by one Newton step (the correctly rounded quotient), and the row is
// written as 16-byte bf16 pieces.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr float kRmsEps = 1e-6f;         // column.py:55
constexpr float kRmsScaleFloor = 1e-3f;  // column.py:56

template <int NSEG>
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ gain,
                                                       __bf16* __restrict__ out, int rows, int d,
                                                       const __bf16* __restrict__ res = nullptr,
                                                       float* __restrict__ sum_out = nullptr) {
  const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;  // whole waves only: no barrier in this kernel
  const float* xr = x + (size_t)row * d;
  float v[NSEG][8];
  float peak = 0.f;
#pragma unroll
  for (int j = 0; j < NSEG; ++j) {
    const int f = 8 * (lane + 64 * j);
    const bool ok = f < d;
    const float4 a = reinterpret_cast<const float4*>(xr + (ok ? f : 0))[0];
    const float4 b = reinterpret_cast<const float4*>(xr + (ok ? f : 0))[1];
    float e[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if (res != nullptr) {
      const bf16x8 rv = *reinterpret_cast<const bf16x8*>(res + (size_t)row * d + (ok ? f : 0));
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] += (float)rv[i];
      if (ok && sum_out != nullptr) {
        float* so = sum_out + (size_t)row * d + f;
        reinterpret_cast<float4*>(so)[0] = make_float4(e[0], e[1], e[2], e[3]);
        reinterpret_cast<float4*>(so)[1] = make_float4(e[4], e[5], e[6], e[7]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[j][i] = ok ? e[i] : 0.f;
      peak = __builtin_fmaxf(peak, fabsf(v[j][i]));
    }
  }
  const float scale = __builtin_fmaxf(group_max<64>(peak), kRmsScaleFloor);
  const float inv_scale = __builtin_amdgcn_rcpf(scale);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NSEG; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s0 = v[j][i] * inv_scale;
      v[j][i] = __builtin_fmaf(__builtin_fmaf(-s0, scale, v[j][i]), inv_scale, s0);
      ss += v[j][i] * v[j][i];
    }
  const float mean = group_sum<64>(ss) / (float)d;
  const float inv_rms = 1.f / __builtin_sqrtf(mean + kRmsEps / (scale * scale));
  __bf16* orow = out + (size_t)row * d;
#pragma unroll
  for (int j = 0; j < NSEG; ++j) {
    const int f = 8 * (lane + 64 * j);
    if (f >= d) continue;
    bf16x8 o;
    if (gain != nullptr) {
      const float4 ga = reinterpret_cast<const float4*>(gain + f)[0];
      const float4 gb = reinterpret_cast<const float4*>(gain + f)[1];
      const float g[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (__bf16)(v[j][i] * inv_rms * g[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (__bf16)(v[j][i] * inv_rms);
    }
    *reinterpret_cast<bf16x8*>(orow + f) = o;
  }
}

}  // namespace
}  // namespace vsp

namespace vsp {
namespace {
int rms_norm(const float* x, const __bf16* res, float* sum_out, const float* gain, void* out, int rows, int d,
             void* stream, const char* who) {
  if (rows < 0 || d < 8 || d > 2048 || d % 8 != 0)
    return fail(ERR_ARG, "%s: rows %d, width %d (a multiple of 8 in 8..2048)", who, rows, d);
  if (rows == 0) return OK;
  if (!x || !out) return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(gain) |
       reinterpret_cast<uintptr_t>(res) | reinterpret_cast<uintptr_t>(sum_out)) & 15)
    return fail(ERR_ARG, "%s: x, the residual, the sum, gain and out must be 16-byte aligned", who);
  const dim3 grid((unsigned)((rows + 3) / 4));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  __bf16* o = static_cast<__bf16*>(out);
  if (d <= 512) hipLaunchKernelGGL(rms_norm_kernel<1>, grid, dim3(256), 0, s, x, gain, o, rows, d, res, sum_out);
  else if (d <= 1024) hipLaunchKernelGGL(rms_norm_kernel<2>, grid, dim3(256), 0, s, x, gain, o, rows, d, res, sum_out);
  else hipLaunchKernelGGL(rms_norm_kernel<4>, grid, dim3(256), 0, s, x, gain, o, rows, d, res, sum_out);
  return check_launch(who);
}
}  // namespace
}  // namespace vsp

extern "C" int vsp_rms_norm_bf16(const float* x, const float* gain, void* out, int rows, int d, void* stream) {
  return vsp::rms_norm(x, nullptr, nullptr, gain, out, rows, d, stream, "vsp_rms_norm_bf16");
}

extern "C" int vsp_add_rms_norm_bf16(const float* x, const void* residual, float* sum_out, const float* gain, void* out,
                                     int rows, int d, void* stream) {
  if (residual == nullptr)
    return vsp::fail(vsp::ERR_ARG, "vsp_add_rms_norm_bf16: null residual");
  return vsp::rms_norm(x, static_cast<const __bf16*>(residual), sum_out, gain, out, rows, d, stream,
                       "vsp_add_rms_norm_bf16");
}
