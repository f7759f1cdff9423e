// The write strength on CDNA4 (gfx950): beta from the write-strength logits and the modulator.
//
// Reference: vesper/recurrence.py:34-88 (`write_strength`): beta = sigmoid(logits) without a
// modulator; with the per-token modulator m and strength alpha, the write odds scaled by
// 1 + alpha m: beta = sigmoid(logits + ln(1 + alpha m)), exactly 0 where 1 + alpha m is 0. The
// arithmetic is write_strength() of common.h, the same function the scan's loads apply when it is
// given logits (vsp_delta_scan_logits_*): elementwise, one thread per (token, head).
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void write_strength_kernel(const T* __restrict__ logits, const float* __restrict__ m,
                                                             float alpha, T* __restrict__ beta, size_t total, int H) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  beta[i] = from_f32<T>(write_strength(to_f32(logits[i]), m, i / (size_t)H, alpha));
}

template <typename T>
int run(const T* logits, const float* m, float alpha, T* beta, int rows, int H, void* stream, const char* who) {
  if (rows < 0 || H < 1) return fail(ERR_ARG, "%s: rows %d, heads %d", who, rows, H);
  if (!(alpha >= 0.f) || alpha == __builtin_inff())
    return fail(ERR_ARG, "%s: alpha %g is not finite and non-negative", who, alpha);
  const size_t total = (size_t)rows * H;
  if (total == 0) return OK;
  if (!logits || !beta) return fail(ERR_ARG, "%s: null pointer", who);
  hipLaunchKernelGGL(write_strength_kernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), logits, m, alpha, beta, total, H);
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_write_strength_bf16(const void* logits, const float* m, float alpha, void* beta, int rows, int H,
                                       void* stream) {
  return vsp::run<__bf16>(static_cast<const __bf16*>(logits), m, alpha, static_cast<__bf16*>(beta), rows, H, stream,
                          "vsp_write_strength_bf16");
}

extern "C" int vsp_write_strength_f32(const float* logits, const float* m, float alpha, float* beta, int rows, int H,
                                      void* stream) {
  return vsp::run<float>(logits, m, alpha, beta, rows, H, stream, "vsp_write_strength_f32");
}
