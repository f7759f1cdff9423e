// The key filter's backward on CDNA4 (gfx950): the kernel template and its host launch, included
// by one translation unit per dtype (keys_backward_{bf16,f16,f32}.hip) so they build in parallel;
// the taps' partial sums and the empty case live in keys.hip.
#pragma once
#include "keys_rows.h"
#include "vesper_kernels.h"

namespace vsp {

// ---- the backward: d z, d taps, d history from the keys' gradient ---------------------------
// Per token and head (the normalization's peak held constant, as the reference detaches it):
//   s = u / peak, q = |s|^2, du = (g / sqrt(max(q, 1)) - [q >= 1] s (g . s) / max(q, 1)^1.5) / peak
// (vesper/kernels/keys_triton.py:87-94), then the filter transposed: dz[t] = sum_r taps[r] du[t + r],
// dtaps[r] = sum_t du[t] x[t - r], and history row p collects taps[r] du[t], t = p - (K - 1) + r
// (vesper/kernels/keys.py:66-78). One pass: a wave recomputes u and du for its run of tokens and
// the K - 1 after it (their du feeds its last dz), so z and the keys' gradient are read once and
// dz written once. The taps' gradient is summed per wave in registers, over the workgroup's waves
// through LDS, and over the workgroups by tap_sum_kernel in a fixed order: deterministic.

constexpr int kBackRun = 8;      // tokens per wave
constexpr int kBackWaves = 8;    // waves per workgroup: one taps partial per 64 tokens

size_t key_backward_parts(int B, int N);
size_t key_backward_workspace(int B, int N, int D, int K);
int key_backward_empty(float* grad_taps, float* grad_history, int B, int D, int K, hipStream_t stream, const char* who);
int key_backward_sum_taps(float* partial, float* grad_taps, int B, int N, int D, int K, hipStream_t stream,
                          const char* who);

namespace {

template <typename TZ, int K, int LPH>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2))) void key_filter_backward_kernel(
    const TZ* __restrict__ z, const float* __restrict__ history, const float* __restrict__ taps,
    const TZ* __restrict__ grad_k, TZ* __restrict__ grad_z, float* __restrict__ partial,
    float* __restrict__ grad_history, int N, int D) {
  using Row = Row8<TZ>;
  constexpr int RUN = kBackRun;
  static_assert(RUN >= K - 1, "a run is at least as long as the filter's history");
  constexpr int NG = RUN + K - 1;  // tokens t0 .. t0 + NG - 1 whose du the run needs
  __shared__ float hand[kBackWaves / 2][K][64 * 8];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
  const int b = blockIdx.z;
  const int f0 = 8 * (64 * blockIdx.x + l);
  const bool on = f0 < D;
  // a run past N (the last workgroup) reads zeros and stores nothing, but joins the barriers
  const int t0 = RUN * (kBackWaves * blockIdx.y + wave);
  const int last = N - 1;
  const unsigned row_bytes = (unsigned)D * sizeof(TZ);
  const unsigned batch_bytes = (unsigned)N * row_bytes;  // below 2^31: the host refuses more
  const auto rz = buffer_rsrc(z + (size_t)b * N * D, batch_bytes);
  const auto rg = buffer_rsrc(grad_k + (size_t)b * N * D, batch_bytes);
  const auto ro = buffer_rsrc(grad_z + (size_t)b * N * D, batch_bytes);
  constexpr unsigned kPast = 0x80000000u;
  const unsigned voff = on ? (unsigned)f0 * sizeof(TZ) : kPast;
  const int fl = on ? f0 : 0;

  float tp[K][8];
#pragma unroll
  for (int r = 0; r < K; ++r) {
    const f32x4 t0v = *reinterpret_cast<const f32x4*>(taps + (size_t)r * D + fl);
    const f32x4 t1v = *reinterpret_cast<const f32x4*>(taps + (size_t)r * D + fl + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tp[r][e] = t0v[e];
      tp[r][4 + e] = t1v[e];
    }
  }
  // the K - 1 input rows before the run: from z, or for a batch row's first run from the history
  // (both loaded, the unused one from past its range, joined bitwise)
  float halo[K > 1 ? K - 1 : 1][8];  // halo[q] = input row t0 - (K - 1) + q
  if constexpr (K > 1) {
    const bool first = t0 == 0;
    const auto rh = buffer_rsrc(history + (size_t)b * (K - 1) * D, (unsigned)(K - 1) * D * 4u);
    const unsigned vz = first ? kPast : voff;
    const unsigned vh = (first && on) ? (unsigned)f0 * 4u : kPast;
#pragma unroll
    for (int q = 0; q < K - 1; ++q) {
      float zr[8], hr[8];
      Row::unpack(Row::load(rz, vz, first ? 0u : (unsigned)min(t0 - (K - 1) + q, last) * row_bytes), zr);
      Row8<float>::unpack(Row8<float>::load(rh, vh, (unsigned)q * D * 4u), hr);
#pragma unroll
      for (int e = 0; e < 8; ++e) halo[q][e] = __uint_as_float(__float_as_uint(zr[e]) | __float_as_uint(hr[e]));
    }
  }
  // the run's input rows and the keys' gradient rows t0 .. t0 + NG - 1 (gradient past N: zeros)
  typename Row::Raw xr[NG], gr[NG];
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const unsigned row = (unsigned)min(t0 + i, last) * row_bytes;
    xr[i] = Row::load(rz, voff, row);
    gr[i] = Row::load(rg, t0 + i < N ? voff : kPast, row);
  }

  float acc[K][8];
#pragma unroll
  for (int r = 0; r < K; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
  float xs[NG + K - 1][8];  // xs[q] = input row t0 - (K - 1) + q, unpacked once
#pragma unroll
  for (int q = 0; q < K - 1; ++q)
#pragma unroll
    for (int e = 0; e < 8; ++e) xs[q][e] = halo[q][e];
  float du[NG][8];

#pragma unroll
  for (int i = 0; i < NG; ++i) {
    Row::unpack(xr[i], xs[i + K - 1]);
    // u in the forward's order, then the normalization's gradient
    float u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = tp[0][e] * xs[i + K - 1][e];
#pragma unroll
      for (int r = 1; r < K; ++r) a = a + tp[r][e] * xs[i + K - 1 - r][e];
      u[e] = a;
    }
    float peak = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) peak = __builtin_fmaxf(peak, fabsf(u[e]));
    const float inv_scale = __builtin_amdgcn_rcpf(__builtin_fmaxf(group_max<LPH>(peak), kKeyFloor));
    float g[8];
    Row::unpack(gr[i], g);
    float ss = 0.f, gs = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      u[e] = u[e] * inv_scale;  // s
      ss += u[e] * u[e];
      gs += g[e] * u[e];
    }
    const float sq = group_sum<LPH>(ss);
    const float dot = group_sum<LPH>(gs);
    const float inv_den = __builtin_amdgcn_rsqf(__builtin_fmaxf(sq, 1.f));
    const float through = sq >= 1.f ? dot * (inv_den * inv_den * inv_den) : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) du[i][e] = (g[e] * inv_den - u[e] * through) * inv_scale;
    if (i < RUN) {  // the taps' gradient counts each token once: in the run that owns it
#pragma unroll
      for (int r = 0; r < K; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] += du[i][e] * xs[i + K - 1 - r][e];
    }
    if (K > 1 && i == K - 2 && grad_history != nullptr && t0 == 0 && on) {
      // history row p: taps[r] du[t] for t = p - (K - 1) + r in 0..p, r ascending
#pragma unroll
      for (int p = 0; p < K - 1; ++p) {
        float h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float a = tp[K - 1 - p][e] * du[0][e];
#pragma unroll
          for (int t = 1; t <= p; ++t) a = a + tp[K - 1 - p + t][e] * du[t][e];
          h[e] = a;
        }
        float* hp = grad_history + ((size_t)b * (K - 1) + p) * D + f0;
        *reinterpret_cast<f32x4*>(hp) = f32x4{h[0], h[1], h[2], h[3]};
        *reinterpret_cast<f32x4*>(hp + 4) = f32x4{h[4], h[5], h[6], h[7]};
      }
    }
    if (i >= K - 1) {  // dz of token t0 + t needs du[t .. t + K - 1], complete now
      const int t = i - (K - 1);
      float dz[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = tp[0][e] * du[t][e];
#pragma unroll
        for (int r = 1; r < K; ++r) a = a + tp[r][e] * du[t + r][e];
        dz[e] = a;
      }
      // row offset in the vector offset, soffset 0 (see the forward's store)
      Row::store(ro, (t0 + t < N ? voff : kPast) + (unsigned)min(t0 + t, last) * row_bytes, 0u, dz);
    }
  }

  // the taps' partial over the workgroup's waves: 4..7 into 0..3, 2..3 into 0..1, 1 into 0
#pragma unroll
  for (int half = kBackWaves / 2; half >= 1; half /= 2) {
    if (wave >= half && wave < 2 * half) {
#pragma unroll
      for (int r = 0; r < K; ++r) {
        float* hp = &hand[wave - half][r][8 * l];
        *reinterpret_cast<f32x4*>(hp) = f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
        *reinterpret_cast<f32x4*>(hp + 4) = f32x4{acc[r][4], acc[r][5], acc[r][6], acc[r][7]};
      }
    }
    __syncthreads();
    if (wave < half) {
#pragma unroll
      for (int r = 0; r < K; ++r) {
        const float* hp = &hand[wave][r][8 * l];
        const f32x4 a = *reinterpret_cast<const f32x4*>(hp), c = *reinterpret_cast<const f32x4*>(hp + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[r][e] += a[e];
          acc[r][4 + e] += c[e];
        }
      }
    }
    __syncthreads();
  }
  if (wave == 0 && on) {
    const size_t part = (size_t)blockIdx.z * gridDim.y + blockIdx.y;
#pragma unroll
    for (int r = 0; r < K; ++r) {
      float* pp = partial + (part * K + r) * D + f0;
      *reinterpret_cast<f32x4*>(pp) = f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
      *reinterpret_cast<f32x4*>(pp + 4) = f32x4{acc[r][4], acc[r][5], acc[r][6], acc[r][7]};
    }
  }
}

template <typename TZ, int K>
void launch_backward_k(const TZ* z, const float* history, const float* taps, const TZ* grad_k, TZ* grad_z, float* partial,
                       float* grad_history, int B, int N, int D, int hd, hipStream_t stream) {
  dim3 grid((unsigned)((D / 8 + 63) / 64), (unsigned)((N + kBackRun * kBackWaves - 1) / (kBackRun * kBackWaves)),
            (unsigned)B);
#define VSP_KB(L)                                                                                                    \
  hipLaunchKernelGGL((key_filter_backward_kernel<TZ, K, L>), grid, dim3(64 * kBackWaves), 0, stream, z, history, taps, \
                     grad_k, grad_z, partial, grad_history, N, D)
  switch (hd / 8) {
    case 1: VSP_KB(1); break;
    case 2: VSP_KB(2); break;
    case 4: VSP_KB(4); break;
    case 8: VSP_KB(8); break;
    case 16: VSP_KB(16); break;
    case 32: VSP_KB(32); break;
    default: VSP_KB(64); break;
  }
#undef VSP_KB
}

template <typename TZ>
int key_filter_backward(const TZ* z, const float* history, const float* taps, const TZ* grad_k, TZ* grad_z,
                        float* grad_taps, float* grad_history, void* workspace, size_t workspace_bytes, int B, int N,
                        int D, int heads, int K, void* stream_ptr, const char* who) {
  if (B < 0 || N < 0 || D < 1 || heads < 1) return fail(ERR_ARG, "%s: bad sizes B=%d N=%d D=%d heads=%d", who, B, N, D, heads);
  if (K < 1 || K > 8) return fail(ERR_UNSUPPORTED, "%s: filter width %d (kernels: 1..8)", who, K);
  if (D % heads != 0) return fail(ERR_ARG, "%s: %d features are not a multiple of %d heads", who, D, heads);
  const int hd = D / heads;
  if (hd < 8 || hd > 512 || (hd & (hd - 1)) != 0)
    return fail(ERR_UNSUPPORTED, "%s: head width %d (kernels: powers of two 8..512)", who, hd);
  if (!grad_taps) return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(grad_taps) | reinterpret_cast<uintptr_t>(grad_history)) & 15)
    return fail(ERR_ARG, "%s: the taps' and the history's gradients must be 16-byte aligned", who);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  if (B == 0 || N == 0) {  // no token: the taps' and the history's gradients are zero
    return key_backward_empty(grad_taps, grad_history, B, D, K, stream, who);
  }
  if (!z || !grad_k || !grad_z || !taps || (K > 1 && !history)) return fail(ERR_ARG, "%s: null pointer", who);
  if ((N + kBackRun * kBackWaves - 1) / (kBackRun * kBackWaves) > 65535 || B > 65535)
    return fail(ERR_UNSUPPORTED, "%s: %d tokens in %d batch rows exceed the launch grid", who, N, B);
  if ((size_t)N * D * sizeof(TZ) > 0x7FFFFFF0u)
    return fail(ERR_UNSUPPORTED, "%s: %d tokens of %d features exceed 2 GiB in one batch row", who, N, D);
  if ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(grad_k) | reinterpret_cast<uintptr_t>(grad_z) |
       reinterpret_cast<uintptr_t>(taps) | reinterpret_cast<uintptr_t>(history) |
       reinterpret_cast<uintptr_t>(workspace)) & 15)
    return fail(ERR_ARG, "%s: z, history, taps, the gradients and the workspace must be 16-byte aligned", who);
  const size_t need = key_backward_workspace(B, N, D, K);
  if (!workspace || workspace_bytes < need)
    return fail(ERR_ARG, "%s: workspace of %zu bytes, %zu needed", who, workspace_bytes, need);
  float* partial = static_cast<float*>(workspace);
  switch (K) {
    case 1: launch_backward_k<TZ, 1>(z, history, taps, grad_k, grad_z, partial, nullptr, B, N, D, hd, stream); break;
    case 2: launch_backward_k<TZ, 2>(z, history, taps, grad_k, grad_z, partial, grad_history, B, N, D, hd, stream); break;
    case 3: launch_backward_k<TZ, 3>(z, history, taps, grad_k, grad_z, partial, grad_history, B, N, D, hd, stream); break;
    case 4: launch_backward_k<TZ, 4>(z, history, taps, grad_k, grad_z, partial, grad_history, B, N, D, hd, stream); break;
    case 5: launch_backward_k<TZ, 5>(z, history, taps, grad_k, grad_z, partial, grad_history, B, N, D, hd, stream); break;
    case 6: launch_backward_k<TZ, 6>(z, history, taps, grad_k, grad_z, partial, grad_history, B, N, D, hd, stream); break;
    case 7: launch_backward_k<TZ, 7>(z, history, taps, grad_k, grad_z, partial, grad_history, B, N, D, hd, stream); break;
    default: launch_backward_k<TZ, 8>(z, history, taps, grad_k, grad_z, partial, grad_history, B, N, D, hd, stream); break;
  }
  return key_backward_sum_taps(partial, grad_taps, B, N, D, K, stream, who);
}

}  // namespace
}  // namespace vsp
