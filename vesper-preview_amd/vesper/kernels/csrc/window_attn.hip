// Sliding-window causal attention on CDNA4 (gfx950): the prefill kernel.
//
// Semantics (reference vesper/kernels/window_attn.py:27-39): q [B, N, H, D] against keys, values
// [B, M + N, HKV, D] whose first M rows are the cache; query i sits at key index M + i and attends
// key indices [M + i - W + 1, M + i]; scale 1/sqrt(D); query head h reads KV head h / (H / HKV).
//
// One workgroup = 64 queries of one (b, h), four waves of 16 queries. Key tiles of 64 rows walk the
// window: K is staged row-major in LDS, V transposed ([d][key]). Each wave computes the score tile
// transposed, S^T = K Q^T (16x16x32 MFMA, Q held in registers as the B operand), so a lane holds
// one query's scores for 16 keys; the online softmax (running max, exp2, running sum) then needs
// only a 4-lane reduction, and the probabilities are already laid out as the B operand of
// O^T += V^T P^T. The next key tile is prefetched into registers while the current one is used.
#include "common.h"
#include "vesper_kernels.h"

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

template <typename T, int D>
__global__ __launch_bounds__(256) void window_attn_kernel(const T* __restrict__ q, const T* __restrict__ keys,
                                                          const T* __restrict__ values, T* __restrict__ o,
                                                          const uint8_t* __restrict__ active, int N, int M, int H,
                                                          int HKV, int W, float scale_log2, int nqt) {
  using V8 = typename Mma<T>::V8;
  using V4 = typename Mma<T>::V4;
  constexpr int DP = D < 32 ? 32 : D;  // feature extent padded to the MFMA k step
  constexpr int PK = DP + 8;           // LDS pitch of K rows
  constexpr int PV = 64 + 8;           // LDS pitch of V^T rows
  constexpr int DT = DP / 16;          // 16-row tiles of O^T
  constexpr int KSQ = DP / 32;         // k steps over features
  constexpr int SEG = DP / 8;          // 16-byte segments per key row
  constexpr int LOADS = (64 * SEG + 255) / 256;
  __shared__ __align__(16) T sK[64 * PK];
  __shared__ __align__(16) T sVt[DP * PV];

  const int lg = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qt = lg % nqt, bh = lg / nqt;
  const int b = bh / H, h = bh - b * H;
  const int kvh = h / (H / HKV);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lq = l & 15, g = l >> 4;
  const int S = M + N;
  const int qbase = qt * 64;
  const int myq = qbase + 16 * w + lq;
  const bool qok = myq < N;
  const bool act = qok && (active == nullptr || active[(size_t)b * N + myq] != 0);
  T* dst = o + (((size_t)b * N + (qok ? myq : 0)) * H + h) * D;

  if (!__syncthreads_or(act)) {  // every query of the tile is inactive (or past N): zeros
    if (qok && g == 0)
      for (int d = 0; d < D; ++d) dst[d] = from_f32<T>(0.f);
    return;
  }

  V8 qf[KSQ];
#pragma unroll
  for (int s = 0; s < KSQ; ++s) {
    const int f = 32 * s + 8 * g;
    if (qok && f < D) {
      qf[s] = *reinterpret_cast<const V8*>(q + (((size_t)b * N + myq) * H + h) * D + f);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[s][j] = from_f32<T>(0.f);
    }
  }

  const int kfirst = max(0, M + qbase - W + 1);
  const int klast = min(S, M + qbase + 64);
  const int qidx = M + myq;
  const size_t kv_row = (size_t)HKV * D;
  const T* kbase = keys + ((size_t)b * S * HKV + kvh) * D;
  const T* vbase = values + ((size_t)b * S * HKV + kvh) * D;

  V8 kreg[LOADS], vreg[LOADS];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int seg = threadIdx.x + 256 * i;
      const int row = seg / SEG, part = seg - row * SEG;
      const int key = k0 + row;
      const bool ok = seg < 64 * SEG && key < klast && 8 * part < D;
      if (ok) {
        kreg[i] = *reinterpret_cast<const V8*>(kbase + (size_t)key * kv_row + 8 * part);
        vreg[i] = *reinterpret_cast<const V8*>(vbase + (size_t)key * kv_row + 8 * part);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          kreg[i][j] = from_f32<T>(0.f);
          vreg[i][j] = from_f32<T>(0.f);
        }
      }
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int seg = threadIdx.x + 256 * i;
      if (seg < 64 * SEG) {
        const int row = seg / SEG, part = seg - row * SEG;
        *reinterpret_cast<V8*>(sK + row * PK + 8 * part) = kreg[i];
#pragma unroll
        for (int j = 0; j < 8; ++j) sVt[(8 * part + j) * PV + row] = vreg[i][j];
      }
    }
  };

  float m_run = -1e30f, l_run = 0.f;
  f32x4 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = zero4();

  fetch(kfirst);
  for (int k0 = kfirst; k0 < klast; k0 += 64) {
    __syncthreads();
    stash();
    __syncthreads();
    if (k0 + 64 < klast) fetch(k0 + 64);

    float s[4][4];
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 acc = zero4();
#pragma unroll
      for (int st = 0; st < KSQ; ++st) {
        const V8 a = *reinterpret_cast<const V8*>(sK + (16 * kb + lq) * PK + 32 * st + 8 * g);
        acc = Mma<T>::run(a, qf[st], acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 16 * kb + 4 * g + r;
        const bool vis = key < klast && key <= qidx && key > qidx - W;
        s[kb][r] = vis ? acc[r] * scale_log2 : -INFINITY;
        mt = fmaxf(mt, s[kb][r]);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2f(s[kb][r] - m_new);
        s[kb][r] = p;
        psum += p;
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] *= alpha;

#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      V8 pb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pb[j] = from_f32<T>(s[2 * ks][j]);
        pb[4 + j] = from_f32<T>(s[2 * ks + 1][j]);
      }
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const T* row = sVt + (16 * t + lq) * PV + 32 * ks + 4 * g;
        const V4 lo = *reinterpret_cast<const V4*>(row);
        const V4 hi = *reinterpret_cast<const V4*>(row + 16);
        V8 a;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a[j] = lo[j];
          a[4 + j] = hi[j];
        }
        oacc[t] = Mma<T>::run(a, pb, oacc[t]);
      }
    }
  }

  float lt = l_run + __shfl_xor(l_run, 16);
  lt += __shfl_xor(lt, 32);
  const float inv = (act && lt > 0.f) ? 1.f / lt : 0.f;
  if (qok) {
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * t + 4 * g + r;
        if (d < D) dst[d] = from_f32<T>(oacc[t][r] * inv);
      }
  }
}

bool attn_width(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }

template <typename T>
int window_attn(const T* q, const T* keys, const T* values, T* o, const uint8_t* active, int B, int N, int M, int H,
                int HKV, int D, int W, float scale, void* stream_ptr, const char* who) {
  if (B < 0 || N < 0 || M < 0 || H < 1 || HKV < 1) return fail(ERR_ARG, "%s: bad sizes B=%d N=%d M=%d H=%d HKV=%d", who, B, N, M, H, HKV);
  if (H % HKV != 0) return fail(ERR_ARG, "%s: %d query heads are not a multiple of %d KV heads", who, H, HKV);
  if (W < 1) return fail(ERR_ARG, "%s: window must be at least 1, got %d", who, W);
  if (!attn_width(D)) return fail(ERR_UNSUPPORTED, "%s: head dimension %d (kernels: 16, 32, 64, 128)", who, D);
  if (B == 0 || N == 0) return OK;
  if (!q || !keys || !values || !o) return fail(ERR_ARG, "%s: null pointer", who);
  const float scale_log2 = scale * 1.4426950408889634f;
  const int nqt = (N + 63) / 64;
  dim3 grid((unsigned)((size_t)nqt * H * B));
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  switch (D) {
    case 16: hipLaunchKernelGGL((window_attn_kernel<T, 16>), grid, dim3(256), 0, stream, q, keys, values, o, active, N, M, H, HKV, W, scale_log2, nqt); break;
    case 32: hipLaunchKernelGGL((window_attn_kernel<T, 32>), grid, dim3(256), 0, stream, q, keys, values, o, active, N, M, H, HKV, W, scale_log2, nqt); break;
    case 64: hipLaunchKernelGGL((window_attn_kernel<T, 64>), grid, dim3(256), 0, stream, q, keys, values, o, active, N, M, H, HKV, W, scale_log2, nqt); break;
    default: hipLaunchKernelGGL((window_attn_kernel<T, 128>), grid, dim3(256), 0, stream, q, keys, values, o, active, N, M, H, HKV, W, scale_log2, nqt); break;
  }
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_window_attn_bf16(const void* q, const void* keys, const void* values, void* o, const uint8_t* active,
                                    int B, int N, int M, int H, int HKV, int D, int window, float scale, void* stream) {
  return vsp::window_attn<__bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(keys),
                                  static_cast<const __bf16*>(values), static_cast<__bf16*>(o), active, B, N, M, H, HKV,
                                  D, window, scale, stream, "vsp_window_attn_bf16");
}

extern "C" int vsp_window_attn_f16(const void* q, const void* keys, const void* values, void* o, const uint8_t* active,
                                   int B, int N, int M, int H, int HKV, int D, int window, float scale, void* stream) {
  return vsp::window_attn<_Float16>(static_cast<const _Float16*>(q), static_cast<const _Float16*>(keys),
                                    static_cast<const _Float16*>(values), static_cast<_Float16*>(o), active, B, N, M,
                                    H, HKV, D, window, scale, stream, "vsp_window_attn_f16");
}
