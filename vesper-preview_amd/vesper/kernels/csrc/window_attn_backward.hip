// Sliding-window causal attention on CDNA4 (gfx950): the gradients.
//
// The backward of the prefill kernel (window_attn.hip; reference vesper/kernels/window_attn.py:27-39,
// run by autograd through WindowedAttention.attend, vesper/attention.py:373-383). With the
// forward's log-sum-exp `lse` (log2 units of the scaled scores), P = exp2(s * scale_log2 - lse),
// and per query Dsum = sum_d dO O:
//   dP = dO V^T,  dS = P (dP - Dsum) scale,  dQ = dS K,  dK = dS^T Q,  dV = P^T dO,
// dK and dV summed over the query heads that share the KV head. An inactive query's lse is +inf
// (the forward writes it so): its P, and every gradient through it, is exactly zero.
//
// Two kernels and no atomics, so the gradients repeat bitwise:
// - attn_dq_kernel, one workgroup per (b, h, 16 NW queries), a wave per 16 queries in registers,
//   walks the window's 64-key tiles through LDS: S^T = K Q^T and dP^T = V dO^T (16x16x32 MFMA, a
//   lane holding 16 keys of one query, as the forward), dS^T elementwise, dQ^T += K^T dS^T with
//   K^T fragments from transposed LDS reads; it also writes Dsum for the second kernel.
// - attn_dkv_kernel, one workgroup per (b, KV head, 16 NW keys), a wave per 16 keys in registers,
//   walks the query heads of the group and the 64-query tiles that see its keys: S = Q K^T and
//   dP = dO V^T (a lane holding 16 queries of one key), dV^T += dO^T P and dK^T += Q^T dS with dO^T
//   and Q^T fragments from transposed LDS reads.
// Both launch 8 waves a workgroup: a staged tile then serves 128 queries (keys), against 64 at 4
// waves, which cuts the window's overlap re-fetch about in half (dq 69.7 -> 62.0 us, dkv 97.2 ->
// 86.5 us at B4 T4096 H8 d64 w512); 16 waves measured slower for both.
#include "attn_mma.h"
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

template <int D> struct BwdShape {
  static constexpr int DP = D < 32 ? 32 : D;  // feature extent padded to the MFMA k step
  static constexpr int KSQ = DP / 32;         // MFMA k steps over the features
  static constexpr int DT = DP / 16;          // 16-row tiles of a transposed [features x 16] result
  static constexpr int SEG = DP / 8;          // 16-byte segments per row
  static constexpr int P = DP + 16;           // LDS pitch (elements) for row and transposed reads
};

// Rows r0 .. r0 + 63 of a [rows, ld]-strided tensor (features 0 .. D - 1) staged into LDS [64][P],
// zero past D and past row `rows`, in two steps: fetch() issues the loads into registers and put()
// writes them to LDS, so the next tile's loads are in flight while the current one is used. Loads
// are unconditional (rows past the end re-read the last row, padding features feature 0) and the
// zeros selected in put(): a load behind a per-lane branch would wait for every earlier one.
template <typename T, int D, int NTH = 256>
struct Stage64 {
  using Sh = BwdShape<D>;
  using V8 = typename Mma<T>::V8;
  static constexpr int kSegs = 64 * Sh::SEG, kIt = (kSegs + NTH - 1) / NTH;
  V8 raw[kIt];
  int r0, rows;
  __device__ __forceinline__ void fetch(const T* src, size_t ld, int first, int nrows) {
    r0 = first;
    rows = nrows;
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int sg = min((int)threadIdx.x + NTH * it, kSegs - 1), row = sg / Sh::SEG, part = sg - row * Sh::SEG;
      raw[it] = *reinterpret_cast<const V8*>(src + (size_t)min(r0 + row, rows - 1) * ld + (8 * part < D ? 8 * part : 0));
    }
  }
  __device__ __forceinline__ void put(T* dst) const {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int sg = threadIdx.x + NTH * it, row = sg / Sh::SEG, part = sg - row * Sh::SEG;
      const bool ok = r0 + row < rows && 8 * part < D;
      // the zeros selected as four 32-bit words (the 16 bytes as one unit, not eight elements)
      const uint4 x = __builtin_bit_cast(uint4, raw[it]);
      const uint4 v = {ok ? x.x : 0u, ok ? x.y : 0u, ok ? x.z : 0u, ok ? x.w : 0u};
      if (kSegs % NTH == 0 || sg < kSegs) *reinterpret_cast<uint4*>(dst + row * Sh::P + 8 * part) = v;
    }
  }
};

// A fragment of rows rbase + lq, features 32 s + 8 g .. + 7 (row-major LDS tile).
template <typename T, int D>
__device__ __forceinline__ typename Mma<T>::V8 row_frag(const T* tile, int rbase, int s) {
  const int l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  return *reinterpret_cast<const typename Mma<T>::V8*>(tile + (rbase + lq) * BwdShape<D>::P + 32 * s + 8 * g);
}

// The transposed A fragment: lane (lq, g) gets column 16 t + lq of rows r0 + 4 g .. + 3 and
// r0 + 16 + 4 g .. + 3 (the k order the accumulator-built B fragments use).
template <typename T, int D>
__device__ __forceinline__ typename Mma<T>::V8 tr_frag(const T* tile, int r0, int t) {
  constexpr int P = BwdShape<D>::P;
  const int l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  const T* base = tile + (r0 + 4 * g + (lq >> 2)) * P + 16 * t + 4 * (lq & 3);
  const auto lo = read_tr<T>(base);
  const auto hi = read_tr<T>(base + 16 * P);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW) void attn_dq_kernel(const T* __restrict__ q, const T* __restrict__ keys,
                                                      const T* __restrict__ values, const T* __restrict__ o,
                                                      const T* __restrict__ dout, const float* __restrict__ lse,
                                                      float* __restrict__ dsum, T* __restrict__ dq, int N, int M,
                                                      int H, int HKV, int W, float scale, float scale_log2, int nqt) {
  using Sh = BwdShape<D>;
  using V8 = typename Mma<T>::V8;
  using V4 = typename Mma<T>::V4;
  constexpr int KT = 64;
  __shared__ __align__(16) T sK[2][KT * Sh::P];
  __shared__ __align__(16) T sV[2][KT * Sh::P];
  // consecutive query tiles of a head on one XCD: their key windows overlap, so most of each
  // tile's K and V reads hit that XCD's L2
  const int lg = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qt = lg % nqt, bh = lg / nqt;
  const int b = bh / H, h = bh - b * H;
  const int kvh = h / (H / HKV);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lq = l & 15, g = l >> 4;
  const int S = M + N;
  const int i = 16 * NW * qt + 16 * w + lq;  // this lane's query
  const bool qok = i < N;
  const size_t qrow = (((size_t)b * N + (qok ? i : 0)) * H + h) * D;

  // the query's Q and dO as B fragments (lane (lq, g): features 32 s + 8 g .. + 7), and Dsum
  V8 qf[Sh::KSQ], df[Sh::KSQ];
  float part = 0.f;
#pragma unroll
  for (int s = 0; s < Sh::KSQ; ++s) {
    const int f = 32 * s + 8 * g;
    if (qok && f < D) {
      qf[s] = *reinterpret_cast<const V8*>(q + qrow + f);
      df[s] = *reinterpret_cast<const V8*>(dout + qrow + f);
      const V8 of = *reinterpret_cast<const V8*>(o + qrow + f);
#pragma unroll
      for (int e = 0; e < 8; ++e) part += to_f32(df[s][e]) * to_f32(of[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qf[s][e] = from_f32<T>(0.f);
        df[s][e] = from_f32<T>(0.f);
      }
    }
  }
  float dsm = part + __shfl_xor(part, 16);
  dsm += __shfl_xor(dsm, 32);
  const float lq_lse = qok ? lse[((size_t)b * H + h) * N + i] : INFINITY;
  if (qok && g == 0) dsum[((size_t)b * H + h) * N + i] = dsm;

  const int qlo = 16 * NW * qt;
  const int kfirst = max(0, M + qlo - W + 1), klast = min(S, M + qlo + 16 * NW);
  const int ntiles = (klast - kfirst + KT - 1) / KT;
  const size_t kv_ld = (size_t)HKV * D;
  const T* kbase = keys + ((size_t)b * S * HKV + kvh) * D;
  const T* vbase = values + ((size_t)b * S * HKV + kvh) * D;
  const int qk = M + i;  // the query's index among the keys
  const int wlo = M + qlo + 16 * w, whi = wlo + 15;

  f32x4 acc[Sh::DT];
#pragma unroll
  for (int t = 0; t < Sh::DT; ++t) acc[t] = zero4();
  // double-buffered key tiles: tile it + 1 is fetched into registers while tile it is used, then
  // written to the other buffer (last read before the previous barrier): one barrier per tile
  Stage64<T, D, 64 * NW> fk, fv;
  if (ntiles > 0) {
    fk.fetch(kbase, kv_ld, kfirst, S);
    fv.fetch(vbase, kv_ld, kfirst, S);
    fk.put(sK[0]);
    fv.put(sV[0]);
  }
  __syncthreads();
  for (int it = 0; it < ntiles; ++it) {
    const int k0 = kfirst + it * KT;
    const T* tK = sK[it & 1];
    const T* tV = sV[it & 1];
    if (it + 1 < ntiles) {
      fk.fetch(kbase, kv_ld, k0 + KT, S);
      fv.fetch(vbase, kv_ld, k0 + KT, S);
    }
    if (k0 <= whi && k0 + KT - 1 > wlo - W) {  // some query of the wave sees this tile
    // every key of the tile visible to every query of the wave: no masks (an inactive query's
    // or a query past N has lse +inf, so its P is 0 without one)
    const bool full = k0 + KT - 1 <= wlo && k0 > whi - W;
    f32x4 sacc[4], pacc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      sacc[kb] = zero4();
      pacc[kb] = zero4();
#pragma unroll
      for (int st = 0; st < Sh::KSQ; ++st) {
        sacc[kb] = Mma<T>::run(row_frag<T, D>(tK, 16 * kb, st), qf[st], sacc[kb]);
        pacc[kb] = Mma<T>::run(row_frag<T, D>(tV, 16 * kb, st), df[st], pacc[kb]);
      }
    }
    // lane (lq, g) holds keys k0 + 16 kb + 4 g + r of its query; dS without the scale (applied to
    // dQ at the end)
    float p[4][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) p[kb][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r], scale_log2, -lq_lse));
    if (!full) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) p[kb][r] = (unsigned)(qk - (k0 + 16 * kb + 4 * g + r)) < (unsigned)W ? p[kb][r] : 0.f;
    }
    V8 dsb[2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) dsb[kb >> 1][4 * (kb & 1) + r] = from_f32<T>(p[kb][r] * (pacc[kb][r] - dsm));
#pragma unroll
    for (int t = 0; t < Sh::DT; ++t)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) acc[t] = Mma<T>::run(tr_frag<T, D>(tK, 32 * ks, t), dsb[ks], acc[t]);
    }
    if (it + 1 < ntiles) {
      fk.put(sK[(it + 1) & 1]);
      fv.put(sV[(it + 1) & 1]);
    }
    __syncthreads();
  }
  if (qok) {
#pragma unroll
    for (int t = 0; t < Sh::DT; ++t) {
      const int d = 16 * t + 4 * g;
      if (d < D) {
        V4 v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = from_f32<T>(acc[t][r] * scale);
        *reinterpret_cast<V4*>(dq + qrow + d) = v;
      }
    }
  }
}

template <typename T, int D, int NW, int WAVES_PER_SIMD, int KB>
__global__ __launch_bounds__(64 * NW, WAVES_PER_SIMD) void attn_dkv_kernel(const T* __restrict__ q, const T* __restrict__ keys,
                                                       const T* __restrict__ values, const T* __restrict__ dout,
                                                       const float* __restrict__ lse, const float* __restrict__ dsum,
                                                       T* __restrict__ dk, T* __restrict__ dv, int N, int M, int H,
                                                       int HKV, int W, float scale, float scale_log2, int nkt) {
  using Sh = BwdShape<D>;
  using V8 = typename Mma<T>::V8;
  using V4 = typename Mma<T>::V4;
  __shared__ __align__(16) T sQ[2][64 * Sh::P];
  __shared__ __align__(16) T sD[2][64 * Sh::P];
  __shared__ __align__(16) float sL[2][64], sS[2][64];
  // consecutive key tiles of a KV head on one XCD: their query ranges overlap (L2 hits for Q, dO)
  const int lg = xcd_logical_block(blockIdx.x, gridDim.x);
  const int kt = lg % nkt, bkv = lg / nkt;
  const int b = bkv / HKV, kvh = bkv - b * HKV;
  const int G = H / HKV;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lq = l & 15, g = l >> 4;
  const int S = M + N;
  // each wave holds KB blocks of 16 keys, so every Q or dO fragment it reads from LDS feeds KB
  // MFMAs (and a workgroup's staged query tiles serve 16 NW KB keys)
  const int k0 = 16 * NW * KB * kt;
  int key[KB];
  bool kok[KB];
  size_t krow[KB];
  V8 kf[KB][Sh::KSQ], vf[KB][Sh::KSQ];
  f32x4 dka[KB][Sh::DT], dva[KB][Sh::DT];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    key[kb] = k0 + 16 * (KB * w + kb) + lq;  // this lane's key of block kb
    kok[kb] = key[kb] < S;
    krow[kb] = (((size_t)b * S + (kok[kb] ? key[kb] : 0)) * HKV + kvh) * D;
#pragma unroll
    for (int s = 0; s < Sh::KSQ; ++s) {
      const int f = 32 * s + 8 * g;
      if (kok[kb] && f < D) {
        kf[kb][s] = *reinterpret_cast<const V8*>(keys + krow[kb] + f);
        vf[kb][s] = *reinterpret_cast<const V8*>(values + krow[kb] + f);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          kf[kb][s][e] = from_f32<T>(0.f);
          vf[kb][s][e] = from_f32<T>(0.f);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < Sh::DT; ++t) {
      dka[kb][t] = zero4();
      dva[kb][t] = zero4();
    }
  }
  // the queries that see the tile's keys: M + i in [k0, k0 + 16 NW KB - 1 + W - 1]
  const int ilo = max(0, k0 - M), ihi = min(N - 1, k0 + 16 * NW * KB - 1 + W - 1 - M);
  const int wk0 = k0 + 16 * KB * w, wk1 = wk0 + 16 * KB - 1;
  const size_t q_ld = (size_t)H * D;
  // the (query head, 64-query tile) steps of the group, in order; each step's Q and dO tiles (and
  // its lse, Dsum) are fetched into registers a step ahead and written to the other LDS buffer
  const int nq = ihi >= ilo ? (ihi - ilo) / 64 + 1 : 0, nsteps = G * nq;
  Stage64<T, D, 64 * NW> fq, fd;
  float fl = INFINITY, fs = 0.f;
  auto fetch_step = [&](int step) {
    const int h = kvh * G + step / nq, i0 = ilo + 64 * (step % nq);
    fq.fetch(q + ((size_t)b * N * H + h) * D, q_ld, i0, N);
    fd.fetch(dout + ((size_t)b * N * H + h) * D, q_ld, i0, N);
    const int ii = min(i0 + (int)(threadIdx.x & 63), N - 1);
    fl = lse[((size_t)b * H + h) * N + ii];
    fs = dsum[((size_t)b * H + h) * N + ii];
  };
  auto put_step = [&](int step, int buf) {
    const int i0 = ilo + 64 * (step % nq);
    fq.put(sQ[buf]);
    fd.put(sD[buf]);
    if (threadIdx.x < 64) {
      const bool in = i0 + (int)threadIdx.x < N;
      sL[buf][threadIdx.x] = in ? fl : INFINITY;
      sS[buf][threadIdx.x] = in ? fs : 0.f;
    }
  };
  if (nsteps > 0) {
    fetch_step(0);
    put_step(0, 0);
  }
  __syncthreads();
  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1, i0 = ilo + 64 * (step % nq);
    const T* tQ = sQ[buf];
    const T* tD = sD[buf];
    const float* tL = sL[buf];
    const float* tS = sS[buf];
    if (step + 1 < nsteps) fetch_step(step + 1);
    if (M + i0 + 63 >= wk0 && M + i0 <= wk1 + W - 1) {  // some key of the wave is seen
      // every query of the step sees every key of the wave: no masks (queries past N or inactive
      // have lse +inf; keys past the end are never stored)
      const bool full = M + i0 >= wk1 && M + i0 + 63 - wk0 < W;
#pragma unroll
      for (int qp = 0; qp < 2; ++qp) {
        V8 pb[KB], dsb[KB];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const int r0 = 32 * qp + 16 * qb;
          f32x4 st[KB], dp[KB];
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) st[kb] = dp[kb] = zero4();
#pragma unroll
          for (int s = 0; s < Sh::KSQ; ++s) {
            const V8 qa = row_frag<T, D>(tQ, r0, s), da = row_frag<T, D>(tD, r0, s);
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
              st[kb] = Mma<T>::run(qa, kf[kb][s], st[kb]);
              dp[kb] = Mma<T>::run(da, vf[kb][s], dp[kb]);
            }
          }
          // lane (lq, g) holds queries r0 + 4 g + r of its key; dS without the scale (applied to dK
          // at the end)
          const f32x4 lv = *reinterpret_cast<const f32x4*>(tL + r0 + 4 * g);
          const f32x4 sv = *reinterpret_cast<const f32x4*>(tS + r0 + 4 * g);
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            float p[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][r], scale_log2, -lv[r]));
            if (!full) {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                p[r] = (unsigned)(M + i0 + r0 + 4 * g + r - key[kb]) < (unsigned)W ? p[r] : 0.f;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              pb[kb][4 * qb + r] = from_f32<T>(p[r]);
              dsb[kb][4 * qb + r] = from_f32<T>(p[r] * (dp[kb][r] - sv[r]));
            }
          }
        }
#pragma unroll
        for (int t = 0; t < Sh::DT; ++t) {
          const V8 da = tr_frag<T, D>(tD, 32 * qp, t), qa = tr_frag<T, D>(tQ, 32 * qp, t);
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            dva[kb][t] = Mma<T>::run(da, pb[kb], dva[kb][t]);
            dka[kb][t] = Mma<T>::run(qa, dsb[kb], dka[kb][t]);
          }
        }
      }
    }
    if (step + 1 < nsteps) put_step(step + 1, buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    if (kok[kb]) {
#pragma unroll
      for (int t = 0; t < Sh::DT; ++t) {
        const int d = 16 * t + 4 * g;
        if (d < D) {
          V4 a, c;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            a[r] = from_f32<T>(dka[kb][t][r] * scale);
            c[r] = from_f32<T>(dva[kb][t][r]);
          }
          *reinterpret_cast<V4*>(dk + krow[kb] + d) = a;
          *reinterpret_cast<V4*>(dv + krow[kb] + d) = c;
        }
      }
    }
  }
}

template <typename T, int D>
void launch_backward(const T* q, const T* keys, const T* values, const T* o, const T* dout, const float* lse, float* dsum,
                     T* dq, T* dk, T* dv, int B, int N, int M, int H, int HKV, int W, float scale, hipStream_t stream) {
  const float scale_log2 = scale * 1.4426950408889634f;
  // waves a workgroup (16 queries a dQ wave, 16 KB keys a dK/dV wave); the dK/dV kernel's bound
  // asks for 2 waves a SIMD at least (256 VGPRs): its D 64 instance takes 126 and so runs 4 (two
  // workgroups a CU). Two key blocks a wave (each Q, dO fragment feeding two MFMAs) took 202
  // VGPRs, halving that, and ran slower (dK/dV 67 -> 77 us at B4 T4096 H8 d64 w512).
  constexpr int kDqWaves = 8, kDkvWaves = 8, kDkvWavesPerSimd = 2, kDkvBlocks = 1;
  const int nqt = (N + 16 * kDqWaves - 1) / (16 * kDqWaves);
  const int nkt = (M + N + 16 * kDkvWaves * kDkvBlocks - 1) / (16 * kDkvWaves * kDkvBlocks);
  hipLaunchKernelGGL((attn_dq_kernel<T, D, kDqWaves>), dim3((unsigned)((size_t)nqt * H * B)), dim3(64 * kDqWaves), 0,
                     stream, q, keys,
                     values, o, dout, lse, dsum, dq, N, M, H, HKV, W, scale, scale_log2, nqt);
  hipLaunchKernelGGL((attn_dkv_kernel<T, D, kDkvWaves, kDkvWavesPerSimd, kDkvBlocks>),
                     dim3((unsigned)((size_t)nkt * HKV * B)),
                     dim3(64 * kDkvWaves), 0, stream, q, keys,
                     values, dout, lse, dsum, dk, dv, N, M, H, HKV, W, scale, scale_log2, nkt);
}

template <typename T>
int window_attn_backward(const T* q, const T* keys, const T* values, const T* o, const T* dout, const float* lse,
                         float* dsum, T* dq, T* dk, T* dv, int B, int N, int M, int H, int HKV, int D, int W,
                         float scale, void* stream_ptr, const char* who) {
  if (B < 0 || N < 0 || M < 0 || H < 1 || HKV < 1) return fail(ERR_ARG, "%s: bad sizes B=%d N=%d M=%d H=%d HKV=%d", who, B, N, M, H, HKV);
  if (H % HKV != 0) return fail(ERR_ARG, "%s: %d query heads are not a multiple of %d KV heads", who, H, HKV);
  if (W < 1) return fail(ERR_ARG, "%s: window must be at least 1, got %d", who, W);
  if (!(scale > 0.f)) return fail(ERR_ARG, "%s: the score scale must be positive, got %g", who, (double)scale);
  if (!(D == 16 || D == 32 || D == 64 || D == 128 || D == 256))
    return fail(ERR_UNSUPPORTED, "%s: head dimension %d (kernels: 16, 32, 64, 128, 256)", who, D);
  if (B == 0 || N == 0) return OK;  // no query: the caller's zero dK, dV stand
  if (!q || !keys || !values || !o || !dout || !lse || !dsum || !dq || !dk || !dv)
    return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(values) |
       reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(dout) | reinterpret_cast<uintptr_t>(dq) |
       reinterpret_cast<uintptr_t>(dk) | reinterpret_cast<uintptr_t>(dv)) & 15)
    return fail(ERR_ARG, "%s: q, keys, values, o, dO and the gradients must be 16-byte aligned", who);
  if ((reinterpret_cast<uintptr_t>(lse) | reinterpret_cast<uintptr_t>(dsum)) & 3)
    return fail(ERR_ARG, "%s: lse and the workspace must be 4-byte aligned", who);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  switch (D) {
    case 16: launch_backward<T, 16>(q, keys, values, o, dout, lse, dsum, dq, dk, dv, B, N, M, H, HKV, W, scale, stream); break;
    case 32: launch_backward<T, 32>(q, keys, values, o, dout, lse, dsum, dq, dk, dv, B, N, M, H, HKV, W, scale, stream); break;
    case 64: launch_backward<T, 64>(q, keys, values, o, dout, lse, dsum, dq, dk, dv, B, N, M, H, HKV, W, scale, stream); break;
    case 128: launch_backward<T, 128>(q, keys, values, o, dout, lse, dsum, dq, dk, dv, B, N, M, H, HKV, W, scale, stream); break;
    default: launch_backward<T, 256>(q, keys, values, o, dout, lse, dsum, dq, dk, dv, B, N, M, H, HKV, W, scale, stream); break;
  }
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_window_attn_backward_bf16(const void* q, const void* keys, const void* values, const void* o,
                                             const void* dout, const float* lse, float* workspace, void* dq, void* dk,
                                             void* dv, int B, int N, int M, int H, int HKV, int D, int window,
                                             float scale, void* stream) {
  using T = __bf16;
  return vsp::window_attn_backward<T>(static_cast<const T*>(q), static_cast<const T*>(keys),
                                      static_cast<const T*>(values), static_cast<const T*>(o),
                                      static_cast<const T*>(dout), lse, workspace, static_cast<T*>(dq),
                                      static_cast<T*>(dk), static_cast<T*>(dv), B, N, M, H, HKV, D, window, scale,
                                      stream, "vsp_window_attn_backward_bf16");
}

extern "C" int vsp_window_attn_backward_f16(const void* q, const void* keys, const void* values, const void* o,
                                            const void* dout, const float* lse, float* workspace, void* dq, void* dk,
                                            void* dv, int B, int N, int M, int H, int HKV, int D, int window,
                                            float scale, void* stream) {
  using T = _Float16;
  return vsp::window_attn_backward<T>(static_cast<const T*>(q), static_cast<const T*>(keys),
                                      static_cast<const T*>(values), static_cast<const T*>(o),
                                      static_cast<const T*>(dout), lse, workspace, static_cast<T*>(dq),
                                      static_cast<T*>(dk), static_cast<T*>(dv), B, N, M, H, HKV, D, window, scale,
                                      stream, "vsp_window_attn_backward_f16");
}
