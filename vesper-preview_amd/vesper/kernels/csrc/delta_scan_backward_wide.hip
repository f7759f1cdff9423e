// The delta-rule scan's backward at head widths the chunked backward kernels do not tile
// (reference: the gradients fla-core gives vesper/kernels/delta_scan.py:132-187 up to its
// MAX_HEAD_DIM = 256, delta_scan.py:38-41), on CDNA4 (gfx950).
//
// The same chunked algebra as delta_scan_backward.hip (per 64-token chunk, with H the state at its
// start, G the state's gradient at its end, L = (I + A)^-1, T = L diag(beta), R = V - K H,
// Delta = T R, P = tril(Q K^T)):
//   dDelta = K G + P^T dO,  dR = T^T dDelta (= dV),  dT = dDelta R^T,
//   dQ = dO H^T + tril(dO Delta^T) K,
//   dK = Delta G^T - dR H^T + tril(dO Delta^T)^T Q + (M + M^T) K,  M = diag(beta) dA,
//   dA = tril(-L^T (dT diag(beta)) L^T, -1),  dbeta_j = sum_i dT_ij L_ij + sum_m dA_jm k_j . k_m,
//   G_start = G + Q^T dO - K^T dR.
// The value columns of H and G evolve independently, so the state-dependent part runs per
// (b, h, group of value columns); the terms that sum over all value columns (dT, tril(dO Delta^T)
// and the H- and G-products of dQ and dK) leave each group as partial sums, added in a fixed order
// by the last kernel (no atomics: the gradients repeat bitwise). Head widths up to 256, multiples
// of 16. Four steps:
// - the token-serial forward stores the state at each chunk's start (delta_scan.hip);
// - wide_prep_kernel, per (b, h, chunk): the Gram matrix K K^T, L by forward substitution in fp32,
//   and P;
// - wide_group_kernel, per (b, h, value group), walks the chunks from the last: R, Delta, dDelta,
//   dR (written as dV), the partial sums, and G (kept in the workspace) carried to the chunk's start;
// - wide_finish_kernel, per (b, h, chunk): the partial sums added, dA, dbeta, dQ and dK.
// Products are 16x16 MFMA tiles of fp32 LDS operands (mm16): fp32 16x16x4 for fp32 inputs, bf16
// 16x16x16 with fp32 accumulation for bf16 inputs, as in the tiled backward. Feature-wide operands
// (K, Q, H and G rows) pass through LDS in blocks of 64 features.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kWC = 64;        // tokens per chunk
constexpr int kWP = kWC + 4;   // pitch (floats) of a [.][64] LDS tile
constexpr int kWT = kWC * kWP;  // floats of one LDS tile
constexpr int kWThreads = 256;
constexpr int kWMaxD = 256;

__device__ __forceinline__ int trow(int r) { return 4 * ((threadIdx.x & 63) >> 4) + r; }
__device__ __forceinline__ int tcol() { return threadIdx.x & 15; }

// The value group width for head width D (a multiple of 16): 64 columns where D allows.
__host__ __device__ constexpr int wide_group(int D) { return D % 64 == 0 ? 64 : (D % 32 == 0 ? 32 : 16); }

// Workspace layout (floats): the chunk-start states [B * H][NC][D][D], the state's gradient G
// [B * H][D][D], the forward's final state [B * H][D][D], then per (b, h, chunk): L, P and the Gram
// matrix [64][64] each, and per value group: dT and tril(dO Delta^T) [64][64], the partial dQ and
// dK [64][D].
struct WideLayout {
  size_t chunk, group;
  int BH, NC, D, NG;
  __host__ __device__ WideLayout(int BH_, int N, int D_)
      : BH(BH_), NC((N + kWC - 1) / kWC), D(D_), NG(D_ / wide_group(D_)) {
    group = 2 * (size_t)kWC * kWC + 2 * (size_t)kWC * D;
    chunk = 3 * (size_t)kWC * kWC + (size_t)NG * group;
  }
  __host__ __device__ size_t dd() const { return (size_t)D * D; }
  __host__ __device__ size_t total() const { return (size_t)BH * ((size_t)(NC + 2) * dd() + (size_t)NC * chunk); }
  __host__ __device__ float* ckpt(float* ws, int bh) const { return ws + (size_t)bh * NC * dd(); }
  __host__ __device__ float* grad(float* ws, int bh) const { return ws + ((size_t)BH * NC + bh) * dd(); }
  __host__ __device__ float* fin(float* ws, int bh) const { return ws + ((size_t)BH * (NC + 1) + bh) * dd(); }
  __host__ __device__ float* chunkp(float* ws, int bh, int c) const {
    return ws + (size_t)BH * (NC + 2) * dd() + ((size_t)bh * NC + c) * chunk;
  }
};

// rows t0 .. t0 + 63 (tokens) of features f0 .. f0 + nf - 1 of a [B, N, H, D] tensor into an LDS
// tile [64][kWP] as fp32; rows past N (or inactive, with `active`) and columns past nf are zero
template <typename TIn>
__device__ __forceinline__ void stage_rows(float* dst, const TIn* src, int b, int h, int t0, int N, int H, int D,
                                           int f0, int nf, const uint8_t* active = nullptr) {
  for (int e = threadIdx.x; e < kWC * 64; e += kWThreads) {
    const int r = e >> 6, c = e & 63, t = t0 + r;
    float x = 0.f;
    if (t < N && c < nf && (active == nullptr || active[(size_t)b * N + t] != 0))
      x = to_f32(src[(((size_t)b * N + t) * H + h) * D + f0 + c]);
    dst[r * kWP + c] = x;
  }
}

// rows f0 .. f0 + nf - 1, columns c0 .. c0 + nc - 1 of a row-major fp32 [.][ld] matrix into an
// LDS tile [64][kWP]; the rest zero
__device__ __forceinline__ void stage_mat(float* dst, const float* src, int ld, int f0, int nf, int c0, int nc) {
  for (int e = threadIdx.x; e < kWC * 64; e += kWThreads) {
    const int r = e >> 6, c = e & 63;
    dst[r * kWP + c] = (r < nf && c < nc) ? src[(size_t)(f0 + r) * ld + c0 + c] : 0.f;
  }
}

// ---- the chunk's Gram matrix, L and P ------------------------------------------------------------
template <typename TIn, bool BF>
__global__ __launch_bounds__(kWThreads) void wide_prep_kernel(const TIn* __restrict__ q, const TIn* __restrict__ k,
                                                              const TIn* __restrict__ beta, float* __restrict__ ws,
                                                              int B, int N, int H, int D) {
  __shared__ __align__(16) float sK[kWT], sQ[kWT], sA[kWT];
  __shared__ float sB[kWC];
  const WideLayout lay(B * H, N, D);
  const int c = blockIdx.x % lay.NC, bh = blockIdx.x / lay.NC;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kWC;
  const int w = threadIdx.x >> 6;
  float* cw = lay.chunkp(ws, bh, c);
  float *gL = cw, *gP = cw + kWC * kWC, *gG = cw + 2 * kWC * kWC;
  if (threadIdx.x < kWC) {
    const int t = t0 + threadIdx.x;
    sB[threadIdx.x] = t < N ? to_f32(beta[((size_t)b * N + t) * H + h]) : 0.f;
  }
  f32x4 gram[4] = {zero4(), zero4(), zero4(), zero4()}, pq[4] = {zero4(), zero4(), zero4(), zero4()};
  for (int f0 = 0; f0 < D; f0 += 64) {
    const int nf = min(64, D - f0);
    __syncthreads();
    stage_rows(sK, k, b, h, t0, N, H, D, f0, nf);
    stage_rows(sQ, q, b, h, t0, N, H, D, f0, nf);
    __syncthreads();
    // wave w: row tile w of K K^T and Q K^T, column tiles 0..3 (k over this block's features)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      gram[ct] = mm16<false, true, BF>(sK + 16 * w * kWP, kWP, sK + 16 * ct * kWP, kWP, nf, gram[ct]);
      pq[ct] = mm16<false, true, BF>(sQ + 16 * w * kWP, kWP, sK + 16 * ct * kWP, kWP, nf, pq[ct]);
    }
  }
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * w + trow(r), j = 16 * ct + tcol();
      gG[i * kWC + j] = gram[ct][r];
      gP[i * kWC + j] = j <= i ? pq[ct][r] : 0.f;
      sA[i * kWP + j] = j < i ? sB[i] * gram[ct][r] : 0.f;
    }
  __syncthreads();
  // L = (I + A)^-1 by forward substitution in fp32: thread j solves column j
  if (threadIdx.x < kWC) {
    const int j = threadIdx.x;
    float x[kWC];
#pragma unroll
    for (int i = 0; i < kWC; ++i) {
      float s = i == j ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) s -= sA[i * kWP + m] * x[m];
      x[i] = s;
    }
#pragma unroll
    for (int i = 0; i < kWC; ++i) gL[i * kWC + j] = x[i];
  }
}

// ---- the state-dependent part, per (b, h, value group), chunks from the last -------------------
template <typename TIn, bool BF>
__global__ __launch_bounds__(kWThreads) void wide_group_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TIn* __restrict__ beta,
    const TIn* __restrict__ d_o, const float* __restrict__ d_state, const uint8_t* __restrict__ active,
    TIn* __restrict__ dv, float* __restrict__ d_state_in, float* __restrict__ ws, int B, int N, int H, int D) {
  __shared__ __align__(16) float sT[kWT], sP[kWT], sR[kWT], sD[kWT], sDD[kWT], sDR[kWT], sO[kWT], sX[kWT], sY[kWT];
  const WideLayout lay(B * H, N, D);
  const int VG = wide_group(D), NG = lay.NG;
  const int g = blockIdx.x % NG, bh = blockIdx.x / NG;
  const int b = bh / H, h = bh - b * H;
  const int v0 = g * VG, nvt = VG / 16;  // the group's value columns and their 16-column tiles
  const int w = threadIdx.x >> 6;
  float* G = lay.grad(ws, bh);
  // G starts as the final state's gradient (zero without one), this group's columns only
  for (int e = threadIdx.x; e < D * VG; e += kWThreads) {
    const int r = e / VG, cc = v0 + e % VG;
    G[(size_t)r * D + cc] = d_state != nullptr ? d_state[((size_t)bh * D + r) * D + cc] : 0.f;
  }
  for (int c = lay.NC - 1; c >= 0; --c) {
    const int t0 = c * kWC;
    const float* Hc = lay.ckpt(ws, bh) + (size_t)c * D * D;
    float* cw = lay.chunkp(ws, bh, c);
    const float *gL = cw, *gP = cw + kWC * kWC;
    float* part = cw + 3 * kWC * kWC + (size_t)g * lay.group;
    float *pDT = part, *pS2 = part + kWC * kWC, *pDQ = part + 2 * kWC * kWC, *pDK = pDQ + (size_t)kWC * D;
    __syncthreads();  // the previous chunk's G writes and LDS reads are done
    for (int e = threadIdx.x; e < kWC * kWC; e += kWThreads) {
      const int i = e >> 6, j = e & 63, tj = t0 + j;
      const float bj = tj < N ? to_f32(beta[((size_t)b * N + tj) * H + h]) : 0.f;
      sT[i * kWP + j] = j <= i ? gL[e] * bj : 0.f;
      sP[i * kWP + j] = gP[e];
    }
    // R = V - K H over the group's columns (features in blocks of 64)
    f32x4 acc[4] = {zero4(), zero4(), zero4(), zero4()};
    for (int f0 = 0; f0 < D; f0 += 64) {
      const int nf = min(64, D - f0);
      __syncthreads();
      stage_rows(sX, k, b, h, t0, N, H, D, f0, nf);
      stage_mat(sY, Hc, D, f0, nf, v0, VG);
      __syncthreads();
      for (int ct = 0; ct < nvt; ++ct) acc[ct] = mm16<false, false, BF>(sX + 16 * w * kWP, kWP, sY + 16 * ct, kWP, nf, acc[ct]);
    }
    for (int ct = 0; ct < nvt; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + trow(r), j = 16 * ct + tcol(), t = t0 + i;
        const float vij = t < N ? to_f32(v[(((size_t)b * N + t) * H + h) * D + v0 + j]) : 0.f;
        sR[i * kWP + j] = vij - acc[ct][r];
      }
    stage_rows(sO, d_o, b, h, t0, N, H, D, v0, VG, active);
    __syncthreads();
    // Delta = T R
    for (int ct = 0; ct < nvt; ++ct) {
      const f32x4 d = mm16<false, false, BF>(sT + 16 * w * kWP, kWP, sR + 16 * ct, kWP, kWC, zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) sD[(16 * w + trow(r)) * kWP + 16 * ct + tcol()] = d[r];
    }
    // dDelta = K G + P^T dO
    for (int ct = 0; ct < nvt; ++ct) acc[ct] = mm16<true, false, BF>(sP + 16 * w, kWP, sO + 16 * ct, kWP, kWC, zero4());
    for (int f0 = 0; f0 < D; f0 += 64) {
      const int nf = min(64, D - f0);
      __syncthreads();
      stage_rows(sX, k, b, h, t0, N, H, D, f0, nf);
      stage_mat(sY, G, D, f0, nf, v0, VG);
      __syncthreads();
      for (int ct = 0; ct < nvt; ++ct) acc[ct] = mm16<false, false, BF>(sX + 16 * w * kWP, kWP, sY + 16 * ct, kWP, nf, acc[ct]);
    }
    for (int ct = 0; ct < nvt; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) sDD[(16 * w + trow(r)) * kWP + 16 * ct + tcol()] = acc[ct][r];
    __syncthreads();
    // dR = T^T dDelta: the values' gradient
    for (int ct = 0; ct < nvt; ++ct) {
      const f32x4 d = mm16<true, false, BF>(sT + 16 * w, kWP, sDD + 16 * ct, kWP, kWC, zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + trow(r), j = 16 * ct + tcol(), t = t0 + i;
        sDR[i * kWP + j] = d[r];
        if (t < N) dv[(((size_t)b * N + t) * H + h) * D + v0 + j] = from_f32<TIn>(d[r]);
      }
    }
    // the group's parts of dT = dDelta R^T and of tril(dO Delta^T) (k over the group's columns)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const f32x4 dt = mm16<false, true, BF>(sDD + 16 * w * kWP, kWP, sR + 16 * ct * kWP, kWP, VG, zero4());
      const f32x4 s2 = mm16<false, true, BF>(sO + 16 * w * kWP, kWP, sD + 16 * ct * kWP, kWP, VG, zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + trow(r), j = 16 * ct + tcol();
        pDT[i * kWC + j] = dt[r];
        pS2[i * kWC + j] = j <= i ? s2[r] : 0.f;
      }
    }
    __syncthreads();  // sR is free; sDR, sD, sO stay
    // the group's parts of dQ = dO H^T and dK = Delta G^T - dR H^T, feature block by block
    for (int f0 = 0; f0 < D; f0 += 64) {
      const int nf = min(64, D - f0);
      __syncthreads();
      stage_mat(sX, G, D, f0, nf, v0, VG);
      stage_mat(sY, Hc, D, f0, nf, v0, VG);
      __syncthreads();
      for (int ft = 0; ft < nf / 16; ++ft) {
        const f32x4 dq = mm16<false, true, BF>(sO + 16 * w * kWP, kWP, sY + 16 * ft * kWP, kWP, VG, zero4());
        f32x4 dk = mm16<false, true, BF>(sD + 16 * w * kWP, kWP, sX + 16 * ft * kWP, kWP, VG, zero4());
        const f32x4 rh = mm16<false, true, BF>(sDR + 16 * w * kWP, kWP, sY + 16 * ft * kWP, kWP, VG, zero4());
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * w + trow(r), f = f0 + 16 * ft + tcol();
          pDQ[(size_t)i * D + f] = dq[r];
          pDK[(size_t)i * D + f] = dk[r] - rh[r];
        }
      }
    }
    // G at the chunk's start: G + Q^T dO - K^T dR (each tile read and written by its own lanes)
    for (int f0 = 0; f0 < D; f0 += 64) {
      const int nf = min(64, D - f0);
      __syncthreads();
      stage_rows(sX, q, b, h, t0, N, H, D, f0, nf);
      stage_rows(sY, k, b, h, t0, N, H, D, f0, nf);
      __syncthreads();
      if (16 * w < nf) {
        for (int ct = 0; ct < nvt; ++ct) {
          const f32x4 qo = mm16<true, false, BF>(sX + 16 * w, kWP, sO + 16 * ct, kWP, kWC, zero4());
          const f32x4 kr = mm16<true, false, BF>(sY + 16 * w, kWP, sDR + 16 * ct, kWP, kWC, zero4());
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float* gp = G + (size_t)(f0 + 16 * w + trow(r)) * D + v0 + 16 * ct + tcol();
            *gp = *gp + qo[r] - kr[r];
          }
        }
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < D * VG; e += kWThreads) {
    const int r = e / VG, cc = v0 + e % VG;
    d_state_in[((size_t)bh * D + r) * D + cc] = G[(size_t)r * D + cc];
  }
}

// ---- the sums over value groups, dA, dbeta, dQ and dK per (b, h, chunk) ---------------------------
template <typename TIn, bool BF>
__global__ __launch_bounds__(kWThreads) void wide_finish_kernel(const TIn* __restrict__ q, const TIn* __restrict__ k,
                                                                const TIn* __restrict__ beta, TIn* __restrict__ dq,
                                                                TIn* __restrict__ dk, TIn* __restrict__ dbeta,
                                                                const float* __restrict__ ws, int B, int N, int H,
                                                                int D) {
  __shared__ __align__(16) float sL[kWT], sGr[kWT], sDT[kWT], sS2[kWT], sM[kWT], sX[kWT], sY[kWT];
  __shared__ float sB[kWC];
  const WideLayout lay(B * H, N, D);
  const int c = blockIdx.x % lay.NC, bh = blockIdx.x / lay.NC;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kWC;
  const int w = threadIdx.x >> 6;
  const float* cw = lay.chunkp(const_cast<float*>(ws), bh, c);
  const float *gL = cw, *gG = cw + 2 * kWC * kWC;
  if (threadIdx.x < kWC) {
    const int t = t0 + threadIdx.x;
    sB[threadIdx.x] = t < N ? to_f32(beta[((size_t)b * N + t) * H + h]) : 0.f;
  }
  for (int e = threadIdx.x; e < kWC * kWC; e += kWThreads) {
    const int i = e >> 6, j = e & 63;
    float dt = 0.f, s2 = 0.f;
    for (int gi = 0; gi < lay.NG; ++gi) {  // the groups' partial sums in a fixed order
      const float* part = cw + 3 * kWC * kWC + (size_t)gi * lay.group;
      dt += part[e];
      s2 += part[kWC * kWC + e];
    }
    sL[i * kWP + j] = gL[e];
    sGr[i * kWP + j] = gG[e];
    sDT[i * kWP + j] = dt;
    sS2[i * kWP + j] = s2;
  }
  __syncthreads();
  // dL = tril(dT diag(beta)) into sX; X1 = L^T dL into sY; dA = -tril(X1 L^T, -1) into sM
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * w + trow(r), j = 16 * ct + tcol();
      sX[i * kWP + j] = j <= i ? sDT[i * kWP + j] * sB[j] : 0.f;
    }
  __syncthreads();
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 x1 = mm16<true, false, false>(sL + 16 * w, kWP, sX + 16 * ct, kWP, kWC, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) sY[(16 * w + trow(r)) * kWP + 16 * ct + tcol()] = x1[r];
  }
  __syncthreads();
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 da = mm16<false, true, false>(sY + 16 * w * kWP, kWP, sL + 16 * ct * kWP, kWP, kWC, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * w + trow(r), j = 16 * ct + tcol();
      sM[i * kWP + j] = j < i ? -da[r] : 0.f;
    }
  }
  __syncthreads();
  // dbeta_j = sum_i dT_ij L_ij + sum_m dA_jm gram_jm (fixed order)
  if (threadIdx.x < kWC) {
    const int j = threadIdx.x, t = t0 + j;
    float s = 0.f;
    for (int i = 0; i < kWC; ++i) s += sDT[i * kWP + j] * sL[i * kWP + j];
    for (int m = 0; m < kWC; ++m) s += sM[j * kWP + m] * sGr[j * kWP + m];
    if (t < N) dbeta[((size_t)b * N + t) * H + h] = from_f32<TIn>(s);
  }
  __syncthreads();
  // M = diag(beta) dA
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * w + trow(r), j = 16 * ct + tcol();
      sM[i * kWP + j] *= sB[i];
    }
  // dQ = sum dO H^T + S2 K and dK = sum (Delta G^T - dR H^T) + S2^T Q + M K + M^T K, feature blocks
  for (int f0 = 0; f0 < D; f0 += 64) {
    const int nf = min(64, D - f0);
    __syncthreads();
    stage_rows(sX, k, b, h, t0, N, H, D, f0, nf);
    stage_rows(sY, q, b, h, t0, N, H, D, f0, nf);
    __syncthreads();
    for (int ft = 0; ft < nf / 16; ++ft) {
      const f32x4 sk = mm16<false, false, BF>(sS2 + 16 * w * kWP, kWP, sX + 16 * ft, kWP, kWC, zero4());
      f32x4 kk = mm16<true, false, BF>(sS2 + 16 * w, kWP, sY + 16 * ft, kWP, kWC, zero4());
      kk = mm16<false, false, BF>(sM + 16 * w * kWP, kWP, sX + 16 * ft, kWP, kWC, kk);
      kk = mm16<true, false, BF>(sM + 16 * w, kWP, sX + 16 * ft, kWP, kWC, kk);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + trow(r), f = f0 + 16 * ft + tcol(), t = t0 + i;
        float pq = 0.f, pk = 0.f;
        for (int gi = 0; gi < lay.NG; ++gi) {
          const float* part = cw + 3 * kWC * kWC + (size_t)gi * lay.group + 2 * kWC * kWC;
          pq += part[(size_t)i * D + f];
          pk += part[(size_t)kWC * D + (size_t)i * D + f];
        }
        if (t < N) {
          const size_t o = (((size_t)b * N + t) * H + h) * D + f;
          dq[o] = from_f32<TIn>(pq + sk[r]);
          dk[o] = from_f32<TIn>(pk + kk[r]);
        }
      }
    }
  }
}

template <typename TIn>
int run_wide(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* state_in, const TIn* d_o,
             const float* d_state, const uint8_t* active, TIn* dq, TIn* dk, TIn* dv, TIn* dbeta, float* d_state_in,
             void* workspace, size_t workspace_bytes, int B, int N, int H, int D, hipStream_t stream, const char* who) {
  if (B < 0 || N < 0 || H < 1) return fail(ERR_ARG, "%s: bad sizes B=%d N=%d H=%d", who, B, N, H);
  if (D < 16 || D > kWMaxD || D % 16 != 0)
    return fail(ERR_UNSUPPORTED, "%s: head dimension %d (the wide backward: multiples of 16 up to %d)", who, D, kWMaxD);
  if (B == 0 || N == 0) return OK;
  if (!q || !k || !v || !beta || !state_in || !d_o || !dq || !dk || !dv || !dbeta || !d_state_in)
    return fail(ERR_ARG, "%s: null pointer", who);
  const size_t need = wide_backward_workspace_bytes(B, N, H, D);
  if (!workspace || workspace_bytes < need)
    return fail(ERR_ARG, "%s: workspace of %zu bytes, %zu needed", who, workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) & 15) return fail(ERR_ARG, "%s: the workspace must be 16-byte aligned", who);
  const WideLayout lay(B * H, N, D);
  float* ws = static_cast<float*>(workspace);
  constexpr bool BF = sizeof(TIn) == 2;
  // the forward's chunk-start states (its final state is not needed)
  if constexpr (BF)
    delta_scan_checkpoints_bf16(q, k, v, beta, state_in, lay.fin(ws, 0), lay.ckpt(ws, 0), B, N, H, D, stream);
  else
    delta_scan_checkpoints_f32(q, k, v, beta, state_in, lay.fin(ws, 0), lay.ckpt(ws, 0), B, N, H, D, stream);
  const unsigned chunks = (unsigned)((size_t)B * H * lay.NC);
  hipLaunchKernelGGL((wide_prep_kernel<TIn, BF>), dim3(chunks), dim3(kWThreads), 0, stream, q, k, beta, ws, B, N, H, D);
  hipLaunchKernelGGL((wide_group_kernel<TIn, BF>), dim3((unsigned)(B * H * lay.NG)), dim3(kWThreads), 0, stream, q, k, v,
                     beta, d_o, d_state, active, dv, d_state_in, ws, B, N, H, D);
  hipLaunchKernelGGL((wide_finish_kernel<TIn, BF>), dim3(chunks), dim3(kWThreads), 0, stream, q, k, beta, dq, dk, dbeta,
                     ws, B, N, H, D);
  return check_launch(who);
}

}  // namespace

size_t wide_backward_workspace_bytes(int B, int N, int H, int D) {
  if (B <= 0 || N <= 0 || H <= 0 || D < 16 || D > kWMaxD || D % 16 != 0) return 0;
  return WideLayout(B * H, N, D).total() * sizeof(float);
}

int scan_backward_wide_bf16(const __bf16* q, const __bf16* k, const __bf16* v, const __bf16* beta,
                            const float* state_in, const __bf16* d_o, const float* d_state, const uint8_t* active,
                            __bf16* dq, __bf16* dk, __bf16* dv, __bf16* dbeta, float* d_state_in, void* workspace,
                            size_t workspace_bytes, int B, int N, int H, int D, hipStream_t stream, const char* who) {
  return run_wide<__bf16>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, workspace,
                          workspace_bytes, B, N, H, D, stream, who);
}

int scan_backward_wide_f32(const float* q, const float* k, const float* v, const float* beta, const float* state_in,
                           const float* d_o, const float* d_state, const uint8_t* active, float* dq, float* dk,
                           float* dv, float* dbeta, float* d_state_in, void* workspace, size_t workspace_bytes, int B,
                           int N, int H, int D, hipStream_t stream, const char* who) {
  return run_wide<float>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, workspace,
                         workspace_bytes, B, N, H, D, stream, who);
}

}  // namespace vsp
