// The delta-rule scan's backward on CDNA4 (gfx950): d q, d k, d v, d beta and d state.
//
// The gradients of the chunked scan (reference vesper/recurrence.py:166-217, run on CUDA by fla-core
// behind vesper/kernels/delta_scan.py:132-187 with its backward). Per chunk of C = 64 tokens, with H
// the state at its start, G the gradient of the state at its end, A = tril(diag(beta) K K^T, -1),
// L = (I + A)^-1, T = L diag(beta), R = V - K H, Delta = T R, P = tril(Q K^T) (diagonal included):
//   dDelta = K G + P^T dO,  dR = T^T dDelta (= dV),  dQ = dO H^T + tril(dO Delta^T) K,
//   dT = dDelta R^T,  dA = tril(-L^T (dT diag(beta)) L^T, -1),  M = diag(beta) dA,
//   dK = Delta G^T + tril(dO Delta^T)^T Q - dR H^T + (M + M^T) K,
//   dbeta_j = sum_i dT_ij L_ij + sum_m dA_jm k_j . k_m,
// and the state's gradient at the chunk's start G + Q^T dO - K^T dR = G - W^T (K G) + Y with
// W = T K, Y = Q^T dO - W^T P^T dO.
//
// Four kernels, all arithmetic in fp32 (16x16x4 MFMA, operands staged in LDS), no atomics:
// - scan_bwd_prep_kernel, per (b, h, chunk): L, W, U = T V and Y into the workspace;
// - scan_bwd_states_kernel, per (b, h, 16 value columns): the states at the chunk starts, by the
//   forward chain Delta = U - W H, H += K^T Delta (value columns evolve independently);
// - scan_bwd_dstate_kernel, per (b, h, 16 value columns): the reverse chain of the state's
//   gradient, recorded at every chunk's end, and the initial state's gradient;
// - scan_bwd_chunk_kernel, per (b, h, chunk): every token gradient of the chunk.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kC = 64;       // tokens per chunk
constexpr int kPC = kC + 4;  // pitch (floats) of a [.][64] LDS matrix

// C[16 x 16] += op(X)[16 x K] op(Y)[K x 16] on fp32 MFMA. op(X)[i][k] is X[i * ldx + k] (TA false)
// or X[k * ldx + i] (TA true, X stored [k][i]); op(Y)[k][j] is Y[k * ldy + j] (TB false) or
// Y[j * ldy + k] (TB true), times yscale[k] when given. X and Y point at the tile's origin. The
// result: lane (j, g) holds rows 4 g .. 4 g + 3 of column j.
template <bool TA, bool TB>
__device__ __forceinline__ f32x4 mm16(const float* X, int ldx, const float* Y, int ldy, int K, f32x4 acc,
                                      const float* yscale = nullptr) {
  const int l = threadIdx.x & 63, i = l & 15, kk = l >> 4;
  for (int k = 0; k < K; k += 4) {
    const float a = TA ? X[(k + kk) * ldx + i] : X[i * ldx + k + kk];
    float b = TB ? Y[i * ldy + k + kk] : Y[(k + kk) * ldy + i];
    if (yscale != nullptr) b *= yscale[k + kk];
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
  }
  return acc;
}

// Within a wave, LDS writes of any lane are visible to later LDS reads of any lane.
__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// element (row, col) of an accumulator tile for register r of this lane
__device__ __forceinline__ int tile_row(int r) { return 4 * ((threadIdx.x & 63) >> 4) + r; }
__device__ __forceinline__ int tile_col() { return threadIdx.x & 15; }

// chunk rows t0 .. t0 + 63 of a [B, N, H, D] tensor (head h of batch row b) into LDS [64][ld] as
// fp32; rows past N are zero, and with `active` so are inactive tokens' rows
template <typename TIn, int D>
__device__ __forceinline__ void load_rows(float* dst, int ld, const TIn* src, int b, int h, int t0, int N, int H,
                                          const uint8_t* active = nullptr) {
  for (int e = threadIdx.x; e < kC * D / 4; e += blockDim.x) {
    const int row = e / (D / 4), c = 4 * (e - row * (D / 4));
    const int t = t0 + row;
    const bool ok = t < N && (active == nullptr || active[(size_t)b * N + t] != 0);
    const TIn* p = src + (((size_t)b * N + (ok ? t : 0)) * H + h) * D + c;
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[row * ld + c + j] = ok ? to_f32(p[j]) : 0.f;
  }
}

template <typename TIn>
__device__ __forceinline__ void load_beta(float* dst, const TIn* beta, int b, int h, int t0, int N, int H) {
  for (int r = threadIdx.x; r < kC; r += blockDim.x) {
    const int t = t0 + r;
    dst[r] = t < N ? to_f32(beta[((size_t)b * N + t) * H + h]) : 0.f;
  }
}

// a [rows][D] fp32 global matrix (row pitch D) into LDS [rows][ld]
template <int D>
__device__ __forceinline__ void load_mat(float* dst, int ld, const float* src, int rows) {
  for (int e = threadIdx.x; e < rows * D / 4; e += blockDim.x) {
    const int row = e / (D / 4), c = 4 * (e - row * (D / 4));
    const f32x4 v = *reinterpret_cast<const f32x4*>(src + (size_t)row * D + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[row * ld + c + j] = v[j];
  }
}

// workspace layout, per (b, h, chunk): L [64][64], W [64][D], U [64][D], Y [D][D], Hs [D][D], dHs [D][D]
template <int D> struct Ws {
  static constexpr size_t kL = (size_t)kC * kC, kW = (size_t)kC * D, kS = (size_t)D * D;
  static constexpr size_t kPer = kL + 2 * kW + 3 * kS;
  __device__ __forceinline__ static float* L(float* ws, size_t chunk) { return ws + chunk * kPer; }
  __device__ __forceinline__ static float* W(float* ws, size_t chunk) { return ws + chunk * kPer + kL; }
  __device__ __forceinline__ static float* U(float* ws, size_t chunk) { return ws + chunk * kPer + kL + kW; }
  __device__ __forceinline__ static float* Y(float* ws, size_t chunk) { return ws + chunk * kPer + kL + 2 * kW; }
  __device__ __forceinline__ static float* Hs(float* ws, size_t chunk) { return ws + chunk * kPer + kL + 2 * kW + kS; }
  __device__ __forceinline__ static float* dHs(float* ws, size_t chunk) {
    return ws + chunk * kPer + kL + 2 * kW + 2 * kS;
  }
};

template <typename TIn, int D>
__global__ __launch_bounds__(256) void scan_bwd_prep_kernel(const TIn* __restrict__ q, const TIn* __restrict__ k,
                                                            const TIn* __restrict__ v, const TIn* __restrict__ beta,
                                                            const TIn* __restrict__ d_o,
                                                            const uint8_t* __restrict__ active,
                                                            float* __restrict__ ws, int N, int H, int NC) {
  constexpr int PD = D + 4;
  __shared__ __align__(16) float sK[kC * PD], sQ[kC * PD], sO[kC * PD], sV[kC * PD], sW[kC * PD];
  __shared__ __align__(16) float sA[kC * kPC], sL[kC * kPC];
  __shared__ float sB[kC];
  const int c = blockIdx.x % NC, bh = blockIdx.x / NC;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kC;
  const size_t chunk = blockIdx.x;
  const int w = threadIdx.x >> 6;
  load_rows<TIn, D>(sK, PD, k, b, h, t0, N, H);
  load_rows<TIn, D>(sQ, PD, q, b, h, t0, N, H);
  load_rows<TIn, D>(sO, PD, d_o, b, h, t0, N, H, active);
  load_rows<TIn, D>(sV, PD, v, b, h, t0, N, H);
  load_beta(sB, beta, b, h, t0, N, H);
  __syncthreads();
  // A = tril(diag(beta) K K^T, -1)
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 acc = mm16<false, true>(sK + 16 * w * PD, PD, sK + 16 * ct * PD, PD, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * w + tile_row(r), j = 16 * ct + tile_col();
      sA[i * kPC + j] = i > j ? sB[i] * acc[r] : 0.f;
    }
  }
  __syncthreads();
  // L = (I + A)^-1 by 16x16 blocks: the diagonal blocks (I + A_bb)^-1 by forward substitution (a
  // lane per column of a block), then L_ij = -L_ii sum_{m = j}^{i - 1} A_im L_mj level by level
  // (i - j = 1, 2, 3) on MFMA; the blocks above the diagonal are zero
  for (int e = threadIdx.x; e < kC * kC; e += blockDim.x) {
    const int i = e / kC, j = e - i * kC;
    if (i / 16 < j / 16) sL[i * kPC + j] = 0.f;
  }
  if (w == 0) {
    const int l = threadIdx.x & 63, blk = l >> 4, col = l & 15;
    const float* ab = sA + 16 * blk * kPC + 16 * blk;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sum = i == col ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) sum -= ab[i * kPC + m] * x[m];
      x[i] = sum;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sL[(16 * blk + i) * kPC + 16 * blk + col] = x[i];
  }
  __syncthreads();
  for (int lev = 1; lev < 4; ++lev) {
    const int i = w + lev, j = w;  // block (i, j) of this level, one per wave
    if (i < 4) {
      f32x4 y = zero4();
      for (int m = j; m < i; ++m)
        y = mm16<false, false>(sA + 16 * i * kPC + 16 * m, kPC, sL + 16 * m * kPC + 16 * j, kPC, 16, y);
      // y is a register tile: stage it in the block's own (zero, not yet read) place of sL, then
      // L_ij = -L_ii y
      float* dst = sL + 16 * i * kPC + 16 * j;
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[tile_row(r) * kPC + tile_col()] = y[r];
      wave_sync_lds();  // every lane's y is in LDS before any lane reads it
      const f32x4 x = mm16<false, false>(sL + 16 * i * kPC + 16 * i, kPC, dst, kPC, 16, zero4());
      wave_sync_lds();  // every lane has read y before any lane overwrites it
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[tile_row(r) * kPC + tile_col()] = -x[r];
    }
    __syncthreads();
  }
  float* gL = Ws<D>::L(ws, chunk);
  for (int e = threadIdx.x; e < kC * kC; e += blockDim.x) gL[e] = sL[(e / kC) * kPC + (e % kC)];
  // W = L diag(beta) K and U = L diag(beta) V (rows 16 w of the wave)
  float* gW = Ws<D>::W(ws, chunk);
  float* gU = Ws<D>::U(ws, chunk);
  for (int ct = 0; ct < D / 16; ++ct) {
    const f32x4 aw = mm16<false, false>(sL + 16 * w * kPC, kPC, sK + 16 * ct, PD, kC, zero4(), sB);
    const f32x4 au = mm16<false, false>(sL + 16 * w * kPC, kPC, sV + 16 * ct, PD, kC, zero4(), sB);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * w + tile_row(r), j = 16 * ct + tile_col();
      gW[i * D + j] = aw[r];
      gU[i * D + j] = au[r];
      sW[i * PD + j] = aw[r];
    }
  }
  // P = tril(Q K^T), diagonal included, into sA
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 acc = mm16<false, true>(sQ + 16 * w * PD, PD, sK + 16 * ct * PD, PD, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * w + tile_row(r), j = 16 * ct + tile_col();
      sA[i * kPC + j] = j <= i ? acc[r] : 0.f;
    }
  }
  __syncthreads();  // sW, sA complete; sV's reads are done
  // Z = P^T dO into sV
  for (int ct = 0; ct < D / 16; ++ct) {
    const f32x4 acc = mm16<true, false>(sA + 16 * w, kPC, sO + 16 * ct, PD, kC, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) sV[(16 * w + tile_row(r)) * PD + 16 * ct + tile_col()] = acc[r];
  }
  __syncthreads();
  // Y = Q^T dO - W^T Z [D x D]: row tiles of Y over the waves
  float* gY = Ws<D>::Y(ws, chunk);
  for (int tile = w; tile < (D / 16) * (D / 16); tile += 4) {
    const int rt = tile / (D / 16), ct = tile - rt * (D / 16);
    f32x4 acc = mm16<true, false>(sQ + 16 * rt, PD, sO + 16 * ct, PD, kC, zero4());
    const f32x4 wz = mm16<true, false>(sW + 16 * rt, PD, sV + 16 * ct, PD, kC, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) gY[(16 * rt + tile_row(r)) * D + 16 * ct + tile_col()] = acc[r] - wz[r];
  }
}

// the states at the chunk starts, 16 value columns per workgroup (one wave per 16 rows)
template <typename TIn, int D>
__global__ __launch_bounds__(256) void scan_bwd_states_kernel(const TIn* __restrict__ k,
                                                              const float* __restrict__ state_in,
                                                              float* __restrict__ ws, int N, int H, int NC) {
  constexpr int PD = D + 4, PS = 20, NS = D / 16;
  __shared__ __align__(16) float sW[kC * PD], sK[kC * PD], sU[kC * PS], sD[kC * PS], sH[D * PS];
  const int s = blockIdx.x % NS, bh = blockIdx.x / NS;
  const int b = bh / H, h = bh - b * H;
  const int w = threadIdx.x >> 6;
  const float* h0 = state_in + (size_t)bh * D * D;
  for (int e = threadIdx.x; e < D * 16; e += blockDim.x) sH[(e / 16) * PS + e % 16] = h0[(e / 16) * D + 16 * s + e % 16];
  for (int c = 0; c < NC; ++c) {
    const size_t chunk = (size_t)bh * NC + c;
    __syncthreads();  // sH complete, the previous chunk's reads done
    float* gH = Ws<D>::Hs(ws, chunk);
    for (int e = threadIdx.x; e < D * 16; e += blockDim.x) gH[(e / 16) * D + 16 * s + e % 16] = sH[(e / 16) * PS + e % 16];
    load_mat<D>(sW, PD, Ws<D>::W(ws, chunk), kC);
    load_rows<TIn, D>(sK, PD, k, b, h, c * kC, N, H);
    const float* gU = Ws<D>::U(ws, chunk);
    for (int e = threadIdx.x; e < kC * 16; e += blockDim.x) sU[(e / 16) * PS + e % 16] = gU[(e / 16) * D + 16 * s + e % 16];
    __syncthreads();
    // Delta = U - W H (rows 16 w)
    {
      const f32x4 acc = mm16<false, false>(sW + 16 * w * PD, PD, sH, PS, D, zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + tile_row(r), j = tile_col();
        sD[i * PS + j] = sU[i * PS + j] - acc[r];
      }
    }
    __syncthreads();
    // H += K^T Delta (rows 16 w of H, for w < D / 16)
    if (w < D / 16) {
      const f32x4 acc = mm16<true, false>(sK + 16 * w, PD, sD, PS, kC, zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) sH[(16 * w + tile_row(r)) * PS + tile_col()] += acc[r];
    }
  }
}

// the state's gradient at every chunk's end (reverse chain) and at the start
template <typename TIn, int D>
__global__ __launch_bounds__(256) void scan_bwd_dstate_kernel(const TIn* __restrict__ k,
                                                              const float* __restrict__ d_state,
                                                              float* __restrict__ d_state_in, float* __restrict__ ws,
                                                              int N, int H, int NC) {
  constexpr int PD = D + 4, PS = 20, NS = D / 16;
  __shared__ __align__(16) float sW[kC * PD], sK[kC * PD], sX[kC * PS], sG[D * PS];
  const int s = blockIdx.x % NS, bh = blockIdx.x / NS;
  const int b = bh / H, h = bh - b * H;
  const int w = threadIdx.x >> 6;
  for (int e = threadIdx.x; e < D * 16; e += blockDim.x)
    sG[(e / 16) * PS + e % 16] = d_state != nullptr ? d_state[(size_t)bh * D * D + (e / 16) * D + 16 * s + e % 16] : 0.f;
  for (int c = NC - 1; c >= 0; --c) {
    const size_t chunk = (size_t)bh * NC + c;
    __syncthreads();
    float* gG = Ws<D>::dHs(ws, chunk);
    for (int e = threadIdx.x; e < D * 16; e += blockDim.x) gG[(e / 16) * D + 16 * s + e % 16] = sG[(e / 16) * PS + e % 16];
    load_mat<D>(sW, PD, Ws<D>::W(ws, chunk), kC);
    load_rows<TIn, D>(sK, PD, k, b, h, c * kC, N, H);
    __syncthreads();
    // X = K G (rows 16 w)
    {
      const f32x4 acc = mm16<false, false>(sK + 16 * w * PD, PD, sG, PS, D, zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) sX[(16 * w + tile_row(r)) * PS + tile_col()] = acc[r];
    }
    __syncthreads();
    // G += Y - W^T X (rows 16 w of G)
    if (w < D / 16) {
      const float* gY = Ws<D>::Y(ws, chunk);
      const f32x4 acc = mm16<true, false>(sW + 16 * w, PD, sX, PS, kC, zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + tile_row(r), j = tile_col();
        sG[i * PS + j] += gY[i * D + 16 * s + j] - acc[r];
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < D * 16; e += blockDim.x)
    d_state_in[(size_t)bh * D * D + (e / 16) * D + 16 * s + e % 16] = sG[(e / 16) * PS + e % 16];
}

template <typename TIn, int D>
__global__ __launch_bounds__(256) void scan_bwd_chunk_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TIn* __restrict__ beta,
    const TIn* __restrict__ d_o, const uint8_t* __restrict__ active, const float* __restrict__ ws,
    TIn* __restrict__ dq, TIn* __restrict__ dk, TIn* __restrict__ dv, TIn* __restrict__ dbeta, int N, int H, int NC) {
  constexpr int P = kPC;  // every buffer is [64][68]
  constexpr int NT = D / 16;
  __shared__ __align__(16) float buf[9][kC * P];
  __shared__ float sB[kC], sDB[kC];
  const int c = blockIdx.x % NC, bh = blockIdx.x / NC;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kC;
  const size_t chunk = blockIdx.x;
  const int w = threadIdx.x >> 6;
  float *Bq = buf[0], *Bk = buf[1], *Bo = buf[2], *Br = buf[3], *Bh = buf[4], *Bg = buf[5], *Bl = buf[6];
  float *Bd = buf[7], *Bp = buf[8];
  load_rows<TIn, D>(Bq, P, q, b, h, t0, N, H);
  load_rows<TIn, D>(Bk, P, k, b, h, t0, N, H);
  load_rows<TIn, D>(Bo, P, d_o, b, h, t0, N, H, active);
  load_rows<TIn, D>(Br, P, v, b, h, t0, N, H);
  load_mat<D>(Bh, P, Ws<D>::Hs(const_cast<float*>(ws), chunk), D);
  load_mat<D>(Bg, P, Ws<D>::dHs(const_cast<float*>(ws), chunk), D);
  load_mat<kC>(Bl, P, Ws<D>::L(const_cast<float*>(ws), chunk), kC);
  load_beta(sB, beta, b, h, t0, N, H);
  __syncthreads();
  const int r0 = 16 * w;  // this wave's 16 rows of every [64 x .] result
  // R = V - K H, in place (each tile reads only its own V entries)
  for (int ct = 0; ct < NT; ++ct) {
    const f32x4 acc = mm16<false, false>(Bk + r0 * P, P, Bh + 16 * ct, P, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) Br[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] -= acc[r];
  }
  // P = tril(Q K^T), diagonal included
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 acc = mm16<false, true>(Bq + r0 * P, P, Bk + 16 * ct * P, P, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      Bp[i * P + j] = j <= i ? acc[r] : 0.f;
    }
  }
  __syncthreads();
  // Delta = L diag(beta) R
  for (int ct = 0; ct < NT; ++ct) {
    const f32x4 acc = mm16<false, false>(Bl + r0 * P, P, Br + 16 * ct, P, kC, zero4(), sB);
#pragma unroll
    for (int r = 0; r < 4; ++r) Bd[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] = acc[r];
  }
  __syncthreads();
  // dK accumulates in registers: the wave's rows r0, every column tile
  f32x4 dka[NT];
  // dDelta = K G + P^T dO (registers), dK += Delta G^T
  f32x4 ddl[NT];
  for (int ct = 0; ct < NT; ++ct) {
    ddl[ct] = mm16<false, false>(Bk + r0 * P, P, Bg + 16 * ct, P, D, zero4());
    ddl[ct] = mm16<true, false>(Bp + r0, P, Bo + 16 * ct, P, kC, ddl[ct]);
    dka[ct] = mm16<false, true>(Bd + r0 * P, P, Bg + 16 * ct * P, P, D, zero4());
  }
  __syncthreads();  // the reads of G are done: dDelta goes into its buffer
  float* Bdd = Bg;
  for (int ct = 0; ct < NT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) Bdd[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] = ddl[ct][r];
  __syncthreads();
  // dR = diag(beta) L^T dDelta into P's buffer (free now); dV = dR
  float* Bdr = Bp;
  for (int ct = 0; ct < NT; ++ct) {
    const f32x4 acc = mm16<true, false>(Bl + r0, P, Bdd + 16 * ct, P, kC, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      const float x = sB[i] * acc[r];
      Bdr[i * P + j] = x;
      if (t0 + i < N) dv[(((size_t)b * N + t0 + i) * H + h) * D + j] = from_f32<TIn>(x);
    }
  }
  __syncthreads();
  // dK -= dR H^T
  for (int ct = 0; ct < NT; ++ct) {
    const f32x4 acc = mm16<false, true>(Bdr + r0 * P, P, Bh + 16 * ct * P, P, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) dka[ct][r] -= acc[r];
  }
  __syncthreads();  // the reads of dR are done
  // S2 = tril(dO Delta^T), diagonal included, into dR's buffer
  float* Bs = Bp;
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 acc = mm16<false, true>(Bo + r0 * P, P, Bd + 16 * ct * P, P, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      Bs[i * P + j] = j <= i ? acc[r] : 0.f;
    }
  }
  __syncthreads();
  // dQ = dO H^T + S2 K; dK += S2^T Q
  for (int ct = 0; ct < NT; ++ct) {
    f32x4 acc = mm16<false, true>(Bo + r0 * P, P, Bh + 16 * ct * P, P, D, zero4());
    acc = mm16<false, false>(Bs + r0 * P, P, Bk + 16 * ct, P, kC, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      if (t0 + i < N) dq[(((size_t)b * N + t0 + i) * H + h) * D + j] = from_f32<TIn>(acc[r]);
    }
    dka[ct] = mm16<true, false>(Bs + r0, P, Bq + 16 * ct, P, kC, dka[ct]);
  }
  __syncthreads();  // H, dO, Q, S2, Delta are done with
  // dT = dDelta R^T into H's buffer
  float* Bt = Bh;
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 acc = mm16<false, true>(Bdd + r0 * P, P, Br + 16 * ct * P, P, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) Bt[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] = acc[r];
  }
  __syncthreads();
  // dbeta from T: sum_i dT_ij L_ij (column j, rows i >= j); then dL = tril(dT diag(beta)) in place
  for (int j = threadIdx.x; j < kC; j += blockDim.x) {
    float s = 0.f;
    for (int i = j; i < kC; ++i) s += Bt[i * P + j] * Bl[i * P + j];
    sDB[j] = s;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kC * kC; e += blockDim.x) {
    const int i = e / kC, j = e - i * kC;
    Bt[i * P + j] = j <= i ? Bt[i * P + j] * sB[j] : 0.f;
  }
  __syncthreads();
  // X1 = L^T dL into Q's buffer
  float* Bx = Bq;
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 acc = mm16<true, false>(Bl + r0, P, Bt + 16 * ct, P, kC, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) Bx[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] = acc[r];
  }
  __syncthreads();
  // dA = -tril(X1 L^T, -1) into dO's buffer; G2 = K K^T into Delta's buffer
  float* Ba = Bo;
  float* Bk2 = Bd;
  for (int ct = 0; ct < 4; ++ct) {
    const f32x4 acc = mm16<false, true>(Bx + r0 * P, P, Bl + 16 * ct * P, P, kC, zero4());
    const f32x4 gk = mm16<false, true>(Bk + r0 * P, P, Bk + 16 * ct * P, P, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      Ba[i * P + j] = j < i ? -acc[r] : 0.f;
      Bk2[i * P + j] = gk[r];
    }
  }
  __syncthreads();
  // dbeta from A: sum_{m < i} dA_im (k_i . k_m); then M = diag(beta) dA in place
  for (int i = threadIdx.x; i < kC; i += blockDim.x) {
    float s = 0.f;
    for (int m = 0; m < i; ++m) s += Ba[i * P + m] * Bk2[i * P + m];
    sDB[i] += s;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kC * kC; e += blockDim.x) {
    const int i = e / kC, j = e - i * kC;
    Ba[i * P + j] *= sB[i];
  }
  __syncthreads();
  // dK += M K + M^T K, then store
  for (int ct = 0; ct < NT; ++ct) {
    dka[ct] = mm16<false, false>(Ba + r0 * P, P, Bk + 16 * ct, P, kC, dka[ct]);
    dka[ct] = mm16<true, false>(Ba + r0, P, Bk + 16 * ct, P, kC, dka[ct]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      if (t0 + i < N) dk[(((size_t)b * N + t0 + i) * H + h) * D + j] = from_f32<TIn>(dka[ct][r]);
    }
  }
  for (int i = threadIdx.x; i < kC; i += blockDim.x)
    if (t0 + i < N) dbeta[((size_t)b * N + t0 + i) * H + h] = from_f32<TIn>(sDB[i]);
}

size_t workspace_floats(int B, int N, int H, int D) {
  const size_t nc = (size_t)(N + kC - 1) / kC;
  const size_t per = (size_t)kC * kC + 2 * (size_t)kC * D + 3 * (size_t)D * D;
  return (size_t)B * H * nc * per;
}

template <typename TIn, int D>
void launch(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* state_in, const TIn* d_o,
            const float* d_state, const uint8_t* active, TIn* dq, TIn* dk, TIn* dv, TIn* dbeta, float* d_state_in,
            float* ws, int B, int N, int H, hipStream_t stream) {
  const int NC = (N + kC - 1) / kC;
  const unsigned chunks = (unsigned)((size_t)B * H * NC), slices = (unsigned)((size_t)B * H * (D / 16));
  hipLaunchKernelGGL((scan_bwd_prep_kernel<TIn, D>), dim3(chunks), dim3(256), 0, stream, q, k, v, beta, d_o, active, ws,
                     N, H, NC);
  hipLaunchKernelGGL((scan_bwd_states_kernel<TIn, D>), dim3(slices), dim3(256), 0, stream, k, state_in, ws, N, H, NC);
  hipLaunchKernelGGL((scan_bwd_dstate_kernel<TIn, D>), dim3(slices), dim3(256), 0, stream, k, d_state, d_state_in, ws, N,
                     H, NC);
  hipLaunchKernelGGL((scan_bwd_chunk_kernel<TIn, D>), dim3(chunks), dim3(256), 0, stream, q, k, v, beta, d_o, active, ws,
                     dq, dk, dv, dbeta, N, H, NC);
}

template <typename TIn>
int scan_backward(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* state_in, const TIn* d_o,
                  const float* d_state, const uint8_t* active, TIn* dq, TIn* dk, TIn* dv, TIn* dbeta,
                  float* d_state_in, void* workspace, size_t workspace_bytes, int B, int N, int H, int D,
                  void* stream_ptr, const char* who) {
  if (B < 0 || N < 0 || H < 1) return fail(ERR_ARG, "%s: bad sizes B=%d N=%d H=%d", who, B, N, H);
  if (!(D == 16 || D == 32 || D == 64)) return fail(ERR_UNSUPPORTED, "%s: head dimension %d (backward: 16, 32, 64)", who, D);
  if (B == 0 || N == 0) return OK;  // no token: the caller's state gradient passes through
  if (!q || !k || !v || !beta || !state_in || !d_o || !dq || !dk || !dv || !dbeta || !d_state_in)
    return fail(ERR_ARG, "%s: null pointer", who);
  const size_t need = workspace_floats(B, N, H, D) * sizeof(float);
  if (!workspace || workspace_bytes < need)
    return fail(ERR_ARG, "%s: workspace of %zu bytes, %zu needed", who, workspace_bytes, need);
  if ((reinterpret_cast<uintptr_t>(workspace) | reinterpret_cast<uintptr_t>(state_in) |
       reinterpret_cast<uintptr_t>(d_state) | reinterpret_cast<uintptr_t>(d_state_in)) & 15)
    return fail(ERR_ARG, "%s: the states, their gradients and the workspace must be 16-byte aligned", who);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  float* ws = static_cast<float*>(workspace);
  switch (D) {
    case 16: launch<TIn, 16>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, ws, B, N, H, stream); break;
    case 32: launch<TIn, 32>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, ws, B, N, H, stream); break;
    default: launch<TIn, 64>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, ws, B, N, H, stream); break;
  }
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" size_t vsp_delta_scan_backward_workspace_bytes(int B, int N, int H, int D) {
  if (B <= 0 || N <= 0 || H <= 0 || D <= 0) return 0;
  return vsp::workspace_floats(B, N, H, D) * sizeof(float);
}

extern "C" int vsp_delta_scan_backward_bf16(const void* q, const void* k, const void* v, const void* beta,
                                            const float* state_in, const void* d_o, const float* d_state,
                                            const uint8_t* active, void* dq, void* dk, void* dv, void* dbeta,
                                            float* d_state_in, void* workspace, size_t workspace_bytes, int B, int N,
                                            int H, int D, void* stream) {
  using T = __bf16;
  return vsp::scan_backward<T>(static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                               static_cast<const T*>(beta), state_in, static_cast<const T*>(d_o), d_state, active,
                               static_cast<T*>(dq), static_cast<T*>(dk), static_cast<T*>(dv), static_cast<T*>(dbeta),
                               d_state_in, workspace, workspace_bytes, B, N, H, D, stream,
                               "vsp_delta_scan_backward_bf16");
}

extern "C" int vsp_delta_scan_backward_f32(const float* q, const float* k, const float* v, const float* beta,
                                           const float* state_in, const float* d_o, const float* d_state,
                                           const uint8_t* active, float* dq, float* dk, float* dv, float* dbeta,
                                           float* d_state_in, void* workspace, size_t workspace_bytes, int B, int N,
                                           int H, int D, void* stream) {
  return vsp::scan_backward<float>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in,
                                   workspace, workspace_bytes, B, N, H, D, stream, "vsp_delta_scan_backward_f32");
}
