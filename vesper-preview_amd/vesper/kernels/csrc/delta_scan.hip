// Delta-rule scan on CDNA4 (gfx950): the prefill scan and the single-token decode step.
//
// Per batch row b and head h the state H [D, D] (key rows, value columns) is read as H^T q; a token
// applies H <- (I - beta k k^T) H + beta k v^T and reads o = H^T q (reference vesper/recurrence.py:
// 1-23, 118-163). Three kernels:
//
//  * delta_serial_kernel  - token by token, the state of a 64-column block in registers (one lane
//    per value column, rows split over up to four waves). Any D <= 256; the decode step (T = 1)
//    and the fallback for widths the chunked path does not tile.
//  * delta_prep_kernel    - per 64-token chunk, the UT factor T = (I + A)^-1 diag(beta) with
//    A = tril(diag(beta) K K^T, -1): the Gram matrix on MFMA, the four diagonal 16x16 blocks by
//    forward substitution in fp32, the off-diagonal blocks level by level on fp32 MFMA. Chunks are
//    independent, so this runs fully parallel (B*H*ceil(T/64) workgroups).
//  * delta_chain_kernel   - walks the chunks of one (b, h, 16-column value slice) in order with
//    the state slice in MFMA accumulators: R = V - K H, Delta = T R, O = Q H + tril(Q K^T) Delta,
//    H += K^T Delta (the WY/UT form of recurrence.py:17-23 and :202-216, with Delta = U - W H
//    written as T (V - K H)). Value columns of the state evolve independently, so slicing them
//    gives B*H*(D/16) concurrent chains.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kChunk = 64;

// --------------------------------------------------------------------------------------------
// token-serial kernel
// --------------------------------------------------------------------------------------------
template <typename TIn>
__global__ __launch_bounds__(256) void delta_serial_kernel(const TIn* __restrict__ q, const TIn* __restrict__ k,
                                                           const TIn* __restrict__ v, const TIn* __restrict__ beta,
                                                           const float* __restrict__ s_in, float* __restrict__ s_out,
                                                           TIn* __restrict__ o, const uint8_t* __restrict__ active,
                                                           int T, int H, int D, int groups) {
  constexpr int NT = 16;  // tokens staged per round
  __shared__ float sk[NT][256];
  __shared__ float sq[NT][256];
  __shared__ float sv[NT][64];
  __shared__ float sb[NT];
  __shared__ uint8_t sa[NT];
  __shared__ float red[2][4][64];

  const int bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int col = blockIdx.y * 64 + lane;
  const bool col_ok = col < D;
  const size_t sbase = (size_t)bh * D * D;

  float st[64];
#pragma unroll
  for (int r = 0; r < 64; ++r) {
    const int row = wv * 64 + r;
    st[r] = (col_ok && row < D) ? s_in[sbase + (size_t)row * D + col] : 0.f;
  }
  for (int i = threadIdx.x; i < NT * 256; i += blockDim.x) {
    (&sk[0][0])[i] = 0.f;
    (&sq[0][0])[i] = 0.f;
  }

  for (int t0 = 0; t0 < T; t0 += NT) {
    const int nt = min(NT, T - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < nt * D; i += blockDim.x) {
      const int tt = i / D, e = i - tt * D;
      const size_t off = (((size_t)b * T + t0 + tt) * H + h) * D + e;
      sk[tt][e] = to_f32(k[off]);
      sq[tt][e] = to_f32(q[off]);
    }
    for (int i = threadIdx.x; i < nt * 64; i += blockDim.x) {
      const int tt = i >> 6, c = blockIdx.y * 64 + (i & 63);
      sv[tt][i & 63] = c < D ? to_f32(v[(((size_t)b * T + t0 + tt) * H + h) * D + c]) : 0.f;
    }
    if ((int)threadIdx.x < nt) {
      const size_t tok = (size_t)b * T + t0 + threadIdx.x;
      sb[threadIdx.x] = to_f32(beta[tok * H + h]);
      sa[threadIdx.x] = active ? active[tok] : (uint8_t)1;
    }
    __syncthreads();
    for (int tt = 0; tt < nt; ++tt) {
      const float* kr = &sk[tt][wv * 64];
      const float* qr = &sq[tt][wv * 64];
      float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
      for (int r = 0; r < 64; r += 4) {
        p0 += st[r] * kr[r];
        p1 += st[r + 1] * kr[r + 1];
        p2 += st[r + 2] * kr[r + 2];
        p3 += st[r + 3] * kr[r + 3];
      }
      float read = (p0 + p1) + (p2 + p3);
      if (groups > 1) {
        red[0][wv][lane] = read;
        __syncthreads();
        read = 0.f;
        for (int g = 0; g < groups; ++g) read += red[0][g][lane];
      }
      const float u = sb[tt] * (sv[tt][lane] - read);
      p0 = p1 = p2 = p3 = 0.f;
#pragma unroll
      for (int r = 0; r < 64; r += 4) {
        st[r] += kr[r] * u;
        st[r + 1] += kr[r + 1] * u;
        st[r + 2] += kr[r + 2] * u;
        st[r + 3] += kr[r + 3] * u;
        p0 += st[r] * qr[r];
        p1 += st[r + 1] * qr[r + 1];
        p2 += st[r + 2] * qr[r + 2];
        p3 += st[r + 3] * qr[r + 3];
      }
      float out = (p0 + p1) + (p2 + p3);
      if (groups > 1) {
        red[1][wv][lane] = out;
        __syncthreads();
        out = 0.f;
        for (int g = 0; g < groups; ++g) out += red[1][g][lane];
      }
      if (wv == 0 && col_ok)
        o[(((size_t)b * T + t0 + tt) * H + h) * D + col] = from_f32<TIn>(sa[tt] ? out : 0.f);
    }
  }
#pragma unroll
  for (int r = 0; r < 64; ++r) {
    const int row = wv * 64 + r;
    if (col_ok && row < D) s_out[sbase + (size_t)row * D + col] = st[r];
  }
}

// --------------------------------------------------------------------------------------------
// chunk preparation: T = (I + A)^-1 diag(beta) per 64-token chunk
// --------------------------------------------------------------------------------------------
__constant__ int kTriRow[10] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3};
__constant__ int kTriCol[10] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3};

template <typename TIn, typename E, int DK>
__global__ __launch_bounds__(256) void delta_prep_kernel(const TIn* __restrict__ k, const TIn* __restrict__ beta,
                                                         E* __restrict__ tmat, int T, int H) {
  constexpr int KS = Mfma<E>::kstep;
  constexpr int DKP = DK < KS ? KS : DK;
  constexpr int PK = DKP + (sizeof(E) == 2 ? 8 : 1);
  constexpr int PA = 65;
  __shared__ __align__(16) E sK[64 * PK];
  __shared__ float sA[64 * PA];
  __shared__ float sX[64 * PA];
  __shared__ float sY[4][16 * 17];
  __shared__ float sB[64];

  const int nc = (T + kChunk - 1) / kChunk;
  const int g = blockIdx.x;
  const int c = g % nc, bh = g / nc;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kChunk, nv = min(kChunk, T - t0);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lc = l & 15, lr = 4 * (l >> 4);

  for (int i = threadIdx.x; i < 64 * DKP; i += 256) {
    const int r = i / DKP, e = i - r * DKP;
    const float x = (r < nv && e < DK) ? to_f32(k[(((size_t)b * T + t0 + r) * H + h) * DK + e]) : 0.f;
    sK[r * PK + e] = from_f32<E>(x);
  }
  if (threadIdx.x < 64) sB[threadIdx.x] = (int)threadIdx.x < nv ? to_f32(beta[((size_t)b * T + t0 + threadIdx.x) * H + h]) : 0.f;
  for (int i = threadIdx.x; i < 64 * PA; i += 256) sX[i] = 0.f;
  __syncthreads();

  // A = beta_i (K K^T)_ij below the diagonal, lower 16x16 tiles only
  for (int t = w; t < 10; t += 4) {
    const int ti = kTriRow[t], tj = kTriCol[t];
    const f32x4 acc = Mfma<E>::run(sK + 16 * ti * PK, PK, sK + 16 * tj * PK, PK, DKP, zero4());
    const int cc = 16 * tj + lc;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rr = 16 * ti + lr + r;
      sA[rr * PA + cc] = rr > cc ? sB[rr] * acc[r] : 0.f;
    }
  }
  __syncthreads();

  // diagonal blocks: wave w inverts I + A_ww by forward substitution, one lane per column
  if (l < 16) {
    const float* ab = sA + 16 * w * PA + 16 * w;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = (i == l) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) s -= ab[i * PA + j] * x[j];
      x[i] = s;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sX[(16 * w + i) * PA + 16 * w + l] = x[i];
  }
  __syncthreads();

  // off-diagonal blocks by distance d: X_ij = -X_ii sum_{m=j}^{i-1} A_im X_mj, i = j + d
  for (int d = 1; d < 4; ++d) {
    const int bi = w + d, bj = w;
    const bool mine = bi < 4;
    if (mine) {
      f32x4 y = zero4();
      for (int m = bj; m < bi; ++m)
        y = mfma_f32_rowmajor_b(sA + 16 * bi * PA + 16 * m, PA, sX + 16 * m * PA + 16 * bj, PA, 16, y);
      store_tile<float>(&sY[w][0], 17, y);
    }
    __syncthreads();
    if (mine) {
      const f32x4 x = mfma_f32_rowmajor_b(sX + 16 * bi * PA + 16 * bi, PA, &sY[w][0], 17, 16, zero4());
      store_tile<float>(sX + 16 * bi * PA + 16 * bj, PA, -x);
    }
    __syncthreads();
  }

  E* out = tmat + (size_t)g * kChunk * kChunk;
  for (int i = threadIdx.x; i < kChunk * kChunk; i += 256) {
    const int r = i >> 6, cidx = i & 63;
    out[i] = from_f32<E>(cidx <= r ? sX[r * PA + cidx] * sB[cidx] : 0.f);
  }
}

// --------------------------------------------------------------------------------------------
// the chunk chain: one (b, h, value slice) per workgroup, chunks in order
// --------------------------------------------------------------------------------------------
template <typename TIn, typename E, int DK>
__global__ __launch_bounds__(256) void delta_chain_kernel(const TIn* __restrict__ q, const TIn* __restrict__ k,
                                                          const TIn* __restrict__ v, const E* __restrict__ tmat,
                                                          const float* __restrict__ s_in, float* __restrict__ s_out,
                                                          TIn* __restrict__ o, const uint8_t* __restrict__ active,
                                                          int T, int H) {
  constexpr int BV = 16;
  constexpr int NS = DK / BV;
  constexpr int KS = Mfma<E>::kstep;
  constexpr int DKP = DK < KS ? KS : DK;
  constexpr int PAD = sizeof(E) == 2 ? 8 : 1;
  constexpr int PK = DKP + PAD;
  constexpr int PT = 64 + PAD;
  constexpr int HB = DK / 16;
  constexpr int HPW = (HB + 3) / 4;

  __shared__ __align__(16) E sQ[64 * PK];
  __shared__ __align__(16) E sK[64 * PK];
  __shared__ __align__(16) E sKt[DK * PT];
  __shared__ __align__(16) E sT[64 * PT];
  __shared__ __align__(16) E sP[64 * PT];
  __shared__ __align__(16) E sHt[BV * PK];
  __shared__ __align__(16) E sRt[BV * PT];
  __shared__ __align__(16) E sDt[BV * PT];

  const int lg = xcd_logical_block(blockIdx.x, gridDim.x);
  const int slice = lg % NS, bh = lg / NS;
  const int b = bh / H, h = bh - b * H;
  const int v0 = slice * BV;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lc = l & 15, lr = 4 * (l >> 4);
  const int nc = (T + kChunk - 1) / kChunk;

  for (int i = threadIdx.x; i < 64 * PK; i += 256) {
    sQ[i] = from_f32<E>(0.f);
    sK[i] = from_f32<E>(0.f);
  }
  for (int i = threadIdx.x; i < 64 * PT; i += 256) sP[i] = from_f32<E>(0.f);
  for (int i = threadIdx.x; i < BV * PK; i += 256) sHt[i] = from_f32<E>(0.f);

  f32x4 hacc[HPW];
#pragma unroll
  for (int m = 0; m < HPW; ++m) {
    const int rb = w + 4 * m;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      hacc[m][r] = rb < HB ? s_in[((size_t)bh * DK + 16 * rb + lr + r) * DK + v0 + lc] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < HPW; ++m) {
    const int rb = w + 4 * m;
    if (rb < HB) store_tile_t<E>(sHt + 16 * rb, PK, hacc[m]);
  }

  const int kend = ((16 * (w + 1) + KS - 1) / KS) * KS;
  for (int c = 0; c < nc; ++c) {
    const int t0 = c * kChunk, nv = min(kChunk, T - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * DK; i += 256) {
      const int r = i / DK, e = i - r * DK;
      float xq = 0.f, xk = 0.f;
      if (r < nv) {
        const size_t off = (((size_t)b * T + t0 + r) * H + h) * DK + e;
        xq = to_f32(q[off]);
        xk = to_f32(k[off]);
      }
      sQ[r * PK + e] = from_f32<E>(xq);
      sK[r * PK + e] = from_f32<E>(xk);
      sKt[e * PT + r] = from_f32<E>(xk);
    }
    const E* tsrc = tmat + ((size_t)bh * nc + c) * kChunk * kChunk;
    for (int i = threadIdx.x; i < kChunk * kChunk; i += 256) sT[(i >> 6) * PT + (i & 63)] = tsrc[i];
    __syncthreads();

    // stage 1: token rows 16w.. - K H, Q H and the causal tiles of Q K^T
    const E* kw = sK + 16 * w * PK;
    const E* qw = sQ + 16 * w * PK;
    const f32x4 kh = Mfma<E>::run(kw, PK, sHt, PK, DKP, zero4());
    const f32x4 qh = Mfma<E>::run(qw, PK, sHt, PK, DKP, zero4());
    for (int j = 0; j <= w; ++j) {
      const f32x4 p = Mfma<E>::run(qw, PK, sK + 16 * j * PK, PK, DKP, zero4());
      const int cc = 16 * j + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rr = 16 * w + lr + r;
        sP[rr * PT + cc] = from_f32<E>(cc <= rr ? p[r] : 0.f);
      }
    }
    f32x4 rv;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * w + lr + r;
      const float vv = t < nv ? to_f32(v[(((size_t)b * T + t0 + t) * H + h) * DK + v0 + lc]) : 0.f;
      rv[r] = vv - kh[r];
    }
    store_tile_t<E>(sRt + 16 * w, PT, rv);
    __syncthreads();

    // stage 2: Delta = T R for token rows 16w..
    const f32x4 dl = Mfma<E>::run(sT + 16 * w * PT, PT, sRt, PT, kend, zero4());
    store_tile_t<E>(sDt + 16 * w, PT, dl);
    __syncthreads();

    // stage 3: O = Q H + P Delta, then H += K^T Delta
    const f32x4 ov = Mfma<E>::run(sP + 16 * w * PT, PT, sDt, PT, kend, qh);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * w + lr + r;
      if (t < nv) {
        const size_t tok = (size_t)b * T + t0 + t;
        const bool on = active == nullptr || active[tok] != 0;
        o[(tok * H + h) * DK + v0 + lc] = from_f32<TIn>(on ? ov[r] : 0.f);
      }
    }
#pragma unroll
    for (int m = 0; m < HPW; ++m) {
      const int rb = w + 4 * m;
      if (rb < HB) {
        hacc[m] = Mfma<E>::run(sKt + 16 * rb * PT, PT, sDt, PT, kChunk, hacc[m]);
        store_tile_t<E>(sHt + 16 * rb, PK, hacc[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < HPW; ++m) {
    const int rb = w + 4 * m;
    if (rb < HB) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s_out[((size_t)bh * DK + 16 * rb + lr + r) * DK + v0 + lc] = hacc[m][r];
    }
  }
}

// --------------------------------------------------------------------------------------------
// host side
// --------------------------------------------------------------------------------------------
bool chunked_width(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }
constexpr int kSerialBelow = 16;  // shorter sequences run token by token

int check_common(const void* q, const void* k, const void* v, const void* beta, const void* s_in, const void* s_out,
                 const void* o, int B, int T, int H, int D, const char* who) {
  if (B < 0 || T < 0 || H < 0) return fail(ERR_ARG, "%s: negative size (B=%d T=%d H=%d)", who, B, T, H);
  if (D < 1 || D > 256) return fail(ERR_ARG, "%s: head dimension %d outside 1..256", who, D);
  if (B == 0 || H == 0) return OK;
  if (!s_in || !s_out) return fail(ERR_ARG, "%s: null state pointer", who);
  if (T > 0 && (!q || !k || !v || !beta || !o)) return fail(ERR_ARG, "%s: null input or output pointer", who);
  return OK;
}

template <typename TIn>
int launch_serial(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, float* s_out, TIn* o,
                  const uint8_t* active, int B, int T, int H, int D, hipStream_t stream, const char* who) {
  const int groups = (D + 63) / 64;
  dim3 grid((unsigned)(B * H), (unsigned)groups);
  hipLaunchKernelGGL(delta_serial_kernel<TIn>, grid, dim3(64 * groups), 0, stream, q, k, v, beta, s_in, s_out, o,
                     active, T, H, D, groups);
  return check_launch(who);
}

size_t workspace_bytes(int B, int T, int H, int D, bool fp32) {
  if (B <= 0 || H <= 0 || T < kSerialBelow || !chunked_width(D)) return 0;
  const size_t nc = (size_t)(T + kChunk - 1) / kChunk;
  return (size_t)B * H * nc * kChunk * kChunk * (fp32 ? sizeof(float) : sizeof(uint16_t));
}

template <typename TIn, typename E, int DK>
void launch_chunked(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, float* s_out, TIn* o,
                    E* tmat, const uint8_t* active, int B, int T, int H, hipStream_t stream) {
  const int nc = (T + kChunk - 1) / kChunk;
  hipLaunchKernelGGL((delta_prep_kernel<TIn, E, DK>), dim3((unsigned)(B * H * nc)), dim3(256), 0, stream, k, beta, tmat,
                     T, H);
  hipLaunchKernelGGL((delta_chain_kernel<TIn, E, DK>), dim3((unsigned)(B * H * (DK / 16))), dim3(256), 0, stream, q, k,
                     v, tmat, s_in, s_out, o, active, T, H);
}

template <typename TIn, typename E>
int delta_scan(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, TIn* o, float* s_out,
               void* workspace, size_t ws_bytes, const uint8_t* active, int B, int T, int H, int D, void* stream_ptr,
               const char* who) {
  int st = check_common(q, k, v, beta, s_in, s_out, o, B, T, H, D, who);
  if (st != OK || B == 0 || H == 0) return st;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  if (T == 0) {
    if (s_in != s_out) {
      hipError_t err = hipMemcpyAsync(s_out, s_in, (size_t)B * H * D * D * sizeof(float), hipMemcpyDeviceToDevice, stream);
      if (err != hipSuccess) return fail(ERR_LAUNCH, "%s: state copy failed: %s", who, hipGetErrorString(err));
    }
    return OK;
  }
  const size_t need = workspace_bytes(B, T, H, D, sizeof(E) == 4);
  if (need == 0) return launch_serial<TIn>(q, k, v, beta, s_in, s_out, o, active, B, T, H, D, stream, who);
  if (workspace == nullptr || ws_bytes < need)
    return fail(ERR_ARG, "%s: workspace of %zu bytes given, %zu needed", who, workspace ? ws_bytes : (size_t)0, need);
  E* tmat = reinterpret_cast<E*>(workspace);
  switch (D) {
    case 16: launch_chunked<TIn, E, 16>(q, k, v, beta, s_in, s_out, o, tmat, active, B, T, H, stream); break;
    case 32: launch_chunked<TIn, E, 32>(q, k, v, beta, s_in, s_out, o, tmat, active, B, T, H, stream); break;
    case 64: launch_chunked<TIn, E, 64>(q, k, v, beta, s_in, s_out, o, tmat, active, B, T, H, stream); break;
    default: launch_chunked<TIn, E, 128>(q, k, v, beta, s_in, s_out, o, tmat, active, B, T, H, stream); break;
  }
  return check_launch(who);
}

template <typename TIn>
int delta_step(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, float* s_out, TIn* o,
               const uint8_t* active, int B, int H, int D, void* stream_ptr, const char* who) {
  int st = check_common(q, k, v, beta, s_in, s_out, o, B, 1, H, D, who);
  if (st != OK || B == 0 || H == 0) return st;
  return launch_serial<TIn>(q, k, v, beta, s_in, s_out, o, active, B, 1, H, D,
                            reinterpret_cast<hipStream_t>(stream_ptr), who);
}

}  // namespace
}  // namespace vsp

using vsp::delta_scan;
using vsp::delta_step;

extern "C" size_t vsp_delta_scan_workspace_bytes(int B, int T, int H, int D, int fp32_inputs) {
  return vsp::workspace_bytes(B, T, H, D, fp32_inputs != 0);
}

extern "C" int vsp_delta_scan_bf16(const void* q, const void* k, const void* v, const void* beta, const float* state_in,
                                   void* o, float* state_out, void* workspace, size_t workspace_bytes,
                                   const uint8_t* active, int B, int T, int H, int D, void* stream) {
  return delta_scan<__bf16, __bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                                    static_cast<const __bf16*>(v), static_cast<const __bf16*>(beta), state_in,
                                    static_cast<__bf16*>(o), state_out, workspace, workspace_bytes, active, B, T, H, D,
                                    stream, "vsp_delta_scan_bf16");
}

extern "C" int vsp_delta_scan_f32(const float* q, const float* k, const float* v, const float* beta,
                                  const float* state_in, float* o, float* state_out, void* workspace,
                                  size_t workspace_bytes, const uint8_t* active, int B, int T, int H, int D,
                                  void* stream) {
  return delta_scan<float, float>(q, k, v, beta, state_in, o, state_out, workspace, workspace_bytes, active, B, T, H,
                                  D, stream, "vsp_delta_scan_f32");
}

extern "C" int vsp_delta_step_f32(const float* q, const float* k, const float* v, const float* beta,
                                  const float* state_in, float* state_out, float* o, const uint8_t* active, int B,
                                  int H, int D, void* stream) {
  return delta_step<float>(q, k, v, beta, state_in, state_out, o, active, B, H, D, stream, "vsp_delta_step_f32");
}

extern "C" int vsp_delta_step_bf16(const void* q, const void* k, const void* v, const void* beta,
                                   const float* state_in, float* state_out, void* o, const uint8_t* active, int B,
                                   int H, int D, void* stream) {
  return delta_step<__bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                            static_cast<const __bf16*>(v), static_cast<const __bf16*>(beta), state_in, state_out,
                            static_cast<__bf16*>(o), active, B, H, D, stream, "vsp_delta_step_bf16");
}
