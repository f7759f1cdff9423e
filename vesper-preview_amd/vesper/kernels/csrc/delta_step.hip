// The single-token delta-rule step on CDNA4 (gfx950): the decode path of the scan.
//
// One token per (b, h) row: H' = H + beta k (v - H^T k)^T and o = H'^T q (reference
// vesper/recurrence.py:118-163). Expanding the read gives o = H^T q + (k . q) u with
// u = beta (v - H^T k), so one pass over H yields both reads (H^T k, H^T q) and the write reuses
// the same registers: the state is read once and written once, which is all the step must move.
//
// Layout: one workgroup per (b, h); thread t owns the float4 column block t % (D/4) of the rows
// t / (D/4) + RG * j (RG row groups), so each row is read by D/4 consecutive lanes in 16-byte
// pieces and every wave instruction touches whole 256-byte rows (D = 64). All of a thread's state
// loads are issued before any arithmetic, so a workgroup has its whole 16 KiB row block in flight
// at once. The column sums over row groups reduce with lane shuffles inside a wave and through LDS
// across waves, in a fixed order (bitwise repeatable).
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

template <int D> struct StepShape {
  static constexpr int NT = D * D / 4 < 256 ? D * D / 4 : 256;  // threads
  static constexpr int CPR = D / 4;                              // float4 blocks per row
  static constexpr int RG = NT / CPR;                            // row groups
  static constexpr int RPT = D / RG;                             // rows per thread
  static constexpr int NW = NT / 64;                             // waves
};

template <typename TIn, int D>
__global__ __launch_bounds__(StepShape<D>::NT) void delta_step_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TIn* __restrict__ beta,
    const float* s_in, float* s_out, TIn* __restrict__ o, const uint8_t* __restrict__ active, int H) {
  // s_in and s_out may alias (an in-place step): each thread writes exactly the elements it read
  using S = StepShape<D>;
  constexpr int CPR = S::CPR, RG = S::RG, RPT = S::RPT, NW = S::NW;
  __shared__ float red[NW][3][D];

  const int bh = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int cb = t % CPR, rg = t / CPR;
  const size_t base = (size_t)bh * D * D;

  float4 st[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) st[j] = reinterpret_cast<const float4*>(s_in + base + (size_t)(rg + RG * j) * D)[cb];
  const TIn* kp = k + (size_t)bh * D;
  const TIn* qp = q + (size_t)bh * D;
  float kr[RPT], qr[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    kr[j] = to_f32(kp[rg + RG * j]);
    qr[j] = to_f32(qp[rg + RG * j]);
  }
  float vv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) vv[c] = to_f32(v[(size_t)bh * D + 4 * cb + c]);
  const float bt = to_f32(beta[bh]);

  // partial column sums of H^T k and H^T q over this thread's rows, and of k . q
  float pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f}, kq = 0.f;
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const float e[4] = {st[j].x, st[j].y, st[j].z, st[j].w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      pk[c] += e[c] * kr[j];
      pq[c] += e[c] * qr[j];
    }
    kq += kr[j] * qr[j];
  }
#pragma unroll
  for (int off = CPR; off < 64; off <<= 1) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      pk[c] += __shfl_xor(pk[c], off);
      pq[c] += __shfl_xor(pq[c], off);
    }
    kq += __shfl_xor(kq, off);
  }
  if constexpr (NW > 1) {
    if (lane < CPR) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        red[wv][0][4 * cb + c] = pk[c];
        red[wv][1][4 * cb + c] = pq[c];
      }
      red[wv][2][cb] = kq;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float a = 0.f, bsum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        a += red[w][0][4 * cb + c];
        bsum += red[w][1][4 * cb + c];
      }
      pk[c] = a;
      pq[c] = bsum;
    }
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += red[w][2][cb];
    kq = s;
  }

  float u[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) u[c] = bt * (vv[c] - pk[c]);
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    float4 w4;
    w4.x = st[j].x + kr[j] * u[0];
    w4.y = st[j].y + kr[j] * u[1];
    w4.z = st[j].z + kr[j] * u[2];
    w4.w = st[j].w + kr[j] * u[3];
    reinterpret_cast<float4*>(s_out + base + (size_t)(rg + RG * j) * D)[cb] = w4;
  }
  if (rg == 0) {
    const bool on = active == nullptr || active[bh / H] != 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[(size_t)bh * D + 4 * cb + c] = from_f32<TIn>(on ? pq[c] + kq * u[c] : 0.f);
  }
}

template <typename TIn, int D>
int launch_step(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, float* s_out, TIn* o,
                const uint8_t* active, int B, int H, hipStream_t stream) {
  hipLaunchKernelGGL((delta_step_kernel<TIn, D>), dim3((unsigned)(B * H)), dim3(StepShape<D>::NT), 0, stream, q, k, v,
                     beta, s_in, s_out, o, active, H);
  return OK;
}

template <typename TIn>
bool step_fast(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, float* s_out, TIn* o,
               const uint8_t* active, int B, int H, int D, hipStream_t stream) {
  // the state rows must be 16-byte aligned for the float4 accesses
  if ((reinterpret_cast<uintptr_t>(s_in) | reinterpret_cast<uintptr_t>(s_out)) & 15) return false;
  switch (D) {
    case 16: launch_step<TIn, 16>(q, k, v, beta, s_in, s_out, o, active, B, H, stream); return true;
    case 32: launch_step<TIn, 32>(q, k, v, beta, s_in, s_out, o, active, B, H, stream); return true;
    case 64: launch_step<TIn, 64>(q, k, v, beta, s_in, s_out, o, active, B, H, stream); return true;
    case 128: launch_step<TIn, 128>(q, k, v, beta, s_in, s_out, o, active, B, H, stream); return true;
    default: return false;
  }
}

}  // namespace

// The register-resident step for head widths 16, 32, 64 and 128; false when the width (or the
// state's alignment) needs the general token-serial kernel instead. Launch errors are left for
// the caller's check_launch.
bool delta_step_fast_f32(const float* q, const float* k, const float* v, const float* beta, const float* s_in,
                         float* s_out, float* o, const uint8_t* active, int B, int H, int D, hipStream_t stream) {
  return step_fast<float>(q, k, v, beta, s_in, s_out, o, active, B, H, D, stream);
}

bool delta_step_fast_bf16(const __bf16* q, const __bf16* k, const __bf16* v, const __bf16* beta, const float* s_in,
                          float* s_out, __bf16* o, const uint8_t* active, int B, int H, int D, hipStream_t stream) {
  return step_fast<__bf16>(q, k, v, beta, s_in, s_out, o, active, B, H, D, stream);
}

}  // namespace vsp
