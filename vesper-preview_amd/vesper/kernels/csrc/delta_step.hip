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
//
// With a key filter of K taps (the decode step's key, vsp_delta_step_keys_bf16) the workgroup
// forms its head's key itself before the step: the first wave filters the head's key inputs z
// with the taps over the key history and normalizes the result (vesper/column.py:255-289 with
// vesper/recurrence.py:91-115), with the key filter kernel's arithmetic (the same order of terms,
// the same reductions over D/8-lane groups, the key rounded to bf16 as that kernel stores it), so
// the step is bitwise the two launches'; it writes the next history over the history (its own
// head's features, read into registers first). The state's loads are issued before, so the
// filter runs while they arrive.
#include "common.h"
#include "keys_rows.h"
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

template <typename TIn, int D, int K = 0>
__global__ __launch_bounds__(StepShape<D>::NT) void delta_step_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TIn* __restrict__ beta,
    const float* s_in, float* s_out, TIn* __restrict__ o, const uint8_t* __restrict__ active, int H,
    float* history = nullptr, const float* __restrict__ taps = nullptr) {
  // s_in and s_out may alias (an in-place step): each thread writes exactly the elements it read.
  // K > 0: k holds the key inputs z [B, H * D] and the key is filtered here (history [B, K-1, H*D],
  // taps [K, H*D], both float32).
  using S = StepShape<D>;
  constexpr int CPR = S::CPR, RG = S::RG, RPT = S::RPT, NW = S::NW;
  __shared__ float red[NW][3][D];
  __shared__ float skey[K > 0 ? D : 1];

  const int bh = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int cb = t % CPR, rg = t / CPR;
  const size_t base = (size_t)bh * D * D;

  // the state streams (read once, written once a step; a decoder's states outgrow the caches):
  // nontemporal loads and stores
  f32x4 st[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j)
    st[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(s_in + base + (size_t)(rg + RG * j) * D) + cb);
  if constexpr (K > 0) {
    // the first wave forms the key: lane l takes features 8 (l % LPH) .. + 7 of the head (the lanes
    // past LPH repeat a group; only the first group stores)
    constexpr int LPH = D / 8;
    if (t < 64) {
      const int fc = t % LPH, b = bh / H, DT = H * D;
      const size_t fo = (size_t)(bh - b * H) * D + 8 * fc;
      float cur[8], tp[K][8], win[K > 1 ? K - 1 : 1][8];
      load8_f32(k + (size_t)b * DT + fo, cur);
#pragma unroll
      for (int r = 0; r < K; ++r) load8_f32(taps + (size_t)r * DT + fo, tp[r]);
      float* hb = history + (size_t)b * (K - 1) * DT + fo;
#pragma unroll
      for (int r = 1; r < K; ++r) load8_f32(hb + (size_t)(K - 1 - r) * DT, win[r - 1]);  // input t - r
      // the filter in the reference's order: taps[0] z[t], then + taps[r] z[t - r] for r = 1, 2, ...
      float u[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = tp[0][e] * cur[e];
#pragma unroll
        for (int r = 1; r < K; ++r) acc = acc + tp[r][e] * win[r - 1][e];
        u[e] = acc;
      }
      // normalize_keys over the head: s = u / max(peak, floor), key = s / sqrt(max(|s|^2, 1))
      float peak = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) peak = __builtin_fmaxf(peak, fabsf(u[e]));
      const float scale = __builtin_fmaxf(group_max<LPH>(peak), kKeyFloor);
      const float inv_scale = __builtin_amdgcn_rcpf(scale);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float s0 = u[e] * inv_scale;
        u[e] = __builtin_fmaf(__builtin_fmaf(-s0, scale, u[e]), inv_scale, s0);
        ss += u[e] * u[e];
      }
      const float inv_den = __builtin_amdgcn_rsqf(__builtin_fmaxf(group_sum<LPH>(ss), 1.f));
      if (t < LPH) {
#pragma unroll
        for (int e = 0; e < 8; ++e) skey[8 * fc + e] = to_f32(from_f32<TIn>(u[e] * inv_den));
        // the next history: rows 1 .. K - 2 move down one, the token's inputs become row K - 2
#pragma unroll
        for (int i = 0; i + 1 < K - 1; ++i) {
          const float* src = win[K - 3 - i];  // old row i + 1
          *reinterpret_cast<float4*>(hb + (size_t)i * DT) = make_float4(src[0], src[1], src[2], src[3]);
          *reinterpret_cast<float4*>(hb + (size_t)i * DT + 4) = make_float4(src[4], src[5], src[6], src[7]);
        }
        if constexpr (K > 1) {
          *reinterpret_cast<float4*>(hb + (size_t)(K - 2) * DT) = make_float4(cur[0], cur[1], cur[2], cur[3]);
          *reinterpret_cast<float4*>(hb + (size_t)(K - 2) * DT + 4) = make_float4(cur[4], cur[5], cur[6], cur[7]);
        }
      }
    }
    __syncthreads();
  }
  const TIn* kp = k + (size_t)bh * D;
  const TIn* qp = q + (size_t)bh * D;
  float kr[RPT], qr[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    kr[j] = K > 0 ? skey[rg + RG * j] : to_f32(kp[rg + RG * j]);
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
    const float e[4] = {st[j][0], st[j][1], st[j][2], st[j][3]};
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
    f32x4 w4;
    w4[0] = st[j][0] + kr[j] * u[0];
    w4[1] = st[j][1] + kr[j] * u[1];
    w4[2] = st[j][2] + kr[j] * u[2];
    w4[3] = st[j][3] + kr[j] * u[3];
    __builtin_nontemporal_store(w4, reinterpret_cast<f32x4*>(s_out + base + (size_t)(rg + RG * j) * D) + cb);
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

template <int D, int K>
void launch_step_keys(const __bf16* q, const __bf16* z, const __bf16* v, const __bf16* beta, float* history,
                      const float* taps, const float* s_in, float* s_out, __bf16* o, const uint8_t* active, int B,
                      int H, hipStream_t stream) {
  hipLaunchKernelGGL((delta_step_kernel<__bf16, D, K>), dim3((unsigned)(B * H)), dim3(StepShape<D>::NT), 0, stream, q,
                     z, v, beta, s_in, s_out, o, active, H, history, taps);
}

template <int D>
void step_keys_by_width(int K, const __bf16* q, const __bf16* z, const __bf16* v, const __bf16* beta,
                        float* history, const float* taps, const float* s_in, float* s_out, __bf16* o,
                        const uint8_t* active, int B, int H, hipStream_t stream) {
  switch (K) {
    case 1: launch_step_keys<D, 1>(q, z, v, beta, history, taps, s_in, s_out, o, active, B, H, stream); break;
    case 2: launch_step_keys<D, 2>(q, z, v, beta, history, taps, s_in, s_out, o, active, B, H, stream); break;
    case 3: launch_step_keys<D, 3>(q, z, v, beta, history, taps, s_in, s_out, o, active, B, H, stream); break;
    case 4: launch_step_keys<D, 4>(q, z, v, beta, history, taps, s_in, s_out, o, active, B, H, stream); break;
    case 5: launch_step_keys<D, 5>(q, z, v, beta, history, taps, s_in, s_out, o, active, B, H, stream); break;
    case 6: launch_step_keys<D, 6>(q, z, v, beta, history, taps, s_in, s_out, o, active, B, H, stream); break;
    case 7: launch_step_keys<D, 7>(q, z, v, beta, history, taps, s_in, s_out, o, active, B, H, stream); break;
    default: launch_step_keys<D, 8>(q, z, v, beta, history, taps, s_in, s_out, o, active, B, H, stream); break;
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

extern "C" int vsp_delta_step_keys_bf16(const void* q, const void* z, const void* v, const void* beta, float* history,
                                        const float* taps, int K, const float* state_in, float* state_out, void* o,
                                        const uint8_t* active, int B, int H, int D, void* stream) {
  using namespace vsp;
  const char* who = "vsp_delta_step_keys_bf16";
  if (B < 0 || H < 1) return fail(ERR_ARG, "%s: bad sizes B=%d H=%d", who, B, H);
  if (D != 16 && D != 32 && D != 64 && D != 128)
    return fail(ERR_UNSUPPORTED, "%s: head dimension %d (kernels: 16, 32, 64, 128)", who, D);
  if (K < 1 || K > 8) return fail(ERR_UNSUPPORTED, "%s: filter width %d (kernels: 1..8)", who, K);
  if (B == 0) return OK;
  if (!q || !z || !v || !beta || !taps || !state_in || !state_out || !o || (K > 1 && !history))
    return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(taps) | reinterpret_cast<uintptr_t>(history) |
       reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out)) & 15)
    return fail(ERR_ARG, "%s: z, taps, history and the states must be 16-byte aligned", who);
  hipStream_t stream_h = reinterpret_cast<hipStream_t>(stream);
  const __bf16 *qb = static_cast<const __bf16*>(q), *zb = static_cast<const __bf16*>(z);
  const __bf16 *vb = static_cast<const __bf16*>(v), *bb = static_cast<const __bf16*>(beta);
  __bf16* ob = static_cast<__bf16*>(o);
  switch (D) {
    case 16: step_keys_by_width<16>(K, qb, zb, vb, bb, history, taps, state_in, state_out, ob, active, B, H, stream_h); break;
    case 32: step_keys_by_width<32>(K, qb, zb, vb, bb, history, taps, state_in, state_out, ob, active, B, H, stream_h); break;
    case 64: step_keys_by_width<64>(K, qb, zb, vb, bb, history, taps, state_in, state_out, ob, active, B, H, stream_h); break;
    default: step_keys_by_width<128>(K, qb, zb, vb, bb, history, taps, state_in, state_out, ob, active, B, H, stream_h); break;
  }
  return check_launch(who);
}
