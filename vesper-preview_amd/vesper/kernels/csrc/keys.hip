// The causal key filter and key normalization on CDNA4 (gfx950): the step before the scan.
//
// Semantics (reference vesper/column.py:255-289, computed on CUDA by vesper/kernels/keys.py:28-32):
// u[t, j] = sum_{r < K} taps[r, j] * z[t - r, j] (depthwise, r = 0 the current token, positions
// before the chunk from history [B, K-1, D], oldest first, float32), then per head of width hd the
// key normalize_keys(u) = s / max(||s||, 1) with s = u / max(max_j |u_j|, 1e-6)
// (vesper/recurrence.py:91-115), returned in z's dtype.
//
// HBM-bound: z is read once (plus a (K-1)-row halo per run of tokens, mostly from L2) and the key
// written once. A lane owns 8 consecutive features (16-byte loads at bf16); a wave walks a run of
// consecutive tokens, keeping the previous K-1 input rows in registers; a head's hd / 8 lanes
// reduce its maximum and squared norm by DPP / permlane exchanges.
#include "keys_rows.h"
#include "keys_backward.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

// A wave owns a run of Row8<TZ>::kRun consecutive tokens of one batch row and 64 segments of 8
// features. Every load of the run (its rows, the K - 1 rows before it, the taps) is issued before
// the first use, so a wave keeps its whole run in flight: the kernel is bound by HBM bandwidth,
// not by one row's latency per token. z and the keys go through buffer resources over one batch
// row: the token's row offset is scalar, and a lane past D gets a vector offset beyond the range,
// so its reads return zeros and its writes are dropped (whole heads idle together: D is a multiple
// of the head width).
// CARRY (copy-forward of halted tokens' key inputs, vesper/column.py:779-782): token t's input row
// is zc's row t where active[b, t] == 0, z's row t elsewhere; the rows before the chunk always
// come from the history. A row's source is wave-uniform (all lanes of a wave hold one token), so
// both are loaded, the unused one from past its range, and joined bitwise.
template <typename TZ, int K, int LPH, bool CARRY>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void key_filter_kernel(const TZ* __restrict__ z, const float* history,
                                                         const float* __restrict__ taps, TZ* __restrict__ out,
                                                         const uint8_t* __restrict__ active, const TZ* zc,
                                                         float* hist_out, int N, int D) {
  using Row = Row8<TZ>;
  constexpr int RUN = Row::kRun;
  static_assert(RUN >= K - 1, "a run is at least as long as the filter's history");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
  const int b = blockIdx.z;
  const int f0 = 8 * (64 * blockIdx.x + l);  // this lane's first feature
  const bool on = f0 < D;
  const int t_begin = RUN * (4 * blockIdx.y + wave);
  if (t_begin >= N) return;  // whole waves only: no workgroup barrier in this kernel
  const unsigned row_bytes = (unsigned)D * sizeof(TZ);
  const unsigned batch_bytes = (unsigned)N * row_bytes;  // below 2^31: the host refuses more
  const auto rz = buffer_rsrc(z + (size_t)b * N * D, batch_bytes);
  const auto ro = buffer_rsrc(out + (size_t)b * N * D, batch_bytes);
  constexpr unsigned kPast = 0x80000000u;  // a vector offset past every range (ranges stay below 2^31)
  const unsigned voff = on ? (unsigned)f0 * sizeof(TZ) : kPast;
  const int fl = on ? f0 : 0;  // taps: idle lanes read feature 0's (never stored)
  // CARRY: lane j holds the flag of token t_begin - (K - 1) + j (clamped into the batch row), so
  // row t's flag is lane t - t_begin + K - 1 of it, read into a scalar
  const auto rzc = buffer_rsrc(CARRY ? zc + (size_t)b * N * D : z, batch_bytes);
  int flags = 1;
  if constexpr (CARRY) flags = active[(size_t)b * N + min(max(t_begin - (K - 1) + l, 0), N - 1)];
  auto load_row = [&](unsigned v, unsigned soff, int lane_of_flag) {
    if constexpr (!CARRY) {
      return Row::load(rz, v, soff);
    } else {
      const bool fresh = __builtin_amdgcn_readlane(flags, lane_of_flag) != 0;
      return Row::join(Row::load(rz, fresh ? v : kPast, soff), Row::load(rzc, fresh ? kPast : v, soff));
    }
  };

  // Loads in the order of use (vmcnt counts in issue order): the taps, the K - 1 rows before the
  // run, then the run's rows, so token i waits only for its own row.
  float tp[K][8];
#pragma unroll
  for (int r = 0; r < K; ++r) {
    const f32x4 t0 = *reinterpret_cast<const f32x4*>(taps + (size_t)r * D + fl);
    const f32x4 t1 = *reinterpret_cast<const f32x4*>(taps + (size_t)r * D + fl + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tp[r][e] = t0[e];
      tp[r][4 + e] = t1[e];
    }
  }
  // The rows before the run come from z, or for the batch row's first run (the run is at least
  // K - 1 tokens long) all from the history. Both are loaded without a branch, the unused one from
  // past its range (zeros), and joined bitwise: exact, signed zeros included.
  float win[K > 1 ? K - 1 : 1][8];  // win[r - 1] = input row t - r
  if constexpr (K > 1) {
    const bool first = t_begin == 0;
    const auto rh = buffer_rsrc(history + (size_t)b * (K - 1) * D, (unsigned)(K - 1) * D * 4u);
    const unsigned vz = first ? kPast : voff;
    const unsigned vh = (first && on) ? (unsigned)f0 * 4u : kPast;
#pragma unroll
    for (int r = 1; r < K; ++r) {
      float zr[8], hr[8];
      Row::unpack(load_row(vz, first ? 0u : (unsigned)(t_begin - r) * row_bytes, K - 1 - r), zr);
      Row8<float>::unpack(Row8<float>::load(rh, vh, (unsigned)(K - 1 - r) * D * 4u), hr);
#pragma unroll
      for (int e = 0; e < 8; ++e) win[r - 1][e] = __uint_as_float(__float_as_uint(zr[e]) | __float_as_uint(hr[e]));
    }
    // The next history may be the history itself (a chunk within one run: then this wave alone
    // reads and writes these features of the batch row); its rows were all read into win above, so
    // every load has to land before the first store.
    if (hist_out == history && hist_out != nullptr) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      asm volatile("" ::: "memory");
    }
    // The next history (the newest K - 1 inputs of history and chunk): a chunk shorter than K - 1
    // keeps the history's rows N .. K - 2 first, written here from win (win[r - 1] holds history
    // row K - 1 - r in the chunk's first run) by the run at the chunk's start; the chunk's own rows
    // follow from the run loop below.
    if (hist_out != nullptr && first && N < K - 1 && on) {
      float* dst = hist_out + (size_t)b * (K - 1) * D + f0;
#pragma unroll
      for (int i = 0; i < K - 1; ++i) {
        const int r = K - 2 - i - N;  // history row K - 2 - i lands in row r of the next one
        if (r >= 0) {
          *reinterpret_cast<f32x4*>(dst + (size_t)r * D) = f32x4{win[i][0], win[i][1], win[i][2], win[i][3]};
          *reinterpret_cast<f32x4*>(dst + (size_t)r * D + 4) = f32x4{win[i][4], win[i][5], win[i][6], win[i][7]};
        }
      }
    }
  }
  typename Row::Raw raw[RUN];  // rows past N (a short last run) re-read row N - 1
#pragma unroll
  for (int i = 0; i < RUN; ++i) raw[i] = load_row(voff, (unsigned)min(t_begin + i, N - 1) * row_bytes, K - 1 + i);

#pragma unroll
  for (int i = 0; i < RUN; ++i) {
    const int t = t_begin + i;  // past N in a short last run: computed, the store dropped
    float cur[8];
    Row::unpack(raw[i], cur);
    if constexpr (K > 1) {
      // the chunk's last K - 1 inputs (as read: carried ones for inactive tokens) into the next history
      const int r = t - (N - (K - 1));
      if (hist_out != nullptr && on && t < N && r >= 0) {
        float* dst = hist_out + ((size_t)b * (K - 1) + r) * D + f0;
        *reinterpret_cast<f32x4*>(dst) = f32x4{cur[0], cur[1], cur[2], cur[3]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{cur[4], cur[5], cur[6], cur[7]};
      }
    }
    // the filter in the reference's order: taps[0] z[t], then + taps[r] z[t - r] for r = 1, 2, ...
    float u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = tp[0][e] * cur[e];
#pragma unroll
      for (int r = 1; r < K; ++r) acc = acc + tp[r][e] * win[r - 1][e];
      u[e] = acc;
    }
#pragma unroll
    for (int r = K - 1; r >= 2; --r)
#pragma unroll
      for (int e = 0; e < 8; ++e) win[r - 1][e] = win[r - 2][e];
    if constexpr (K > 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[0][e] = cur[e];
    }
    // normalize_keys per head: s = u / max(peak, floor), key = s / sqrt(max(|s|^2, 1)). The first
    // division is a reciprocal (v_rcp, 1 ulp) refined by one Newton step on the residual
    // (r = u - s0 * scale by FMA, s = s0 + r / scale), which gives the correctly rounded quotient
    // here: the peak component of a row scales to exactly 1 and a row under the floor to exactly
    // u / 1e-6, as the reference's division does. The second is v_rsq (1 ulp) times the 8
    // features, far inside float32's 2e-5 bound, and exact where the norm is floored at one.
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
#pragma unroll
    for (int e = 0; e < 8; ++e) u[e] = u[e] * inv_den;
    // The row offset goes in the vector offset with soffset 0. With a register soffset the
    // compiler inserts no wait state between a store of more than 8 bytes and a VALU write of its
    // data registers, and on gfx950 that write then reached the store's first dword (in lanes
    // 12..15 of each row of 16); with soffset 0 the wait state is inserted.
    Row::store(ro, (t < N ? voff : kPast) + (unsigned)min(t, N - 1) * row_bytes, 0u, u);
  }
}

template <typename TZ, int K, bool CARRY>
void launch_k(const TZ* z, const float* history, const float* taps, TZ* out, const uint8_t* active, const TZ* zc,
              float* hist_out, int B, int N, int D, int hd, hipStream_t stream) {
  constexpr int per_block = 4 * Row8<TZ>::kRun;
  dim3 grid((unsigned)((D / 8 + 63) / 64), (unsigned)((N + per_block - 1) / per_block), (unsigned)B);
#define VSP_KEY_LAUNCH(LPH)                                                                                          \
  hipLaunchKernelGGL((key_filter_kernel<TZ, K, LPH, CARRY>), grid, dim3(256), 0, stream, z, history, taps, out, active, \
                     zc, hist_out, N, D)
  switch (hd / 8) {
    case 1: VSP_KEY_LAUNCH(1); break;
    case 2: VSP_KEY_LAUNCH(2); break;
    case 4: VSP_KEY_LAUNCH(4); break;
    case 8: VSP_KEY_LAUNCH(8); break;
    case 16: VSP_KEY_LAUNCH(16); break;
    case 32: VSP_KEY_LAUNCH(32); break;
    default: VSP_KEY_LAUNCH(64); break;
  }
#undef VSP_KEY_LAUNCH
}

template <typename TZ, int K>
void launch_k(const TZ* z, const float* history, const float* taps, TZ* out, const uint8_t* active, const TZ* zc,
              float* hist_out, int B, int N, int D, int hd, hipStream_t stream) {
  if (zc != nullptr)
    launch_k<TZ, K, true>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream);
  else
    launch_k<TZ, K, false>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream);
}

template <typename TZ>
int key_filter(const TZ* z, const float* history, const float* taps, TZ* out, int B, int N, int D, int heads, int K,
               void* stream_ptr, const char* who, const uint8_t* active = nullptr, const TZ* zc = nullptr,
               float* hist_out = nullptr) {
  if (B < 0 || N < 0 || D < 1 || heads < 1) return fail(ERR_ARG, "%s: bad sizes B=%d N=%d D=%d heads=%d", who, B, N, D, heads);
  if (K < 1 || K > 8) return fail(ERR_UNSUPPORTED, "%s: filter width %d (kernels: 1..8)", who, K);
  if (D % heads != 0) return fail(ERR_ARG, "%s: %d features are not a multiple of %d heads", who, D, heads);
  const int hd = D / heads;
  if (hd < 8 || hd > 512 || (hd & (hd - 1)) != 0)
    return fail(ERR_UNSUPPORTED, "%s: head width %d (kernels: powers of two 8..512)", who, hd);
  if (B == 0 || N == 0) return OK;
  if (!z || !taps || !out || (K > 1 && !history)) return fail(ERR_ARG, "%s: null pointer", who);
  if ((N + 4 * Row8<TZ>::kRun - 1) / (4 * Row8<TZ>::kRun) > 65535 || B > 65535)
    return fail(ERR_UNSUPPORTED, "%s: %d tokens in %d batch rows exceed the launch grid", who, N, B);
  if ((size_t)N * D * sizeof(TZ) > 0x7FFFFFF0u)
    return fail(ERR_UNSUPPORTED, "%s: %d tokens of %d features exceed 2 GiB in one batch row", who, N, D);
  if ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(taps) |
       reinterpret_cast<uintptr_t>(history)) & 15)
    return fail(ERR_ARG, "%s: z, history, taps and the output must be 16-byte aligned", who);
  if (zc != nullptr && (!active || (reinterpret_cast<uintptr_t>(zc) & 15)))
    return fail(ERR_ARG, "%s: carried key inputs need the active flags and 16-byte alignment", who);
  if (hist_out != nullptr && K > 1) {
    const size_t bytes = (size_t)B * (K - 1) * D * sizeof(float);
    const uintptr_t o = reinterpret_cast<uintptr_t>(hist_out), h0 = reinterpret_cast<uintptr_t>(history);
    if (o & 15) return fail(ERR_ARG, "%s: the next history must be 16-byte aligned", who);
    // in place only where one run holds a batch row's tokens (one wave reads and writes each feature)
    if (o == h0 ? N > Row8<TZ>::kRun : (o < h0 + bytes && h0 < o + bytes))
      return fail(ERR_ARG, "%s: the next history overlaps the history (in place: at most %d tokens)", who,
                  Row8<TZ>::kRun);
  }
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  switch (K) {
    case 1: launch_k<TZ, 1>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream); break;
    case 2: launch_k<TZ, 2>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream); break;
    case 3: launch_k<TZ, 3>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream); break;
    case 4: launch_k<TZ, 4>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream); break;
    case 5: launch_k<TZ, 5>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream); break;
    case 6: launch_k<TZ, 6>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream); break;
    case 7: launch_k<TZ, 7>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream); break;
    default: launch_k<TZ, 8>(z, history, taps, out, active, zc, hist_out, B, N, D, hd, stream); break;
  }
  return check_launch(who);
}

// out[c] = sum over r < rows of in[r, c], 16 columns per workgroup: 64 row groups (one per lane of
// a wave's worth of threads per column quad) each add the rows g, g + 64, g + 128, ... in order,
// eight loads issued before their adds; then groups 0..7 each add eight group sums (g, g + 8, ...)
// and group 0 adds those eight, all in a fixed order for a shape (deterministic).
__global__ __launch_bounds__(256) void tap_sum_kernel(const float* __restrict__ in, float* __restrict__ out, int rows,
                                                      int cols) {
  constexpr int kGroups = 64, kBatch = 8;
  __shared__ f32x4 part[kGroups][4];
  const int cq = threadIdx.x & 3, rg = threadIdx.x >> 2;
  const int c = 4 * (4 * blockIdx.x + cq);
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if (c < cols) {
    int r = rg;
    for (; r + (kBatch - 1) * kGroups < rows; r += kBatch * kGroups) {
      f32x4 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) v[u] = *reinterpret_cast<const f32x4*>(in + (size_t)(r + u * kGroups) * cols + c);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) s += v[u];
    }
    for (; r < rows; r += kGroups) s += *reinterpret_cast<const f32x4*>(in + (size_t)r * cols + c);
  }
  part[rg][cq] = s;
  __syncthreads();
  if (rg < 8) {
    f32x4 t = part[rg][cq];
#pragma unroll
    for (int g = 1; g < 8; ++g) t += part[rg + 8 * g][cq];
    part[rg][cq] = t;  // only group rg reads or writes row rg here
  }
  __syncthreads();
  if (rg == 0 && c < cols) {
    f32x4 t = part[0][cq];
#pragma unroll
    for (int g = 1; g < 8; ++g) t += part[g][cq];
    *reinterpret_cast<f32x4*>(out + c) = t;
  }
}

__global__ __launch_bounds__(256) void zero_fill_kernel(float* __restrict__ p, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

}  // namespace

size_t key_backward_parts(int B, int N) {
  return (size_t)B * (size_t)((N + kBackRun * kBackWaves - 1) / (kBackRun * kBackWaves));
}

size_t key_backward_workspace(int B, int N, int D, int K) {
  if (B <= 0 || N <= 0 || D <= 0 || K < 1) return 0;
  return key_backward_parts(B, N) * (size_t)K * D * sizeof(float);
}

// No token: the taps' and the history's gradients are zero (fill kernels, capturable).
int key_backward_empty(float* grad_taps, float* grad_history, int B, int D, int K, hipStream_t stream, const char* who) {
  const size_t cols = (size_t)K * D;
  hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((cols + 255) / 256)), dim3(256), 0, stream, grad_taps, cols);
  const size_t nh = (size_t)B * (K - 1) * D;
  if (grad_history && nh)
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((nh + 255) / 256)), dim3(256), 0, stream, grad_history, nh);
  return check_launch(who);
}

// The workgroups' partials of the taps' gradient summed into grad_taps in one pass, in a fixed order.
int key_backward_sum_taps(float* partial, float* grad_taps, int B, int N, int D, int K, hipStream_t stream,
                          const char* who) {
  const size_t cols = (size_t)K * D;
  const int parts = (int)key_backward_parts(B, N);
  hipLaunchKernelGGL(tap_sum_kernel, dim3((unsigned)((cols + 15) / 16)), dim3(256), 0, stream, partial, grad_taps,
                     parts, (int)cols);
  return check_launch(who);
}

}  // namespace vsp


extern "C" int vsp_key_filter_bf16(const void* z, const float* history, const float* taps, void* keys, int B, int N,
                                   int D, int heads, int K, void* stream) {
  return vsp::key_filter<__bf16>(static_cast<const __bf16*>(z), history, taps, static_cast<__bf16*>(keys), B, N, D,
                                 heads, K, stream, "vsp_key_filter_bf16");
}

extern "C" int vsp_key_filter_f16(const void* z, const float* history, const float* taps, void* keys, int B, int N,
                                  int D, int heads, int K, void* stream) {
  return vsp::key_filter<_Float16>(static_cast<const _Float16*>(z), history, taps, static_cast<_Float16*>(keys), B, N,
                                   D, heads, K, stream, "vsp_key_filter_f16");
}

extern "C" int vsp_key_filter_f32(const float* z, const float* history, const float* taps, float* keys, int B, int N,
                                  int D, int heads, int K, void* stream) {
  return vsp::key_filter<float>(z, history, taps, keys, B, N, D, heads, K, stream, "vsp_key_filter_f32");
}

extern "C" size_t vsp_key_filter_backward_workspace_bytes(int B, int N, int D, int K) {
  return vsp::key_backward_workspace(B, N, D, K);
}

extern "C" int vsp_key_step_bf16(const void* z, const void* z_carried, const uint8_t* active, const float* history,
                                 const float* taps, void* keys, float* history_out, int B, int N, int D, int heads,
                                 int K, void* stream) {
  return vsp::key_filter<__bf16>(static_cast<const __bf16*>(z), history, taps, static_cast<__bf16*>(keys), B, N, D,
                                 heads, K, stream, "vsp_key_step_bf16", active, static_cast<const __bf16*>(z_carried),
                                 history_out);
}

extern "C" int vsp_key_step_f16(const void* z, const void* z_carried, const uint8_t* active, const float* history,
                                const float* taps, void* keys, float* history_out, int B, int N, int D, int heads,
                                int K, void* stream) {
  return vsp::key_filter<_Float16>(static_cast<const _Float16*>(z), history, taps, static_cast<_Float16*>(keys), B, N,
                                   D, heads, K, stream, "vsp_key_step_f16", active,
                                   static_cast<const _Float16*>(z_carried), history_out);
}

extern "C" int vsp_key_step_f32(const float* z, const float* z_carried, const uint8_t* active, const float* history,
                                const float* taps, float* keys, float* history_out, int B, int N, int D, int heads,
                                int K, void* stream) {
  return vsp::key_filter<float>(z, history, taps, keys, B, N, D, heads, K, stream, "vsp_key_step_f32", active,
                                z_carried, history_out);
}
