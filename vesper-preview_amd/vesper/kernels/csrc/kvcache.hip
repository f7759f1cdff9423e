// The chronological attention window carried across chunks on CDNA4 (gfx950): one launch per push.
//
// Reference: vesper/attention.py:142-175 (`kv_cache_push`): after a chunk of n tokens the cache
// holds the newest min(m + n, w) entries of (cache, chunk), oldest first, at exactly that size:
// the last keep_old = min(m, w - keep_new) cache rows, then the last keep_new = min(n, w) chunk
// rows. Here one kernel writes the new keys, values and positions together: one wave per output
// row, 16-byte pieces where the rows allow (else 2-byte elements).
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

template <typename U>
__global__ __launch_bounds__(256) void kv_push_kernel(const U* __restrict__ ck, const U* __restrict__ cv,
                                                      const int64_t* __restrict__ cpos, const U* __restrict__ k,
                                                      const U* __restrict__ v, const int64_t* __restrict__ pos,
                                                      U* __restrict__ ok, U* __restrict__ ov, int64_t* __restrict__ opos,
                                                      int B, int M, int N, int keep_old, int keep_new, int units) {
  const int keep = keep_old + keep_new;
  const int r = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= B * keep) return;
  const int b = r / keep, i = r - b * keep;
  const bool old = i < keep_old;
  const size_t src = old ? (size_t)b * M + (M - keep_old + i) : (size_t)b * N + (N - keep_new + (i - keep_old));
  const U* sk = (old ? ck : k) + src * units;
  const U* sv = (old ? cv : v) + src * units;
  for (int u = lane; u < units; u += 64) {
    ok[(size_t)r * units + u] = sk[u];
    ov[(size_t)r * units + u] = sv[u];
  }
  if (lane == 0) opos[r] = (old ? cpos : pos)[src];
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_kv_cache_push(const void* cache_k, const void* cache_v, const int64_t* cache_pos, const void* k,
                                 const void* v, const int64_t* pos, void* out_k, void* out_v, int64_t* out_pos, int B,
                                 int M, int N, int HKV, int D, int elem_bytes, int window, void* stream) {
  using namespace vsp;
  const char* who = "vsp_kv_cache_push";
  if (B < 0 || M < 0 || N < 0 || HKV < 1 || D < 1 || window < 1 || M > window)
    return fail(ERR_ARG, "%s: sizes B=%d M=%d N=%d HKV=%d D=%d window=%d", who, B, M, N, HKV, D, window);
  if (elem_bytes != 2 && elem_bytes != 4) return fail(ERR_ARG, "%s: element size %d", who, elem_bytes);
  const int keep_new = N < window ? N : window;
  const int keep_old = M < window - keep_new ? M : window - keep_new;
  const int keep = keep_old + keep_new;
  if (B == 0 || keep == 0) return OK;
  if ((keep_old && (!cache_k || !cache_v || !cache_pos)) || (keep_new && (!k || !v || !pos)) || !out_k || !out_v ||
      !out_pos)
    return fail(ERR_ARG, "%s: null pointer", who);
  const size_t row_bytes = (size_t)HKV * D * elem_bytes;
  const uintptr_t mix = reinterpret_cast<uintptr_t>(cache_k) | reinterpret_cast<uintptr_t>(cache_v) |
                        reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                        reinterpret_cast<uintptr_t>(out_k) | reinterpret_cast<uintptr_t>(out_v) | row_bytes;
  const dim3 grid((unsigned)(((size_t)B * keep + 3) / 4));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if ((mix & 15) == 0) {
    hipLaunchKernelGGL(kv_push_kernel<uint4>, grid, dim3(256), 0, s, static_cast<const uint4*>(cache_k),
                       static_cast<const uint4*>(cache_v), cache_pos, static_cast<const uint4*>(k),
                       static_cast<const uint4*>(v), pos, static_cast<uint4*>(out_k), static_cast<uint4*>(out_v),
                       out_pos, B, M, N, keep_old, keep_new, (int)(row_bytes / 16));
  } else {
    hipLaunchKernelGGL(kv_push_kernel<uint16_t>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(cache_k),
                       static_cast<const uint16_t*>(cache_v), cache_pos, static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(v), pos, static_cast<uint16_t*>(out_k),
                       static_cast<uint16_t*>(out_v), out_pos, B, M, N, keep_old, keep_new, (int)(row_bytes / 2));
  }
  return check_launch(who);
}
