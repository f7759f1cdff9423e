// HBM streaming probes on CDNA4 (gfx950): what a plain read, copy or fill of device memory reaches.
//
// Measurement only (bench.py --hbm-ceiling): the bandwidth-bound kernels of the library are judged
// against what the memory system gives to the simplest possible access pattern, not only against
// the nominal 8 TB/s. Each kernel walks the buffer in 16-byte pieces, a grid-stride loop with U
// independent pieces per thread in flight (all U loads are issued before any is used), 256 threads
// a workgroup. The read probe folds what it reads into one word per thread and stores it only when
// it equals a value the data never holds, so the loads cannot be dropped and nothing is written.
// Not part of the mixers' C ABI: built into its own library, libvesper_probe.so.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT, typename P> __device__ __forceinline__ u32x4 ld(const P* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT, typename P> __device__ __forceinline__ void st(const u32x4& x, P* p) {
  if constexpr (NT) __builtin_nontemporal_store(x, p);
  else *p = x;
}

template <int U, bool NT>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, size_t n,
                                                          uint32_t* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (U - 1) * stride < n; i += U * stride) {
    u32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = ld<NT>(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= x[u].x ^ x[u].y ^ x[u].z ^ x[u].w;
  }
  for (; i < n; i += stride) {
    const u32x4 x = src[i];
    acc ^= x.x ^ x.y ^ x.z ^ x.w;
  }
  if (acc == 0x9E3779B9u) sink[(size_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

template <int U, bool NT>
__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                          size_t n) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + (U - 1) * stride < n; i += U * stride) {
    u32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = ld<NT>(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) st<NT>(x[u], dst + i + u * stride);
  }
  for (; i < n; i += stride) dst[i] = src[i];
}

template <bool NT>
__global__ __launch_bounds__(256) void stream_fill_kernel(u32x4* __restrict__ dst, size_t n, uint32_t value) {
  const size_t stride = (size_t)gridDim.x * 256;
  const u32x4 x = {value, value, value, value};
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) st<NT>(x, dst + i);
}

}  // namespace

// mode 0: read `bytes` of src (sink: one uint32 per thread of the grid, blocks * 256, never
// written in practice); mode 1: copy src to dst; mode 2: fill dst; modes 3, 4, 5: the same with
// nontemporal loads and stores. bytes a multiple of 16, src and dst 16-byte aligned; blocks >= 1.
// Returns 0, or 1 on a bad argument, 3 on a launch error.
extern "C" int vsp_probe_stream(int mode, const void* src, void* dst, size_t bytes, int blocks, void* stream) {
  if (blocks < 1 || mode < 0 || mode > 5 || (bytes & 15) ||
      ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15))
    return 1;
  if (!dst || (mode % 3 != 2 && !src)) return 1;
  const size_t n = bytes / 16;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)blocks), block(256);
  const u32x4* in = static_cast<const u32x4*>(src);
  u32x4* out = static_cast<u32x4*>(dst);
  switch (mode) {
    case 0: hipLaunchKernelGGL((stream_read_kernel<8, false>), grid, block, 0, s, in, n, reinterpret_cast<uint32_t*>(out)); break;
    case 1: hipLaunchKernelGGL((stream_copy_kernel<4, false>), grid, block, 0, s, in, out, n); break;
    case 2: hipLaunchKernelGGL((stream_fill_kernel<false>), grid, block, 0, s, out, n, 0x3F800000u); break;
    case 3: hipLaunchKernelGGL((stream_read_kernel<8, true>), grid, block, 0, s, in, n, reinterpret_cast<uint32_t*>(out)); break;
    case 4: hipLaunchKernelGGL((stream_copy_kernel<4, true>), grid, block, 0, s, in, out, n); break;
    default: hipLaunchKernelGGL((stream_fill_kernel<true>), grid, block, 0, s, out, n, 0x3F800000u); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 3;
}
