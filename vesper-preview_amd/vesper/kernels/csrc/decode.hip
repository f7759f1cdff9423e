// Decoding on CDNA4 (gfx950): attention of one new token per row over a fixed-capacity KV ring.
//
// Semantics (reference vesper/attention.py:62-139, :298-338): a token at position p lives in slot
// p % W; slots are not in age order. The query at position p attends the ring slots that are valid
// and hold a position in (p - W, p], plus the new token itself, which is attended exactly once from
// its own argument; only then is the new token written into its slot. Query head h reads KV head
// h / (H / HKV); scale 1/sqrt(D).
//
// ring_attn_kernel (reads only): one workgroup per (b, KV head) serves the G = H / HKV query heads
// of that group, so each ring row is read from HBM once. D/8 lanes share a key row (16-byte loads);
// scores go to LDS, the softmax runs per head over W + 1 scores, and the weighted sum of V rows is
// reduced across lanes, then across waves.
// ring_write_kernel: writes the new keys, values, position and valid flag after every read of the
// step has finished (a separate launch on the same stream, so no workgroup can observe a slot half
// updated by another).
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kMaxGroup = 8;

template <typename T, int D>
__global__ __launch_bounds__(256) void ring_attn_kernel(const T* __restrict__ q, const T* __restrict__ knew,
                                                        const T* __restrict__ vnew, const int64_t* __restrict__ pos,
                                                        const T* __restrict__ ring_k, const T* __restrict__ ring_v,
                                                        const int64_t* __restrict__ ring_pos,
                                                        const uint8_t* __restrict__ ring_valid, T* __restrict__ o,
                                                        const uint8_t* __restrict__ active, int H, int HKV, int W,
                                                        float scale_log2) {
  constexpr int KL = D / 8;          // lanes per key row
  constexpr int KPP = 256 / KL;      // keys per pass of the workgroup
  extern __shared__ float ss[];      // [G][W + 1] scores, then probabilities
  __shared__ float sq[kMaxGroup][D];
  __shared__ float sred[4][kMaxGroup];
  __shared__ float sstat[2][kMaxGroup];
  __shared__ float sacc[4][kMaxGroup][D];

  const int b = blockIdx.x / HKV, kvh = blockIdx.x - b * HKV;
  const int G = H / HKV;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int part = tid % KL, kg = tid / KL;
  const int64_t p = pos[b];
  T* out = o + ((size_t)b * H + (size_t)kvh * G) * D;

  if (active != nullptr && active[b] == 0) {
    for (int i = tid; i < G * D; i += 256) out[i] = from_f32<T>(0.f);
    return;
  }
  for (int i = tid; i < G * D; i += 256) sq[i / D][i % D] = to_f32(q[((size_t)b * H + (size_t)kvh * G) * D + i]);
  __syncthreads();

  // scores of the ring slots
  const size_t row_stride = (size_t)HKV * D;
  const T* kb = ring_k + ((size_t)b * W * HKV + kvh) * D + 8 * part;
  for (int j = kg; j < W; j += KPP) {
    const int64_t rp = ring_pos[(size_t)b * W + j];
    const bool vis = ring_valid[(size_t)b * W + j] != 0 && rp <= p && rp > p - W;
    float kv8[8];
    load8_f32(kb + (size_t)j * row_stride, kv8);
    for (int gi = 0; gi < G; ++gi) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += kv8[e] * sq[gi][8 * part + e];
#pragma unroll
      for (int off = 1; off < KL; off <<= 1) acc += __shfl_xor(acc, off);
      if (part == 0) ss[gi * (W + 1) + j] = vis ? acc * scale_log2 : -INFINITY;
    }
  }
  // the new token's own score
  if (kg == 0) {
    float kv8[8];
    load8_f32(knew + ((size_t)b * HKV + kvh) * D + 8 * part, kv8);
    for (int gi = 0; gi < G; ++gi) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += kv8[e] * sq[gi][8 * part + e];
#pragma unroll
      for (int off = 1; off < KL; off <<= 1) acc += __shfl_xor(acc, off);
      if (part == 0) ss[gi * (W + 1) + W] = acc * scale_log2;
    }
  }
  __syncthreads();

  // softmax per head over W + 1 scores (the new token is always visible, so the max is finite)
  for (int gi = 0; gi < G; ++gi) {
    float* row = ss + gi * (W + 1);
    float m = -INFINITY;
    for (int j = tid; j <= W; j += 256) m = fmaxf(m, row[j]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) sred[wv][gi] = m;
  }
  __syncthreads();
  if (tid < G) sstat[0][tid] = fmaxf(fmaxf(sred[0][tid], sred[1][tid]), fmaxf(sred[2][tid], sred[3][tid]));
  __syncthreads();
  for (int gi = 0; gi < G; ++gi) {
    float* row = ss + gi * (W + 1);
    const float m = sstat[0][gi];
    float s = 0.f;
    for (int j = tid; j <= W; j += 256) {
      const float e = exp2f(row[j] - m);
      row[j] = e;
      s += e;
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) s += __shfl_xor(s, off);
    if (lane == 0) sred[wv][gi] = s;
  }
  __syncthreads();
  if (tid < G) sstat[1][tid] = (sred[0][tid] + sred[1][tid]) + (sred[2][tid] + sred[3][tid]);
  __syncthreads();

  // weighted values
  float acc[kMaxGroup][8];
#pragma unroll
  for (int gi = 0; gi < kMaxGroup; ++gi)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[gi][e] = 0.f;
  const T* vb = ring_v + ((size_t)b * W * HKV + kvh) * D + 8 * part;
  for (int j = kg; j < W; j += KPP) {
    float vv[8];
    load8_f32(vb + (size_t)j * row_stride, vv);
#pragma unroll
    for (int gi = 0; gi < kMaxGroup; ++gi) {
      if (gi < G) {
        const float pj = ss[gi * (W + 1) + j];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[gi][e] += pj * vv[e];
      }
    }
  }
  if (kg == 0) {
    float vv[8];
    load8_f32(vnew + ((size_t)b * HKV + kvh) * D + 8 * part, vv);
#pragma unroll
    for (int gi = 0; gi < kMaxGroup; ++gi) {
      if (gi < G) {
        const float pj = ss[gi * (W + 1) + W];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[gi][e] += pj * vv[e];
      }
    }
  }
  // reduce over the key groups of a wave, then over the four waves
#pragma unroll
  for (int gi = 0; gi < kMaxGroup; ++gi) {
    if (gi < G) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = acc[gi][e];
#pragma unroll
        for (int off = KL; off < 64; off <<= 1) x += __shfl_xor(x, off);
        acc[gi][e] = x;
      }
    }
  }
  if (lane < KL) {
#pragma unroll
    for (int gi = 0; gi < kMaxGroup; ++gi)
      if (gi < G)
#pragma unroll
        for (int e = 0; e < 8; ++e) sacc[wv][gi][8 * lane + e] = acc[gi][e];
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += 256) {
    const int gi = i / D, d = i - gi * D;
    const float sum = (sacc[0][gi][d] + sacc[1][gi][d]) + (sacc[2][gi][d] + sacc[3][gi][d]);
    out[i] = from_f32<T>(sum / sstat[1][gi]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ring_write_kernel(const T* __restrict__ knew, const T* __restrict__ vnew,
                                                         const int64_t* __restrict__ pos, T* __restrict__ ring_k,
                                                         T* __restrict__ ring_v, int64_t* __restrict__ ring_pos,
                                                         uint8_t* __restrict__ ring_valid, int HKV, int D, int W) {
  const int b = blockIdx.x;
  const int64_t p = pos[b];
  if (p < 0) return;  // refused by the host wrapper; never index with a negative slot
  const int slot = (int)(p % W);
  const size_t dst = ((size_t)b * W + slot) * HKV * D;
  const size_t src = (size_t)b * HKV * D;
  for (int i = threadIdx.x; i < HKV * D; i += blockDim.x) {
    ring_k[dst + i] = knew[src + i];
    ring_v[dst + i] = vnew[src + i];
  }
  if (threadIdx.x == 0) {
    ring_pos[(size_t)b * W + slot] = p;
    ring_valid[(size_t)b * W + slot] = 1;
  }
}

bool ring_width(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }

template <typename T>
int ring_attn(const T* q, const T* knew, const T* vnew, const int64_t* pos, T* ring_k, T* ring_v, int64_t* ring_pos,
              uint8_t* ring_valid, T* o, const uint8_t* active, int B, int H, int HKV, int D, int W, float scale,
              int write, void* stream_ptr, const char* who) {
  if (B < 0 || H < 1 || HKV < 1 || W < 1) return fail(ERR_ARG, "%s: bad sizes B=%d H=%d HKV=%d W=%d", who, B, H, HKV, W);
  if (H % HKV != 0) return fail(ERR_ARG, "%s: %d query heads are not a multiple of %d KV heads", who, H, HKV);
  if (H / HKV > kMaxGroup) return fail(ERR_UNSUPPORTED, "%s: %d query heads per KV head (at most %d)", who, H / HKV, kMaxGroup);
  if (!ring_width(D)) return fail(ERR_UNSUPPORTED, "%s: head dimension %d (kernels: 16, 32, 64, 128)", who, D);
  const size_t smem = (size_t)(H / HKV) * (W + 1) * sizeof(float);
  if (smem > 96 * 1024) return fail(ERR_UNSUPPORTED, "%s: window %d with %d heads per group needs %zu bytes of LDS", who, W, H / HKV, smem);
  if (B == 0) return OK;
  if (!q || !knew || !vnew || !pos || !ring_k || !ring_v || !ring_pos || !ring_valid || !o)
    return fail(ERR_ARG, "%s: null pointer", who);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  const float scale_log2 = scale * 1.4426950408889634f;
  dim3 grid((unsigned)(B * HKV));
  switch (D) {
    case 16: hipLaunchKernelGGL((ring_attn_kernel<T, 16>), grid, dim3(256), smem, stream, q, knew, vnew, pos, ring_k, ring_v, ring_pos, ring_valid, o, active, H, HKV, W, scale_log2); break;
    case 32: hipLaunchKernelGGL((ring_attn_kernel<T, 32>), grid, dim3(256), smem, stream, q, knew, vnew, pos, ring_k, ring_v, ring_pos, ring_valid, o, active, H, HKV, W, scale_log2); break;
    case 64: hipLaunchKernelGGL((ring_attn_kernel<T, 64>), grid, dim3(256), smem, stream, q, knew, vnew, pos, ring_k, ring_v, ring_pos, ring_valid, o, active, H, HKV, W, scale_log2); break;
    default: hipLaunchKernelGGL((ring_attn_kernel<T, 128>), grid, dim3(256), smem, stream, q, knew, vnew, pos, ring_k, ring_v, ring_pos, ring_valid, o, active, H, HKV, W, scale_log2); break;
  }
  int st = check_launch(who);
  if (st != OK || !write) return st;
  hipLaunchKernelGGL((ring_write_kernel<T>), dim3((unsigned)B), dim3(256), 0, stream, knew, vnew, pos, ring_k, ring_v,
                     ring_pos, ring_valid, HKV, D, W);
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_ring_attn_bf16(const void* q, const void* k, const void* v, const int64_t* pos, void* ring_k,
                                  void* ring_v, int64_t* ring_pos, uint8_t* ring_valid, void* o,
                                  const uint8_t* active, int B, int H, int HKV, int D, int window, float scale,
                                  int write, void* stream) {
  return vsp::ring_attn<__bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                                static_cast<const __bf16*>(v), pos, static_cast<__bf16*>(ring_k),
                                static_cast<__bf16*>(ring_v), ring_pos, ring_valid, static_cast<__bf16*>(o), active, B,
                                H, HKV, D, window, scale, write, stream, "vsp_ring_attn_bf16");
}

extern "C" int vsp_ring_attn_f16(const void* q, const void* k, const void* v, const int64_t* pos, void* ring_k,
                                 void* ring_v, int64_t* ring_pos, uint8_t* ring_valid, void* o, const uint8_t* active,
                                 int B, int H, int HKV, int D, int window, float scale, int write, void* stream) {
  return vsp::ring_attn<_Float16>(static_cast<const _Float16*>(q), static_cast<const _Float16*>(k),
                                  static_cast<const _Float16*>(v), pos, static_cast<_Float16*>(ring_k),
                                  static_cast<_Float16*>(ring_v), ring_pos, ring_valid, static_cast<_Float16*>(o),
                                  active, B, H, HKV, D, window, scale, write, stream, "vsp_ring_attn_f16");
}
