// Rotary position embedding on CDNA4 (gfx950): the attention's queries and keys rotated in one launch.
//
// Reference: vesper/attention.py:178-217 (`rotary`) as `WindowedAttention.project` applies it to q
// and k (attention.py:292): pairs (x[2j], x[2j+1]) of a token at position p turn by
// p * base^(-2j/dk); the angle is computed in float64, only cos and sin are cast to the
// activations' dtype, and the rotation x1 cos - x2 sin, x1 sin + x2 cos is computed in that dtype
// (each product and the sum rounded to it, as torch evaluates it). The inverse frequencies
// base^(-2j/dk) arrive as a float64 table the host computed exactly as the reference does.
//
// A workgroup takes four token rows (b, n): first its threads compute each (row, pair)'s cos and
// sin once into LDS (the float64 part), then the rows' query and key heads are cut into pieces of
// consecutive pairs (16 bytes where the head width and alignment allow, else one pair), each an
// independent piece of work spread over all 256 threads, consecutive threads on consecutive
// pieces, four pieces' loads issued before their arithmetic. q and k may be rotated in
// place (each element is read and written by one thread).
#include "common.h"
#include "rotary_math.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

// PP consecutive pairs of one head as one vector access (16 bytes where the rows allow it)
template <typename T, int PP> struct Pieces {
  typedef T V __attribute__((ext_vector_type(2 * PP)));
};

constexpr int kRotRows = 4;  // token rows a workgroup

template <typename T, int PP>
__global__ __launch_bounds__(256) void rotary_qk_kernel(const T* q, const T* k, const int64_t* __restrict__ pos,
                                                        const double* __restrict__ inv_freq, T* qo, T* ko, int rows,
                                                        int H, int HKV, int D) {
  __shared__ T cs[kRotRows][512], sn[kRotRows][512];
  const int half = D / 2, row0 = blockIdx.x * kRotRows;
  const int nrows = min(kRotRows, rows - row0);
  // piece t: row r = t / (heads * groups), head hh, pairs PP g .. PP g + PP - 1 (heads: the H query
  // heads, then the HKV key heads)
  typedef typename Pieces<T, PP>::V V;
  const int groups = half / PP, heads = H + HKV, per_row = heads * groups, total = nrows * per_row;
  V xv[4];
  size_t off[4];
  bool isq[4];
  int rr[4], jj[4];
  auto load_round = [&](int t0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = min(t0 + 256 * u, total - 1);
      const int r = t / per_row, rem = t - r * per_row, hh = rem / groups, j = PP * (rem - hh * groups);
      isq[u] = hh < H;
      off[u] = isq[u] ? ((size_t)(row0 + r) * H + hh) * D + 2 * j : ((size_t)(row0 + r) * HKV + (hh - H)) * D + 2 * j;
      rr[u] = r;
      jj[u] = j;
      xv[u] = *reinterpret_cast<const V*>((isq[u] ? q : k) + off[u]);
    }
  };
  load_round(threadIdx.x);  // the first pieces' loads do not wait for the cos and sin
  for (int e = threadIdx.x; e < nrows * half; e += 256) {
    const int r = e / half, j = e - r * half;
    const double angle = (double)pos[row0 + r] * inv_freq[j];
    cs[r][j] = rot_from_f64<T>(cos(angle));
    sn[r][j] = rot_from_f64<T>(sin(angle));
  }
  __syncthreads();
  for (int t0 = threadIdx.x; t0 < total; t0 += 4 * 256) {
    if (t0 != (int)threadIdx.x) load_round(t0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (t0 + 256 * u >= total) continue;
      V y;
#pragma unroll
      for (int i = 0; i < PP; ++i) {
        T y1, y2;
        rot_pair<T>(xv[u][2 * i], xv[u][2 * i + 1], cs[rr[u]][jj[u] + i], sn[rr[u]][jj[u] + i], y1, y2);
        y[2 * i] = y1;
        y[2 * i + 1] = y2;
      }
      *reinterpret_cast<V*>((isq[u] ? qo : ko) + off[u]) = y;
    }
  }
}

template <typename T>
int rotary_qk(const T* q, const T* k, const int64_t* pos, const double* inv_freq, T* qo, T* ko, int B, int N, int H,
              int HKV, int D, void* stream, const char* who) {
  if (B < 0 || N < 0 || H < 0 || HKV < 0) return fail(ERR_ARG, "%s: negative size", who);
  if (D < 2 || D % 2 != 0 || D > 1024) return fail(ERR_ARG, "%s: head dimension %d (even, 2..1024)", who, D);
  if ((size_t)B * N == 0 || H + HKV == 0) return OK;
  if (!pos || !inv_freq || (H > 0 && (!q || !qo)) || (HKV > 0 && (!k || !ko)))
    return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(qo) |
       reinterpret_cast<uintptr_t>(ko)) & (2 * sizeof(T) - 1))
    return fail(ERR_ARG, "%s: q, k and the outputs must be aligned to a pair", who);
  const int rows = B * N;
  // 16-byte pieces (PW pairs) where every row of pairs splits into them and the tensors are aligned
  constexpr int PW = 8 / sizeof(T);
  const bool wide = (D / 2) % PW == 0 && ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                                          reinterpret_cast<uintptr_t>(qo) | reinterpret_cast<uintptr_t>(ko)) & 15) == 0;
  const dim3 grid((unsigned)((rows + kRotRows - 1) / kRotRows));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (wide)
    hipLaunchKernelGGL((rotary_qk_kernel<T, PW>), grid, dim3(256), 0, s, q, k, pos, inv_freq, qo, ko, rows, H, HKV, D);
  else
    hipLaunchKernelGGL((rotary_qk_kernel<T, 1>), grid, dim3(256), 0, s, q, k, pos, inv_freq, qo, ko, rows, H, HKV, D);
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_rotary_qk_bf16(const void* q, const void* k, const int64_t* pos, const double* inv_freq, void* q_out,
                                  void* k_out, int B, int N, int H, int HKV, int D, void* stream) {
  return vsp::rotary_qk<__bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k), pos, inv_freq,
                                static_cast<__bf16*>(q_out), static_cast<__bf16*>(k_out), B, N, H, HKV, D, stream,
                                "vsp_rotary_qk_bf16");
}

extern "C" int vsp_rotary_qk_f16(const void* q, const void* k, const int64_t* pos, const double* inv_freq, void* q_out,
                                 void* k_out, int B, int N, int H, int HKV, int D, void* stream) {
  return vsp::rotary_qk<_Float16>(static_cast<const _Float16*>(q), static_cast<const _Float16*>(k), pos, inv_freq,
                                  static_cast<_Float16*>(q_out), static_cast<_Float16*>(k_out), B, N, H, HKV, D, stream,
                                  "vsp_rotary_qk_f16");
}

extern "C" int vsp_rotary_qk_f32(const float* q, const float* k, const int64_t* pos, const double* inv_freq,
                                 float* q_out, float* k_out, int B, int N, int H, int HKV, int D, void* stream) {
  return vsp::rotary_qk<float>(q, k, pos, inv_freq, q_out, k_out, B, N, H, HKV, D, stream, "vsp_rotary_qk_f32");
}
