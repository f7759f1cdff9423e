// The looped column's copy-forward bookkeeping on CDNA4 (gfx950): token rows copied where a flag is set.
//
// Reference: vesper/loop.py:523-537 (`_merge`: the tokens halting now freeze their fresh
// projections into the carried ones, six `where`s per column and pass) and vesper/loop.py:441-452
// (a halted token's hidden state is carried forward, `where(active, h, x)`). Each is a select over
// whole token rows. Here one launch copies the flagged rows of up to eight tensors in place,
// dst[r] = src[r] where flags[r] != 0: only the flagged rows are read and written.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kMaxItems = 8;

struct CopyItems {
  const uint8_t* src[kMaxItems];
  uint8_t* dst[kMaxItems];
  const uint8_t* flags[kMaxItems];
  unsigned row_units[kMaxItems];       // copy units per row
  unsigned unit_log2[kMaxItems];       // a unit is 1 << unit_log2 bytes (1 .. 16)
  int count;
};

template <typename U>
__device__ __forceinline__ void copy_unit(const uint8_t* src, uint8_t* dst, size_t u) {
  reinterpret_cast<U*>(dst)[u] = reinterpret_cast<const U*>(src)[u];
}

// One token row per wave, every item in turn: a row whose flag is 0 costs one flag read, a flagged
// row is copied by the wave's lanes in units of 1 << unit_log2 bytes.
__global__ __launch_bounds__(256) void copy_rows_kernel(const CopyItems items, unsigned rows) {
  const unsigned row = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  for (int i = 0; i < items.count; ++i) {
    if (items.flags[i][row] == 0) continue;
    const unsigned per = items.row_units[i];
    const size_t base = (size_t)row * per;
    const uint8_t* s = items.src[i];
    uint8_t* d = items.dst[i];
    for (unsigned u = lane; u < per; u += 64) {
      switch (items.unit_log2[i]) {
        case 4: copy_unit<uint4>(s, d, base + u); break;
        case 3: copy_unit<uint2>(s, d, base + u); break;
        case 2: copy_unit<uint32_t>(s, d, base + u); break;
        case 1: copy_unit<uint16_t>(s, d, base + u); break;
        default: copy_unit<uint8_t>(s, d, base + u); break;
      }
    }
  }
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_copy_rows_where(int count, const void* const* src, void* const* dst, const size_t* row_bytes,
                                   const uint8_t* const* flags, int rows, void* stream) {
  using namespace vsp;
  const char* who = "vsp_copy_rows_where";
  if (count < 0 || count > kMaxItems) return fail(ERR_ARG, "%s: %d tensors (1 .. %d per launch)", who, count, kMaxItems);
  if (rows < 0) return fail(ERR_ARG, "%s: %d rows", who, rows);
  if (count == 0 || rows == 0) return OK;
  if (!src || !dst || !row_bytes || !flags) return fail(ERR_ARG, "%s: null array", who);
  CopyItems items{};
  items.count = count;
  for (int i = 0; i < count; ++i) {
    if (!src[i] || !dst[i] || !flags[i]) return fail(ERR_ARG, "%s: null pointer in tensor %d", who, i);
    if (row_bytes[i] == 0) return fail(ERR_ARG, "%s: tensor %d has empty rows", who, i);
    const uintptr_t mix = reinterpret_cast<uintptr_t>(src[i]) | reinterpret_cast<uintptr_t>(dst[i]) | row_bytes[i];
    unsigned lg = 4;
    while (lg > 0 && (mix & ((1u << lg) - 1)) != 0) --lg;
    const size_t per = row_bytes[i] >> lg;
    if (per > 0xFFFFFFFFu) return fail(ERR_UNSUPPORTED, "%s: rows of %zu bytes", who, row_bytes[i]);
    items.src[i] = static_cast<const uint8_t*>(src[i]);
    items.dst[i] = static_cast<uint8_t*>(dst[i]);
    items.flags[i] = flags[i];
    items.row_units[i] = (unsigned)per;
    items.unit_log2[i] = lg;
  }
  hipLaunchKernelGGL(copy_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), items, (unsigned)rows);
  return check_launch(who);
}

namespace vsp {
namespace {

// The pass loop's halting bookkeeping for one pass (vesper/loop.py:441-452 with the pass count of
// column.py's loop): halts = active & exits (every active token on the last pass, exits NULL),
// n_iters += active, next = active & !halts. One thread per token.
__global__ __launch_bounds__(256) void halt_step_kernel(const uint8_t* __restrict__ active,
                                                        const uint8_t* __restrict__ exits,
                                                        int* __restrict__ n_iters, uint8_t* __restrict__ halts,
                                                        uint8_t* __restrict__ next, int count) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const uint8_t a = active[i] != 0;
  const uint8_t h = a & (exits == nullptr ? (uint8_t)1 : (uint8_t)(exits[i] != 0));
  n_iters[i] += a;
  halts[i] = h;
  next[i] = a & (uint8_t)!h;
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_halt_step(const uint8_t* active, const uint8_t* exits, int* n_iters, uint8_t* halts, uint8_t* next,
                             int count, void* stream) {
  using namespace vsp;
  const char* who = "vsp_halt_step";
  if (count < 0) return fail(ERR_ARG, "%s: %d tokens", who, count);
  if (count == 0) return OK;
  if (!active || !n_iters || !halts || !next) return fail(ERR_ARG, "%s: null pointer", who);
  if (next == active || halts == active) return fail(ERR_ARG, "%s: the outputs must not be the active flags", who);
  hipLaunchKernelGGL(halt_step_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), active, exits, n_iters, halts, next, count);
  return check_launch(who);
}

namespace vsp {
namespace {

// The residual stream after a pass's attention, for the rows still in the loop: x[r] = x1[r] + a[r]
// (x1 float32, a the attention's bf16 output, added in float32 as the column's residual add) where
// flags[r] != 0 (every row when flags is NULL); other rows of x keep what they hold (the halted
// tokens' carried hidden states, vesper/loop.py:452). One wave a row, 16-byte pieces.
__global__ __launch_bounds__(256) void residual_rows_kernel(const float* __restrict__ x1, const __bf16* __restrict__ a,
                                                            float* __restrict__ x, const uint8_t* __restrict__ flags,
                                                            int rows, int d) {
  const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  if (flags != nullptr && flags[row] == 0) return;
  const size_t base = (size_t)row * d;
  for (int f = 8 * lane; f < d; f += 512) {
    const float4 u = reinterpret_cast<const float4*>(x1 + base + f)[0];
    const float4 w = reinterpret_cast<const float4*>(x1 + base + f)[1];
    const bf16x8 r = *reinterpret_cast<const bf16x8*>(a + base + f);
    reinterpret_cast<float4*>(x + base + f)[0] =
        make_float4(u.x + (float)r[0], u.y + (float)r[1], u.z + (float)r[2], u.w + (float)r[3]);
    reinterpret_cast<float4*>(x + base + f)[1] =
        make_float4(w.x + (float)r[4], w.y + (float)r[5], w.z + (float)r[6], w.w + (float)r[7]);
  }
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_residual_rows_where(const float* x1, const void* a, float* x, const uint8_t* flags, int rows, int d,
                                       void* stream) {
  using namespace vsp;
  const char* who = "vsp_residual_rows_where";
  if (rows < 0 || d < 8 || d % 8 != 0) return fail(ERR_ARG, "%s: rows %d, width %d (a multiple of 8)", who, rows, d);
  if (rows == 0) return OK;
  if (!x1 || !a || !x) return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(x1) | reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(x)) & 15)
    return fail(ERR_ARG, "%s: x1, a and x must be 16-byte aligned", who);
  hipLaunchKernelGGL(residual_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), x1, static_cast<const __bf16*>(a), x, flags, rows, d);
  return check_launch(who);
}
