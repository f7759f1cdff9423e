// Shared device helpers for the CDNA4 (gfx950) mixer kernels: element conversions, MFMA tile
// products with their operand fragment layouts, wave reductions, and the C ABI's error state.
//
// MFMA conventions used throughout (64-lane wavefronts, 16x16 output tiles):
//   v_mfma_f32_16x16x32_bf16 : lane l holds A[l%16][8*(l/16) .. +7] and B[8*(l/16) .. +7][l%16]
//   v_mfma_f32_16x16x4_f32   : lane l holds A[l%16][l/16]           and B[l/16][l%16]
//   accumulator (both)       : lane l holds D[4*(l/16) + r][l%16], r = 0..3
// A and B always use the same lane -> k assignment, so any consistent permutation of k between
// the two operands leaves the product unchanged.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

namespace vsp {

// ---- host-side error state (defined in abi.cpp) ------------------------------------------------
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

enum Status { OK = 0, ERR_ARG = 1, ERR_UNSUPPORTED = 2, ERR_LAUNCH = 3 };

// ---- bounded waits and the fault record --------------------------------------------------------
// Kernels whose waves hand work to each other through LDS flags wait with a bounded number of
// polls. A wait that gives up stores 1 into its kernel family's word of the fault record (pinned
// host memory, set up by vsp_init; the host reads it without a device synchronisation), and the
// kernel writes NaN in place of its later outputs: a broken hand-over can neither hang the device
// nor pass unnoticed. The limit is a kernel argument, so a test can make the waits give up from
// the host (vsp_set_wait_limit) while every kernel still runs to its end.
enum FaultFamily { FAULT_SCAN_CHAIN = 0, kFaultWords = 16 };
unsigned* fault_record();  // device address of the fault words; null before vsp_init
int wait_limit();          // polls before a bounded wait gives up
// The form of the bf16 scan at head width 64: 0 value-slice chains over the whole sequence
// (delta_chain_bf16_kernel), 1 segments of whole-head state joined by their affine maps
// (delta_seg_kernel), 2 (the default) by shape. Both compute the same scan; vsp_set_scan_segments
// sets it.
int scan_segments();

// The allocation-free ring attention entry's static scratch (decode.hip): rows of one call at most,
// and its per-device set-up, run by vsp_init.
constexpr int kNoAllocMaxRows = 1 << 16;
int ring_scratch_init();

__device__ __forceinline__ void record_fault(unsigned* record, int family) {
  // a plain (system-scope) store of a constant: no atomic read-modify-write on host memory
  if (record != nullptr) __hip_atomic_store(record + family, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// ---- launchers shared between translation units ------------------------------------------------
// The register-resident single-token delta step (delta_step.hip) for head widths 16, 32, 64 and
// 128; false when the width or the state's alignment needs the general token-serial kernel.
bool delta_step_fast_f32(const float* q, const float* k, const float* v, const float* beta, const float* s_in,
                         float* s_out, float* o, const uint8_t* active, int B, int H, int D, hipStream_t stream);
bool delta_step_fast_bf16(const __bf16* q, const __bf16* k, const __bf16* v, const __bf16* beta, const float* s_in,
                          float* s_out, __bf16* o, const uint8_t* active, int B, int H, int D, hipStream_t stream);

// The token-serial forward's states at each 64-token chunk's start (delta_scan.hip), and the
// backward at head widths the chunked backward does not tile (delta_scan_backward_wide.hip).
int delta_scan_checkpoints_bf16(const __bf16* q, const __bf16* k, const __bf16* v, const __bf16* beta,
                                const float* s_in, float* s_out, float* ckpt, int B, int T, int H, int D,
                                hipStream_t stream);
int delta_scan_checkpoints_f32(const float* q, const float* k, const float* v, const float* beta, const float* s_in,
                               float* s_out, float* ckpt, int B, int T, int H, int D, hipStream_t stream);
size_t wide_backward_workspace_bytes(int B, int N, int H, int D);
int scan_backward_wide_bf16(const __bf16* q, const __bf16* k, const __bf16* v, const __bf16* beta,
                            const float* state_in, const __bf16* d_o, const float* d_state, const uint8_t* active,
                            __bf16* dq, __bf16* dk, __bf16* dv, __bf16* dbeta, float* d_state_in, void* workspace,
                            size_t workspace_bytes, int B, int N, int H, int D, hipStream_t stream, const char* who);
int scan_backward_wide_f32(const float* q, const float* k, const float* v, const float* beta, const float* state_in,
                           const float* d_o, const float* d_state, const uint8_t* active, float* dq, float* dk,
                           float* dv, float* dbeta, float* d_state_in, void* workspace, size_t workspace_bytes, int B,
                           int N, int H, int D, hipStream_t stream, const char* who);

// ---- the write strength (vesper/recurrence.py:34-88) -------------------------------------------
// beta = sigmoid(logit + ln(1 + alpha m)) of a write-strength logit and the token's modulator m,
// exactly 0 where 1 + alpha m is 0 (a negative factor is refused by the host); without a
// modulator (m null) sigmoid(logit). In float32, the factor floored at the smallest normal
// before the logarithm as the reference floors it.
__device__ __forceinline__ float write_strength(float logit, const float* m, size_t token, float alpha) {
  float x = logit;
  if (m != nullptr) {
    const float f = 1.f + alpha * m[token];
    if (!(f > 0.f)) return 0.f;
    x += logf(__builtin_fmaxf(f, 1.17549435e-38f));
  }
  return 1.f / (1.f + expf(-x));
}

// ---- element conversions ----------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }

// Eight consecutive elements (16-byte aligned) as floats, with one vector load.
template <typename T>
__device__ __forceinline__ void load8_f32(const T* p, float* out) {
  if constexpr (sizeof(T) == 2) {
    typedef T V8 __attribute__((ext_vector_type(8)));
    const V8 v = *reinterpret_cast<const V8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = to_f32(v[e]);
  } else {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

// ---- MFMA tile products -----------------------------------------------------------------------
// Operand element type E selects the instruction: __bf16 -> 16x16x32 bf16, float -> 16x16x4 f32.
// `a` points at A[r0][k0] of a row-major [row][k] array with pitch lda (elements); `bt` points at
// B[k0][c0] stored as [col][k] ("k-contiguous") with pitch ldb. K is a multiple of kstep<E>.
template <typename E> struct Mfma;

template <> struct Mfma<__bf16> {
  static constexpr int kstep = 32;
  __device__ __forceinline__ static f32x4 run(const __bf16* a, int lda, const __bf16* bt, int ldb, int K,
                                              f32x4 acc) {
    const int l = threadIdx.x & 63;
    const __bf16* pa = a + (l & 15) * lda + 8 * (l >> 4);
    const __bf16* pb = bt + (l & 15) * ldb + 8 * (l >> 4);
    for (int k = 0; k < K; k += 32) {
      bf16x8 av = *reinterpret_cast<const bf16x8*>(pa + k);
      bf16x8 bv = *reinterpret_cast<const bf16x8*>(pb + k);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
    }
    return acc;
  }
};

template <> struct Mfma<float> {
  static constexpr int kstep = 4;
  __device__ __forceinline__ static f32x4 run(const float* a, int lda, const float* bt, int ldb, int K,
                                              f32x4 acc) {
    const int l = threadIdx.x & 63;
    const float* pa = a + (l & 15) * lda + (l >> 4);
    const float* pb = bt + (l & 15) * ldb + (l >> 4);
    for (int k = 0; k < K; k += 4) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[k], pb[k], acc, 0, 0, 0);
    return acc;
  }
};

// fp32 product with B row-major ([k][col], pitch ldb): used by the small triangular solves.
__device__ __forceinline__ f32x4 mfma_f32_rowmajor_b(const float* a, int lda, const float* b, int ldb, int K,
                                                     f32x4 acc) {
  const int l = threadIdx.x & 63;
  const float* pa = a + (l & 15) * lda + (l >> 4);
  const float* pb = b + (l >> 4) * ldb + (l & 15);
  for (int k = 0; k < K; k += 4) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[k], pb[k * ldb], acc, 0, 0, 0);
  return acc;
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Store an accumulator tile into a row-major [row][col] array (pitch ld) with conversion to E.
template <typename E>
__device__ __forceinline__ void store_tile(E* base, int ld, f32x4 acc) {
  const int l = threadIdx.x & 63;
  const int c = l & 15, r0 = 4 * (l >> 4);
#pragma unroll
  for (int r = 0; r < 4; ++r) base[(r0 + r) * ld + c] = from_f32<E>(acc[r]);
}

// Store an accumulator tile transposed: dst[col][row] (pitch ld), i.e. into a k-contiguous B operand.
template <typename E>
__device__ __forceinline__ void store_tile_t(E* base, int ld, f32x4 acc) {
  const int l = threadIdx.x & 63;
  const int c = l & 15, r0 = 4 * (l >> 4);
#pragma unroll
  for (int r = 0; r < 4; ++r) base[c * ld + r0 + r] = from_f32<E>(acc[r]);
}

// C[16 x 16] += op(X)[16 x K] op(Y)[K x 16] on fp32 MFMA. op(X)[i][k] is X[i * ldx + k] (TA false)
// or X[k * ldx + i] (TA true, X stored [k][i]); op(Y)[k][j] is Y[k * ldy + j] (TB false) or
// Y[j * ldy + k] (TB true), times yscale[k] when given. X and Y point at the tile's origin (16-byte
// aligned, pitches multiples of 4). Lane group g supplies k = (K / 4) g + m in step m (the sum's
// order is free), so a row-contiguous operand comes in 16-byte LDS reads of four k. The result:
// lane (j, g) holds rows 4 g .. 4 g + 3 of column j. BF: the four k of a step are rounded to bf16
// and multiplied by one 16x16x16 bf16 MFMA (fp32 accumulation) instead of four fp32 ones.
template <bool TA, bool TB, bool BF = false>
__device__ __forceinline__ f32x4 mm16(const float* X, int ldx, const float* Y, int ldy, int K, f32x4 acc,
                                      const float* yscale = nullptr) {
  const int l = threadIdx.x & 63, i = l & 15, g = l >> 4;
  const int KM = K / 4, kb = KM * g;
  for (int m = 0; m < KM; m += 4) {
    float a[4], b[4];
    if constexpr (!TA) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(X + i * ldx + kb + m);
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = v[u];
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = X[(kb + m + u) * ldx + i];
    }
    if constexpr (TB) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(Y + i * ldy + kb + m);
#pragma unroll
      for (int u = 0; u < 4; ++u) b[u] = v[u];
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) b[u] = Y[(kb + m + u) * ldy + i];
    }
    if (yscale != nullptr) {
#pragma unroll
      for (int u = 0; u < 4; ++u) b[u] *= yscale[kb + m + u];
    }
    if constexpr (BF) {
      bf16x4 av, bv;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        av[u] = (__bf16)a[u];
        bv[u] = (__bf16)b[u];
      }
      acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, av), __builtin_bit_cast(s16x4_t, bv),
                                                      acc, 0, 0, 0);
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[u], acc, 0, 0, 0);
    }
  }
  return acc;
}

// ---- lane reductions through DPP (a VALU modifier: no LDS traffic, unlike ds_bpermute) --------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
// Reduction over aligned groups of N consecutive lanes (N a power of two, 1..64); every lane of a
// group gets the same result. quad_perm [1,0,3,2] and [2,3,0,1] pair lanes within a quad,
// row_half_mirror swaps the two quads of 8 lanes, row_mirror the two halves of 16, and
// v_permlane16_swap / v_permlane32_swap hand each lane the value of lane l ^ 16 / l ^ 32 (the even
// group's value first, so the last steps combine in one order on every lane).
template <int N, typename Op>
__device__ __forceinline__ float group_reduce(float x, Op op) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "group of 1..64 lanes");
  if constexpr (N >= 2) x = op(x, dpp_f32<0xB1>(x));
  if constexpr (N >= 4) x = op(x, dpp_f32<0x4E>(x));
  if constexpr (N >= 8) x = op(x, dpp_f32<0x141>(x));
  if constexpr (N >= 16) x = op(x, dpp_f32<0x140>(x));
  if constexpr (N >= 32) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = op(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
  if constexpr (N >= 64) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = op(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
  return x;
}
struct SumOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return __builtin_fmaxf(a, b); }
};
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  return group_reduce<N>(x, SumOp{});
}
// Each lane gets the sum of x over the four lanes of the wave with its index within a 16-lane row
// (l, l ^ 16, l ^ 32, l ^ 48): a column sum of an MFMA result tile, whose rows sit in lane groups.
__device__ __forceinline__ float sum_over_rows(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}
template <int N>
__device__ __forceinline__ float group_max(float x) {
  return group_reduce<N>(x, MaxOp{});
}

// ---- transposed LDS reads (gfx950 ds_read_b64_tr_b16) ------------------------------------------
// Within each 16-lane group, lane i receives element i % 4 of the 8-byte pieces addressed by lanes
// 4e + i / 4 (e = 0..3). So when lane j of a group addresses row r0 + j / 4, column c0 + 4 (j % 4)
// of a row-major tile of 16-bit elements, lane i receives column c0 + i of rows r0 .. r0 + 3: the
// k-contiguous operand fragment of an MFMA whose k index runs down the tile's rows.
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
template <typename V4, typename T>
__device__ __forceinline__ V4 read_tr16(const T* p) {
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p));
  return __builtin_bit_cast(V4, v);
}
// The transposed fragment of a row-major tile for lane (lq, g) of a wave: column c0 + lq of rows
// r0 + 4 g .. r0 + 4 g + 3 (pitch in elements).
template <typename V4, typename T>
__device__ __forceinline__ V4 read_tr16_rows(const T* tile, int pitch, int r0, int c0) {
  const int l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  return read_tr16<V4>(tile + (r0 + 4 * g + (lq >> 2)) * pitch + c0 + 4 * (lq & 3));
}

// a.x * b.x + a.y * b.y + c on a pair of 16-bit values, accumulated in fp32 (v_dot2).
template <typename T> struct Dot2;
template <> struct Dot2<__bf16> {
  typedef __bf16 P2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static float run(P2 a, P2 b, float c) { return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false); }
};
template <> struct Dot2<_Float16> {
  typedef _Float16 P2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static float run(P2 a, P2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
};

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4): lane i writes
// lds + 16 i, so `lds` must be the same for the whole wave. Device pass only: the host pass of a
// kernel template does not take the builtin.
__device__ __forceinline__ void load_lds16(const void* src, void* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
#endif
}

// Buffer resources (raw, stride 0) over `bytes` bytes from `base`: 32-bit offsets from a scalar
// base, reads past the range return zeros and writes there are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes per lane from a buffer straight into LDS: lane i writes lds + 16 i (`lds` wave-uniform).
// Device pass only, like load_lds16: the host pass of a kernel template does not take the builtin.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, void* lds, unsigned voff, unsigned soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
#endif
}

// ---- XCD-aware block order --------------------------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (block g runs on XCD g % 8), and each XCD
// has its own L2. Renumber so that consecutive logical ids share an XCD: blocks that read the same
// data (e.g. the value slices of one head) then hit the same L2.
__device__ __forceinline__ int xcd_logical_block(int g, int n) {
  constexpr int kXcd = 8;
  if (n % kXcd != 0) return g;
  return (g % kXcd) * (n / kXcd) + g / kXcd;
}

}  // namespace vsp
