// Delta-rule scan on CDNA4 (gfx950): the prefill scan and the single-token decode step.
//
// Per batch row b and head h the state H [D, D] (key rows, value columns) is read as H^T q; a token
// applies H <- (I - beta k k^T) H + beta k v^T and reads o = H^T q (reference vesper/recurrence.py:
// 1-23, 118-163). Four kernels (the decode step's register-resident kernel is in delta_step.hip):
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
//    gives B*H*(D/16) concurrent chains. fp32 inputs and head widths 16 and 128.
//  * delta_chain_bf16_kernel - the same chains for bf16 inputs at head widths 32 and 64, with the
//    state-independent products (W = T K, U = T V, P = tril(Q K^T), the outputs) moved to helper
//    waves, so the chain wave runs only Delta = U - W H and H += K^T Delta per chunk.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kChunk = 64;

// Copy-forward: where a token is inactive (halted), its k, v and beta are read from the carried
// tensors (same layout) instead of the fresh ones. All three null: every token reads the fresh ones.
template <typename TIn>
struct Carried {
  const TIn* k;
  const TIn* v;
  const TIn* beta;
  // The source of a token's row: the carried tensor where the token is inactive. The kernels take
  // CARRY as a template argument, so without carried inputs no address waits for a flag.
  template <bool CARRY>
  __device__ __forceinline__ static const TIn* pick(const TIn* fresh, const TIn* held, uint8_t active) {
    if constexpr (CARRY) return active == 0 ? held : fresh;
    return fresh;
  }
};

// --------------------------------------------------------------------------------------------
// token-serial kernel
// --------------------------------------------------------------------------------------------
template <typename TIn>
__global__ __launch_bounds__(256) void delta_serial_kernel(const TIn* __restrict__ q, const TIn* __restrict__ k,
                                                           const TIn* __restrict__ v, const TIn* __restrict__ beta,
                                                           const float* s_in, float* s_out,  // may alias
                                                           TIn* __restrict__ o, const uint8_t* __restrict__ active,
                                                           const TIn* kc, const TIn* vc, const TIn* bc, int T, int H,
                                                           int D, int groups, const float* mod_m, float mod_alpha,
                                                           int beta_logits, float* ckpt) {
  // (scalar pointer arguments: a struct argument would be read through private memory and count as
  // divergent, which turns every buffer access on it into a loop over lanes)
  const Carried<TIn> carried{kc, vc, bc};
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
    if ((int)threadIdx.x < nt) sa[threadIdx.x] = active ? active[(size_t)b * T + t0 + threadIdx.x] : (uint8_t)1;
    if (carried.k != nullptr) __syncthreads();  // the flags choose each token's source
    for (int i = threadIdx.x; i < nt * D; i += blockDim.x) {
      const int tt = i / D, e = i - tt * D;
      const size_t off = (((size_t)b * T + t0 + tt) * H + h) * D + e;
      sk[tt][e] = to_f32((carried.k != nullptr && sa[tt] == 0 ? carried.k : k)[off]);
      sq[tt][e] = to_f32(q[off]);
    }
    for (int i = threadIdx.x; i < nt * 64; i += blockDim.x) {
      const int tt = i >> 6, c = blockIdx.y * 64 + (i & 63);
      const TIn* src = carried.k != nullptr && sa[tt] == 0 ? carried.v : v;
      sv[tt][i & 63] = c < D ? to_f32(src[(((size_t)b * T + t0 + tt) * H + h) * D + c]) : 0.f;
    }
    if ((int)threadIdx.x < nt) {
      const size_t tok = (size_t)b * T + t0 + threadIdx.x;
      const float raw = to_f32((carried.k != nullptr && sa[threadIdx.x] == 0 ? carried.beta : beta)[tok * H + h]);
      // beta from its logit is rounded to the inputs' dtype, as the reference column casts it
      // before its scan (column.py:313)
      sb[threadIdx.x] = beta_logits ? to_f32(from_f32<TIn>(write_strength(raw, mod_m, tok, mod_alpha))) : raw;
    }
    __syncthreads();
    for (int tt = 0; tt < nt; ++tt) {
      if (ckpt != nullptr && ((t0 + tt) & 63) == 0) {
        // the state at a 64-token chunk's start, for the backward: [b, h][chunk][row][column]
        float* dst = ckpt + ((size_t)bh * ((T + 63) >> 6) + ((t0 + tt) >> 6)) * D * D;
#pragma unroll
        for (int r = 0; r < 64; ++r) {
          const int row = wv * 64 + r;
          if (col_ok && row < D) dst[(size_t)row * D + col] = st[r];
        }
      }
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
      if (wv == 0 && col_ok && o != nullptr)
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
// MFMA operand flavours
// --------------------------------------------------------------------------------------------
__device__ __forceinline__ int lane_group() { return (threadIdx.x & 63) >> 4; }

// A chunk's 64 active flags as a wave-uniform mask (bit r: token r of the chunk is active), from
// lanes holding the flag of token 16 i + (lane % 16) in a[i].
__device__ __forceinline__ uint64_t chunk_mask(const uint8_t (&a)[4]) {
  uint64_t m = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) m |= (__builtin_amdgcn_ballot_w64(a[i] != 0) & 0xFFFFull) << (16 * i);
  return m;
}

// Within a wave, make LDS writes of any lane visible to later LDS reads of any lane.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// "Acc" flavour: the B operand is a pair of accumulator tiles (rows 16 apart, 32 k values), so a
// lane of group g supplies k = 4g + r and 16 + 4g + r (r = 0..3); the A operand is read from a
// row-major LDS row with that same k permutation. Products of two chained contractions never
// leave registers this way.
template <typename E> struct Acc;
template <> struct Acc<__bf16> {
  struct B { bf16x8 v; };
  __device__ __forceinline__ static B pack(f32x4 t0, f32x4 t1) {
    B b;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      b.v[r] = (__bf16)t0[r];
      b.v[4 + r] = (__bf16)t1[r];
    }
    return b;
  }
  __device__ __forceinline__ static f32x4 mma(const __bf16* arow, const B& b, f32x4 acc) {
    const int g = lane_group();
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(arow + 4 * g);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(arow + 16 + 4 * g);
    const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b.v, acc, 0, 0, 0);
  }
};
template <> struct Acc<float> {
  struct B { f32x4 t0, t1; };
  __device__ __forceinline__ static B pack(f32x4 t0, f32x4 t1) { return B{t0, t1}; }
  __device__ __forceinline__ static f32x4 mma(const float* arow, const B& b, f32x4 acc) {
    const int g = lane_group();
    const f32x4 lo = *reinterpret_cast<const f32x4*>(arow + 4 * g);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(arow + 16 + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(lo[r], b.t0[r], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(hi[r], b.t1[r], acc, 0, 0, 0);
    return acc;
  }
};

// "Nat" flavour: rows loaded straight from memory, K values along the row. bf16: lane group g holds
// k = 32s + 8g + e (s < K/32, e < 8). fp32: k = (K/4) g + 4s + e (s < K/16, e < 4), so each lane
// reads one contiguous run of its row.
template <typename E, int K> struct Nat;
template <int K> struct Nat<__bf16, K> {
  static constexpr int NREG = K / 32;
  static constexpr int PER = 8;
  using R = bf16x8;
  __device__ __forceinline__ static int feat(int s) { return 32 * s + 8 * lane_group(); }
  __device__ __forceinline__ static f32x4 mma(const R* a, const R* b, f32x4 acc) {
#pragma unroll
    for (int s = 0; s < NREG; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[s], b[s], acc, 0, 0, 0);
    return acc;
  }
  __device__ __forceinline__ static f32x4 mma_lds(const __bf16* arow, const R* b, f32x4 acc) {
#pragma unroll
    for (int s = 0; s < NREG; ++s) {
      const R a = *reinterpret_cast<const R*>(arow + feat(s));
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[s], acc, 0, 0, 0);
    }
    return acc;
  }
};
template <int K> struct Nat<float, K> {
  static constexpr int FPL = K / 4;
  static constexpr int NREG = FPL / 4;
  static constexpr int PER = 4;
  using R = f32x4;
  __device__ __forceinline__ static int feat(int s) { return FPL * lane_group() + 4 * s; }
  __device__ __forceinline__ static f32x4 mma(const R* a, const R* b, f32x4 acc) {
#pragma unroll
    for (int s = 0; s < NREG; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s][e], b[s][e], acc, 0, 0, 0);
    return acc;
  }
  __device__ __forceinline__ static f32x4 mma_lds(const float* arow, const R* b, f32x4 acc) {
#pragma unroll
    for (int s = 0; s < NREG; ++s) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(arow + feat(s));
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[s][e], acc, 0, 0, 0);
    }
    return acc;
  }
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

template <typename E>
__device__ __forceinline__ E elem_of(const u32x4& v, int i) {
  if constexpr (sizeof(E) == 2) {
    const uint32_t w = v[i >> 1];
    const uint16_t hbits = (i & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
    return __builtin_bit_cast(E, hbits);
  } else {
    // through a scalar: a bit_cast applied to the vector element directly was compiled as
    // element 0 for every i by this toolchain
    const uint32_t w = v[i];
    return __uint_as_float(w);
  }
}

// The compact per-chunk UT factor: the ten 16x16 tiles (i, j), j <= i, of T = (I + A)^-1 diag(beta),
// tile t = i (i + 1) / 2 + j, each row-major.
constexpr int kTiles = 10;
constexpr int kTileElems = 256;
constexpr int kChunkT = kTiles * kTileElems;
// constexpr (not __constant__): indices into register arrays must fold at compile time
constexpr int kTileRow[kTiles] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3};
constexpr int kTileCol[kTiles] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3};
__device__ __forceinline__ int tile_of(int i, int j) { return i * (i + 1) / 2 + j; }

// --------------------------------------------------------------------------------------------
// the UT factor of one chunk, by one wave
// --------------------------------------------------------------------------------------------
constexpr int kUtPitch = 17;  // pitch of the fp32 16x16 scratch tiles
constexpr int kUtScratch = 8 * 16 * kUtPitch;  // floats: the four diagonal A tiles, then their inverses

// T = (I + A)^-1 diag(beta) with A = tril(diag(beta) K K^T, -1) for one 64-token chunk, computed
// by one wave with no workgroup barrier: the Gram matrix on MFMA from the key rows `kn` (Nat
// layout, zero rows past the chunk's end), the four diagonal 16x16 blocks of the inverse by
// forward substitution in fp32, the off-diagonal blocks level by level on fp32 MFMA. The six
// off-diagonal A tiles never leave registers: computed transposed (K_j K_i^T = (K_i K_j^T)^T), an
// accumulator tile is already the A operand of the fp32 16x16x4 products. Only the diagonal A
// tiles and their inverses use the LDS scratch `scr` (kUtScratch floats, 8.5 KiB). `bl` is beta
// of token l on lane l (zero past the end). Element (r, c) of the lower 16x16 tile (ti, tj) of T
// goes to out(ti, tj, r, c), an LDS or global address that may alias `scr`. Upper tiles are not
// written. Ends with a wave_sync, so the wave may read LDS tiles back.
template <typename E, int DKP, typename Out>
__device__ __forceinline__ void ut_solve(const typename Nat<E, DKP>::R (&kn)[4][Nat<E, DKP>::NREG], float bl,
                                         float* scr, Out out) {
  using N = Nat<E, DKP>;
  constexpr int TP = kUtPitch;
  const int l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  float* Ad = scr;                // diagonal A tiles, row-major
  float* Xd = scr + 4 * 16 * TP;  // their inverses (I + A_bb)^-1, row-major

  // A tiles: diagonal ones into LDS (strictly lower part), off-diagonal ones transposed in
  // registers: aoff holds A[16 i + lq][16 j + 4 g + r] on lane (lq, g)
  f32x4 aoff[6];  // (1,0) (2,0) (2,1) (3,0) (3,1) (3,2)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float brow = __shfl(bl, 16 * i + lq);  // beta of row 16 i + lq (the transposed layout's row)
#pragma unroll
    for (int j = 0; j < i; ++j) {
      const f32x4 gt = N::mma(kn[j], kn[i], zero4());
      f32x4 a;
#pragma unroll
      for (int r = 0; r < 4; ++r) a[r] = brow * gt[r];
      aoff[i * (i - 1) / 2 + j] = a;
    }
    const f32x4 gd = N::mma(kn[i], kn[i], zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * g + r;
      const float br = __shfl(bl, 16 * i + row);
      Ad[i * 16 * TP + row * TP + lq] = row > lq ? br * gd[r] : 0.f;
    }
  }
  wave_sync();

  // diagonal blocks: lane (blk, col) solves (I + A_bb) x = e_col by forward substitution, column by
  // column (once x_j is known it leaves every later row's sum, each row's terms in the order of j),
  // so the rows' updates are independent and the dependent chain is 15 steps long
  {
    const int blk = g, col = lq;
    const float* ab = Ad + blk * 16 * TP;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = (i == col) ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
      for (int i = j + 1; i < 16; ++i) x[i] -= ab[i * TP + j] * x[j];
#pragma unroll
    for (int i = 0; i < 16; ++i) Xd[blk * 16 * TP + i * TP + col] = x[i];
  }
  wave_sync();

  // 16x16x16 products; k permuted as 4g + r so accumulator tiles serve as B operands. For bf16
  // inputs (whose factor is stored in bf16) one bf16 16x16x16 MFMA with fp32 accumulation; for fp32
  // inputs four fp32 16x16x4 MFMAs, keeping the fp32 entry's precision
  auto mm = [&](const float* atile_lds, const f32x4* areg, const float* btile_lds, const f32x4* breg, f32x4 acc) {
    if constexpr (sizeof(E) == 2) {
      typedef short s16x4_v __attribute__((ext_vector_type(4)));
      bf16x4 a4, b4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        a4[r] = (__bf16)(areg ? (*areg)[r] : atile_lds[lq * TP + 4 * g + r]);
        b4[r] = (__bf16)(breg ? (*breg)[r] : btile_lds[(4 * g + r) * TP + lq]);
      }
      return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_v, a4), __builtin_bit_cast(s16x4_v, b4),
                                                       acc, 0, 0, 0);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float av = areg ? (*areg)[r] : atile_lds[lq * TP + 4 * g + r];
        const float bv = breg ? (*breg)[r] : btile_lds[(4 * g + r) * TP + lq];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
      }
      return acc;
    }
  };
  auto xd = [&](int blk) { return (const float*)(Xd + blk * 16 * TP); };
  auto ao = [&](int i, int j) { return &aoff[i * (i - 1) / 2 + j]; };

  f32x4 x1[3], x2[2], x3;
#pragma unroll
  for (int bb = 0; bb < 3; ++bb) {
    const f32x4 y = mm(nullptr, ao(bb + 1, bb), xd(bb), nullptr, zero4());
    x1[bb] = -mm(xd(bb + 1), nullptr, nullptr, &y, zero4());
  }
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    f32x4 y = mm(nullptr, ao(bb + 2, bb), xd(bb), nullptr, zero4());
    y = mm(nullptr, ao(bb + 2, bb + 1), nullptr, &x1[bb], y);
    x2[bb] = -mm(xd(bb + 2), nullptr, nullptr, &y, zero4());
  }
  {
    f32x4 y = mm(nullptr, ao(3, 0), xd(0), nullptr, zero4());
    y = mm(nullptr, ao(3, 1), nullptr, &x1[0], y);
    y = mm(nullptr, ao(3, 2), nullptr, &x2[0], y);
    x3 = -mm(xd(3), nullptr, nullptr, &y, zero4());
  }

  // T = X diag(beta): the diagonal tiles from the LDS inverses (read before any output write
  // that may alias them), the off-diagonal ones from registers
  float dcol[16];
  {
    const int blk = g, col = lq;
    const float bc = __shfl(bl, 16 * blk + col);
#pragma unroll
    for (int i = 0; i < 16; ++i) dcol[i] = Xd[blk * 16 * TP + i * TP + col] * bc;
  }
  wave_sync();
#pragma unroll
  for (int i = 0; i < 16; ++i) *out(g, g, i, lq) = from_f32<E>(dcol[i]);
  auto put = [&](int i, int j, const f32x4& x) {
    const float bc = __shfl(bl, 16 * j + lq);
#pragma unroll
    for (int r = 0; r < 4; ++r) *out(i, j, 4 * g + r, lq) = from_f32<E>(x[r] * bc);
  };
  put(1, 0, x1[0]);
  put(2, 1, x1[1]);
  put(3, 2, x1[2]);
  put(2, 0, x2[0]);
  put(3, 1, x2[1]);
  put(3, 0, x3);
  wave_sync();
}

// --------------------------------------------------------------------------------------------
// chunk preparation: one wave per 64-token chunk, no workgroup barriers
// --------------------------------------------------------------------------------------------
template <typename TIn, typename E, int DK, bool CARRY>
__global__ __launch_bounds__(256, 3) void delta_prep_kernel(const TIn* __restrict__ k, const TIn* __restrict__ beta,
                                                         E* __restrict__ tmat, const uint8_t* __restrict__ active,
                                                         const TIn* kc, const TIn* vc, const TIn* bc, int T, int H,
                                                         int total, const float* mod_m, float mod_alpha, int beta_logits) {
  const Carried<TIn> carried{kc, vc, bc};
  constexpr int DKP = DK < 32 ? 32 : DK;
  using N = Nat<E, DKP>;
  // the compact factor is staged in LDS for 16-byte global stores: it overlays the scratch
  constexpr int kScr = kChunkT * (int)sizeof(E) / 4 > kUtScratch ? kChunkT * (int)sizeof(E) / 4 : kUtScratch;
  __shared__ __align__(16) float sScr[4][kScr];

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lq = l & 15;
  const int chunk = blockIdx.x * 4 + w;
  if (chunk >= total) return;  // whole waves only: this kernel has no workgroup barrier
  const int nc = (T + kChunk - 1) / kChunk;
  const int c = chunk % nc, bh = chunk / nc;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kChunk, nv = min(kChunk, T - t0);

  // Every load is unconditional (tokens past the end re-read the last one, padding features re-read
  // feature 0) and the zeros are selected once all are issued: a load behind a per-lane branch
  // would wait for every earlier one.
  // with carried inputs, the flags of the lane's rows choose their source (loaded first)
  uint8_t ak[4] = {1, 1, 1, 1}, ab = 1;
  if constexpr (CARRY) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ak[i] = active[(size_t)b * T + min(t0 + 16 * i + lq, T - 1)];
    ab = active[(size_t)b * T + min(t0 + l, T - 1)];
  }
  typename N::R kn[4][N::NREG];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const TIn* row = Carried<TIn>::template pick<CARRY>(k, carried.k, ak[i]) + (((size_t)b * T + min(t0 + 16 * i + lq, T - 1)) * H + h) * DK;
#pragma unroll
    for (int sgi = 0; sgi < N::NREG; ++sgi) {
      const int f = N::feat(sgi);
      kn[i][sgi] = *reinterpret_cast<const typename N::R*>(row + (f < DK ? f : 0));
    }
  }
  const TIn braw = Carried<TIn>::template pick<CARRY>(beta, carried.beta, ab)[((size_t)b * T + min(t0 + l, T - 1)) * H + h];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int sgi = 0; sgi < N::NREG; ++sgi) {
      const bool ok = 16 * i + lq < nv && N::feat(sgi) < DK;
#pragma unroll
      for (int e = 0; e < N::PER; ++e) kn[i][sgi][e] = ok ? kn[i][sgi][e] : from_f32<E>(0.f);
    }
  // the write strength from its logit (and the token's modulator) where the entry takes logits,
  // rounded to the inputs' dtype as the reference column casts beta before its scan (column.py:313)
  const float braw_f =
      beta_logits ? to_f32(from_f32<TIn>(write_strength(to_f32(braw), mod_m, (size_t)b * T + min(t0 + l, T - 1), mod_alpha)))
                  : to_f32(braw);
  const float bl = l < nv ? braw_f : 0.f;
  E* tc = reinterpret_cast<E*>(&sScr[w][0]);  // compact tiles: tile t = i (i + 1) / 2 + j, row-major
  ut_solve<E, DKP>(kn, bl, &sScr[w][0],
                   [&](int ti, int tj, int r, int cc) { return tc + tile_of(ti, tj) * kTileElems + r * 16 + cc; });
  // the compact factor to global memory in 16-byte pieces
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  constexpr int SEGS = kChunkT * (int)sizeof(E) / 16;
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(tmat + (size_t)chunk * kChunkT);
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(tc);
  for (int j = l; j < SEGS; j += 64) dst[j] = src[j];
}

// --------------------------------------------------------------------------------------------
// the chunk chain: wave 0 carries the state of one (b, h, 16-column value slice) through the chunks
// with every intermediate in registers; waves 1..NH stage chunk data ahead of it, form
// P^T = tril(Q K^T)^T and write the outputs O^T = H^T Q^T + Delta^T P^T one iteration behind it.
// --------------------------------------------------------------------------------------------
// Helper waves per workgroup (= chunks staged ahead of the chain). Seven keep the bf16 chain fed
// through HBM latency at head width 64; wider heads and fp32 need the registers of a 4-wave group.
template <typename E, int DK> struct ChainShape {
  static constexpr int NH = (sizeof(E) == 2 && DK <= 64) ? 7 : 3;
};

template <typename TIn, typename E, int DK, bool CARRY>
__global__ __launch_bounds__(64 * (ChainShape<E, DK>::NH + 1)) void delta_chain_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const E* __restrict__ tmat,
    const float* __restrict__ s_in, float* __restrict__ s_out, TIn* __restrict__ o, const uint8_t* __restrict__ active,
    const TIn* kc, const TIn* vc, const TIn* bc, int T, int H) {
  const Carried<TIn> carried{kc, vc, bc};
  constexpr int NH = ChainShape<E, DK>::NH;
  constexpr int NW = NH + 1;
  constexpr int BV = 16;
  constexpr int NS = DK / BV;
  constexpr bool BF = sizeof(E) == 2;
  constexpr int DKP = DK < 32 ? 32 : DK;
  constexpr int PAD = BF ? 8 : 4;
  constexpr int PK = DKP + PAD;
  constexpr int PT = 64 + PAD;
  constexpr int HB = DK / 16;
  constexpr int KBF = DKP / 32;
  constexpr int EPS = 16 / (int)sizeof(E);               // elements per 16-byte segment
  constexpr int TSEG = kChunkT * (int)sizeof(E) / 16 / 64;  // compact-T segments per lane
  constexpr int VSPT = BV * (int)sizeof(E) / 16;            // V segments per token
  constexpr int VSEG = 64 * VSPT / 64;                      // V segments per lane
  // Q for the outputs: bf16 keeps it in three LDS buffers (written when the chunk is staged, read
  // two iterations later); fp32 re-reads it from L2 in the helper's idle iteration (no LDS left)
  constexpr bool kQInLds = BF;
  using N = Nat<E, DKP>;
  using AB = typename Acc<E>::B;
  using NR = typename N::R;

  __shared__ __align__(16) E sK[2][64 * PK];
  __shared__ __align__(16) E sKt[2][DK * PT];
  __shared__ __align__(16) E sT[2][64 * PT];
  __shared__ __align__(16) E sVt[2][BV * PT];
  __shared__ __align__(16) E sHo[2][BV * PK];
  __shared__ __align__(16) E sDo[2][BV * PT];
  __shared__ __align__(16) E sQ[kQInLds ? 3 : 1][kQInLds ? 64 * PK : 16];

  const int lg = xcd_logical_block(blockIdx.x, gridDim.x);
  const int slice = lg % NS, bh = lg / NS;
  const int b = bh / H, h = bh - b * H;
  const int v0 = slice * BV;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lq = l & 15, g = l >> 4;
  const int nc = (T + kChunk - 1) / kChunk;

  {
    const E zero = from_f32<E>(0.f);
    E* base[6] = {&sK[0][0], &sKt[0][0], &sT[0][0], &sVt[0][0], &sHo[0][0], &sDo[0][0]};
    const int len[6] = {2 * 64 * PK, 2 * DK * PT, 2 * 64 * PT, 2 * BV * PT, 2 * BV * PK, 2 * BV * PT};
#pragma unroll
    for (int a = 0; a < 6; ++a)
      for (int i = threadIdx.x; i < len[a]; i += 64 * NW) base[a][i] = zero;
  }

  // ---- helper state ----
  const int hj = wave - 1;  // helper index; chunks c with c % NH == hj
  NR qn[4][N::NREG], kn[4][N::NREG];
  u32x4 tseg[TSEG], vseg[BF ? 1 : VSEG];
  bf16x4 vn[BF ? 4 : 1];  // bf16: V slice rows, value columns 4g..4g+3 (16x16x16 operand layout)
  uint8_t actraw[4];  // active bytes as loaded; compared only when staged (no wait at issue)
  NR qr[kQInLds ? 1 : 4][N::NREG];  // fp32: Q re-read for the pending output
  AB pt[6];
  uint8_t actk[4];

  // Rows of one (b, h) from a uniform base with 32-bit lane offsets (the host keeps T*H*DK below
  // 2^31): one VGPR per address keeps the helpers' staging registers from spilling.
  const int rstride = H * DK;
  const size_t bh_base = ((size_t)b * T * H + h) * DK;
  // Loads are unconditional (rows past the end re-read the last row, padding features feature 0)
  // and zeros are selected once all are issued: a load behind a per-lane branch would wait for
  // every earlier one. Row 16 i + lq of the lane reads `held` where actraw[i] says the token is
  // inactive and carried inputs are given.
  auto load_rows = [&](NR (&dst)[4][N::NREG], const TIn* base, const TIn* held, int c) {
    const int nvc = min(kChunk, T - c * kChunk);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = min(16 * i + lq, nvc - 1);
      const TIn* cb = Carried<TIn>::template pick<CARRY>(base, held, actraw[i]) + bh_base + (size_t)c * kChunk * rstride;
#pragma unroll
      for (int s = 0; s < N::NREG; ++s) {
        const int f = N::feat(s);
        dst[i][s] = *reinterpret_cast<const NR*>(cb + (tok * rstride + (f < DK ? f : 0)));
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int s = 0; s < N::NREG; ++s) {
        const bool ok = 16 * i + lq < nvc && N::feat(s) < DK;
#pragma unroll
        for (int e = 0; e < N::PER; ++e) dst[i][s][e] = ok ? dst[i][s][e] : from_f32<E>(0.f);
      }
  };
  auto issue_loads = [&](int c) {
    const int nvc = min(kChunk, T - c * kChunk);
    // the flags first: with carried inputs they choose the sources of the K and V rows
#pragma unroll
    for (int i = 0; i < 4; ++i)
      actraw[i] = active != nullptr ? active[(size_t)b * T + (size_t)c * kChunk + min(16 * i + lq, nvc - 1)] : (uint8_t)1;
    load_rows(qn, q, q, c);
    load_rows(kn, k, carried.k, c);
    const u32x4* ts = reinterpret_cast<const u32x4*>(tmat + ((size_t)bh * nc + c) * kChunkT);
#pragma unroll
    for (int j = 0; j < TSEG; ++j) tseg[j] = ts[l + 64 * j];
    if constexpr (BF) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const TIn* cb = Carried<TIn>::template pick<CARRY>(v, carried.v, actraw[i]) + bh_base + (size_t)c * kChunk * rstride + v0;
        vn[i] = *reinterpret_cast<const bf16x4*>(cb + (min(16 * i + lq, nvc - 1) * rstride + 4 * g));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) vn[i][e] = 16 * i + lq < nvc ? vn[i][e] : (__bf16)0.f;
    } else {
      // V segment rows are not the lane's flag rows: their flags come from the chunk's mask
      uint64_t held_rows = 0;
      if constexpr (CARRY) held_rows = ~chunk_mask(actraw);
#pragma unroll
      for (int j = 0; j < VSEG; ++j) {
        const int sg = l + 64 * j, tok = sg / VSPT, part = sg - tok * VSPT;
        const int tl = min(tok, nvc - 1);  // the row loaded, with its own source flag
        const TIn* cb = (((held_rows >> tl) & 1) ? carried.v : v) + bh_base + (size_t)c * kChunk * rstride + v0;
        vseg[j] = *reinterpret_cast<const u32x4*>(cb + (tl * rstride + part * EPS));
      }
#pragma unroll
      for (int j = 0; j < VSEG; ++j)
        if ((l + 64 * j) / VSPT >= nvc) vseg[j] = u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_chunk = [&](int c) {
    const int bs = c & 1;
    E* K = sK[bs];
    E* Kt = sKt[bs];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = 16 * i + lq;
#pragma unroll
      for (int s = 0; s < N::NREG; ++s) {
        const int f = N::feat(s);
        *reinterpret_cast<NR*>(K + tok * PK + f) = kn[i][s];
        if constexpr (!BF) {
#pragma unroll
          for (int e = 0; e < N::PER; ++e)
            if (f + e < DK) Kt[(f + e) * PT + tok] = kn[i][s][e];
        }
      }
    }
    if constexpr (BF) {
      // transposes through the MFMA unit: (rows x 32) . I selects 16 columns and returns them in
      // the accumulator layout, where a lane holds four consecutive rows of one column - so each
      // lane writes 8 contiguous bytes of the transposed tile. Exact: products with 1 and 0.
      bf16x8 eye[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int j = 0; j < 8; ++j) eye[hh][j] = (__bf16)((8 * g + j == 16 * hh + lq) ? 1.f : 0.f);
      bf16x4 eye4;  // the 16x16x16 operand: lane group g holds k = 4g..4g+3
#pragma unroll
      for (int j = 0; j < 4; ++j) eye4[j] = (__bf16)((4 * g + j == lq) ? 1.f : 0.f);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int ft = 0; ft < DK / 16; ++ft) {
          const f32x4 tr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kn[i][ft / 2], eye[ft % 2], zero4(), 0, 0, 0);
          bf16x4 w4;
#pragma unroll
          for (int r = 0; r < 4; ++r) w4[r] = (__bf16)tr[r];
          *reinterpret_cast<bf16x4*>(Kt + (16 * ft + lq) * PT + 16 * i + 4 * g) = w4;
        }
        const f32x4 tv = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
            __builtin_bit_cast(s16x4, vn[i]), __builtin_bit_cast(s16x4, eye4), zero4(), 0, 0, 0);
        bf16x4 v4;
#pragma unroll
        for (int r = 0; r < 4; ++r) v4[r] = (__bf16)tv[r];
        *reinterpret_cast<bf16x4*>(sVt[bs] + lq * PT + 16 * i + 4 * g) = v4;
      }
    }
    E* Tm = sT[bs];
#pragma unroll
    for (int j = 0; j < TSEG; ++j) {
      const int el = (l + 64 * j) * EPS;
      const int t = el / kTileElems, within = el - t * kTileElems;
      // tile t -> (ti, tj) by arithmetic: a lane-varying index into a table would be a memory load
      const int ti = (t >= 1) + (t >= 3) + (t >= 6), tj = t - ti * (ti + 1) / 2;
      const int row = 16 * ti + within / 16, col = 16 * tj + within % 16;
      *reinterpret_cast<u32x4*>(Tm + row * PT + col) = tseg[j];
    }
    if constexpr (!BF) {
      E* Vt = sVt[bs];
#pragma unroll
      for (int j = 0; j < VSEG; ++j) {
        const int sg = l + 64 * j, tok = sg / VSPT, part = sg - tok * VSPT;
#pragma unroll
        for (int e = 0; e < EPS; ++e) Vt[(part * EPS + e) * PT + tok] = elem_of<E>(vseg[j], e);
      }
    }
    // P^T tiles (key tile jj, query tile ii), keys after the query masked, packed per k-block;
    // each tile is formed right before its pack so at most two are live
    auto ptile = [&](int jj, int ii) {
      const f32x4 acc = N::mma(kn[jj], qn[ii], zero4());
      f32x4 r4;
#pragma unroll
      for (int r = 0; r < 4; ++r) r4[r] = (16 * jj + 4 * g + r <= 16 * ii + lq) ? acc[r] : 0.f;
      return r4;
    };
    pt[0] = Acc<E>::pack(ptile(0, 0), zero4());
    pt[1] = Acc<E>::pack(ptile(0, 1), ptile(1, 1));
    pt[2] = Acc<E>::pack(ptile(0, 2), ptile(1, 2));
    pt[3] = Acc<E>::pack(ptile(2, 2), zero4());
    pt[4] = Acc<E>::pack(ptile(0, 3), ptile(1, 3));
    pt[5] = Acc<E>::pack(ptile(2, 3), ptile(3, 3));
    if constexpr (kQInLds) {
      E* Qs = sQ[c % 3];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int s = 0; s < N::NREG; ++s) *reinterpret_cast<NR*>(Qs + (16 * i + lq) * PK + N::feat(s)) = qn[i][s];
    }
    const int nvc = min(kChunk, T - c * kChunk);
#pragma unroll
    for (int i = 0; i < 4; ++i) actk[i] = (16 * i + lq < nvc && (active == nullptr || actraw[i] != 0)) ? 1 : 0;
  };
  auto write_output = [&](int c) {
    const int bs = c & 1;
    const int nvc = min(kChunk, T - c * kChunk);
    NR ql[kQInLds ? 4 : 1][N::NREG];
    if constexpr (kQInLds) {
      const E* Qs = sQ[c % 3];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int s = 0; s < N::NREG; ++s) ql[i][s] = *reinterpret_cast<const NR*>(Qs + (16 * i + lq) * PK + N::feat(s));
    }
    const E* ho = sHo[bs] + lq * PK;
    const E* dd = sDo[bs] + lq * PT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 acc;
      if constexpr (kQInLds) {
        acc = N::mma_lds(ho, ql[i], zero4());
      } else {
        acc = N::mma_lds(ho, qr[i], zero4());
      }
      acc = Acc<E>::mma(dd, pt[i == 0 ? 0 : (i == 1 ? 1 : (i == 2 ? 2 : 4))], acc);
      if (i >= 2) acc = Acc<E>::mma(dd + 32, pt[i == 2 ? 3 : 5], acc);
      const int tok = 16 * i + lq;
      if (tok < nvc) {
        TIn* dst = o + bh_base + (size_t)c * kChunk * rstride + v0 + (tok * rstride + 4 * g);
        const bool on = actk[i] != 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = from_f32<TIn>(on ? acc[r] : 0.f);
      }
    }
  };

  // ---- chain state ----
  f32x4 hreg[HB];
  if (wave == 0) {
#pragma unroll
    for (int m = 0; m < HB; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) hreg[m][r] = s_in[((size_t)bh * DK + 16 * m + 4 * g + r) * DK + v0 + lq];
  }
  auto chain_step = [&](int c) {
    const int bs = c & 1;
    AB hb[KBF];
#pragma unroll
    for (int kb = 0; kb < KBF; ++kb) hb[kb] = Acc<E>::pack(hreg[2 * kb], 2 * kb + 1 < HB ? hreg[2 * kb + 1] : zero4());
#pragma unroll
    for (int m = 0; m < HB; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) sHo[bs][lq * PK + 16 * m + 4 * g + r] = from_f32<E>(hreg[m][r]);
    const E* K = sK[bs];
    f32x4 rr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 kh = zero4();
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) kh = Acc<E>::mma(K + (16 * i + lq) * PK + 32 * kb, hb[kb], kh);
      const E* vt = sVt[bs] + lq * PT + 16 * i + 4 * g;
#pragma unroll
      for (int r = 0; r < 4; ++r) rr[i][r] = to_f32(vt[r]) - kh[r];
    }
    const AB rb0 = Acc<E>::pack(rr[0], rr[1]);
    const AB rb1 = Acc<E>::pack(rr[2], rr[3]);
    const E* Tm = sT[bs];
    f32x4 dl[4];
    dl[0] = Acc<E>::mma(Tm + lq * PT, rb0, zero4());
    dl[1] = Acc<E>::mma(Tm + (16 + lq) * PT, rb0, zero4());
    dl[2] = Acc<E>::mma(Tm + (32 + lq) * PT + 32, rb1, Acc<E>::mma(Tm + (32 + lq) * PT, rb0, zero4()));
    dl[3] = Acc<E>::mma(Tm + (48 + lq) * PT + 32, rb1, Acc<E>::mma(Tm + (48 + lq) * PT, rb0, zero4()));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) sDo[bs][lq * PT + 16 * i + 4 * g + r] = from_f32<E>(dl[i][r]);
    const AB db0 = Acc<E>::pack(dl[0], dl[1]);
    const AB db1 = Acc<E>::pack(dl[2], dl[3]);
    const E* Kt = sKt[bs];
#pragma unroll
    for (int m = 0; m < HB; ++m) {
      hreg[m] = Acc<E>::mma(Kt + (16 * m + lq) * PT, db0, hreg[m]);
      hreg[m] = Acc<E>::mma(Kt + (16 * m + lq) * PT + 32, db1, hreg[m]);
    }
  };

  __syncthreads();  // zeroed buffers
  if (wave > 0 && hj < nc) issue_loads(hj);
  for (int it = -1; it < nc; ++it) {
    if (wave == 0) {
      if (it >= 0) chain_step(it);
    } else {
      const int cs = it + 1, co = it - 1;
      if (cs < nc && cs % NH == hj) store_chunk(cs);
      if (co >= 0 && co % NH == hj) write_output(co);
      if (it >= 0 && it % NH == hj) {  // the idle iteration of chunk it's helper
        if (it + NH < nc) issue_loads(it + NH);
        if constexpr (!kQInLds) load_rows(qr, q, q, it);
      }
    }
    __syncthreads();
  }
  if (wave > 0 && nc >= 1 && (nc - 1) % NH == hj) write_output(nc - 1);
  if (wave == 0) {
#pragma unroll
    for (int m = 0; m < HB; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_out[((size_t)bh * DK + 16 * m + 4 * g + r) * DK + v0 + lq] = hreg[m][r];
  }
}
// --------------------------------------------------------------------------------------------
// the bf16 chunk chain (head widths 32 and 64)
// --------------------------------------------------------------------------------------------
// Per chunk, with W = T K and U = T V (T the chunk's UT factor),
//   Delta = U - W H,   H' = H + K^T Delta,   O = Q H + P Delta,   P = tril(Q K^T)
// (the WY/UT form of recurrence.py:17-23 and :202-216). The chain wave runs only the two
// state-dependent levels, Delta and H', from operands that helper waves have laid out in its MFMA
// fragment order; the helpers form everything else.
//  * helper c % 7 owns chunk c: it loads Q, the compact T and the active flags into registers and
//    K and the V slice straight into its own LDS tiles (issued one chunk period ahead), reads the
//    token-major fragments of K and V from them (ds_read_b64_tr_b16), forms -W (as the accumulator
//    tiles of W^T = K^T T^T), U = T V and P^T = tril(K Q^T)^T on MFMA, hands -W, K^T and U to the
//    chain through one of three LDS slots, and once the chain has run the chunk writes
//    O^T = H^T Q^T + Delta^T P^T from the chunk's H^T and Delta;
//  * every product's accumulator tiles serve directly as the next product's operand (the "Acc"
//    k permutation); slot contents are stored lane by lane in fragment order, so the chain reads
//    them with conflict-free 16-byte loads;
//  * the waves hand chunks over through LDS flags, never a workgroup barrier: staged[c % 3] = c once
//    chunk c's operands are in their slot; done = c once the chain has run chunk c (its slot reads
//    are performed, and H^T before chunk c and Delta of chunk c are in state slot c % 3);
//    consumed[c % 3] = c once the helper has read that state slot. The helper of chunk c fills its
//    slot after done >= c - 3 and writes the output after done >= c; the chain runs chunk c after
//    staged[c % 3] >= c and consumed[c % 3] >= c - 3. Every wait is on an earlier chain step or on
//    a helper step that needs only earlier chain steps, so all end.
// Loads and stores go through buffer resources over each (b, h)'s rows: reads past the sequence's
// end return zeros and stores there are dropped, so a partial chunk needs no masking.
// --------------------------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 join4(const bf16x4& lo, const bf16x4& hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
// the Acc-permuted operand of a pair of accumulator tiles (rows 16 apart), optionally negated
__device__ __forceinline__ bf16x8 pack_acc(const f32x4& t0, const f32x4& t1, float sign = 1.f) {
  bf16x8 b;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    b[r] = (__bf16)(sign * t0[r]);
    b[4 + r] = (__bf16)(sign * t1[r]);
  }
  return b;
}

// LDS flags of the chunk hand-over. The LDS executes one wave's DS instructions in issue order, so a
// flag written after a wave's LDS reads and writes is seen by another wave only once those have
// been performed, and LDS accesses issued after a flag read that returned the awaited value see
// what the writer did before setting it. Ordering is therefore kept by the compiler alone (signal
// fences): no wait for the wave's outstanding LDS operations, which would put the LDS queue's
// latency on the chain's path. (The helpers' direct global-to-LDS loads are not DS instructions;
// their own vmcnt wait covers them.)
__device__ __forceinline__ void flag_release(int* f, int value) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __hip_atomic_store(f, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ int flag_peek(const int* f) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const int value = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return value;
}
// Wait until *f >= want, polling every 64 * SLEEP cycles, at most `limit` polls after the first
// look. The limit (2^19 polls by default, seconds) is never reached while the hand-over protocol
// holds; a wait that gives up returns false, and the caller records the fault (record_fault) and
// marks the workgroup broken, so its later outputs are written as NaN.
template <int SLEEP = 1>
__device__ __forceinline__ bool flag_wait(const int* f, int want, int limit) {
  for (int spin = 0;; ++spin) {
    if (flag_peek(f) >= want) return true;
    if (spin >= limit) return false;
    __builtin_amdgcn_s_sleep(SLEEP);
  }
}

template <typename TIn, int DK, bool CARRY>
__global__ __launch_bounds__(512) void delta_chain_bf16_kernel(const TIn* __restrict__ q, const TIn* __restrict__ k,
                                                               const TIn* __restrict__ v,
                                                               const __bf16* __restrict__ tmat,
                                                               const float* __restrict__ s_in, float* __restrict__ s_out,
                                                               TIn* __restrict__ o, const uint8_t* __restrict__ active,
                                                               const TIn* kc, const TIn* vc, const TIn* bc, int T, int H,
                                                               __bf16* __restrict__ hrec, unsigned* fault,
                                                               int wait_limit) {
  const Carried<TIn> carried{kc, vc, bc};
  using E = __bf16;
  static_assert(sizeof(TIn) == 2, "bf16 inputs");
  constexpr int NH = 7;          // helper waves: chunks in flight
  constexpr int NSL = 3;         // LDS slots of chunk operands and of chunk states
  constexpr int BV = 16;         // value columns per chain
  constexpr int NS = DK / BV;    // value slices per head
  constexpr int PK = DK + 8;     // pitch of H^T rows (elements)
  constexpr int KSEG = DK / 8;   // 16-byte segments of a K row
  constexpr int HB = DK / 16;    // 16-row tiles over dk
  constexpr int KBF = DK / 32;   // 32-wide k blocks over dk
  constexpr int FR = 64 * 8;     // elements of one lane-linear bf16 fragment

  __shared__ __align__(16) E hK[NH][64 * DK];         // each helper's K rows (segments swizzled by row)
  __shared__ __align__(16) E hV[NH][64 * BV];         // each helper's V slice rows
  __shared__ __align__(16) E sW[NSL][4 * KBF * FR];   // -W: token tile ti, dk block kb
  __shared__ __align__(16) E sKt[NSL][HB * 2 * FR];   // K^T: dk tile m, token block kb
  __shared__ __align__(16) float sU[NSL][4 * 64 * 4]; // U: token tile ti, accumulator layout
  __shared__ __align__(16) E sHo[NSL][BV * PK];       // H^T of the slice before the chunk: row = value column
  __shared__ __align__(16) E sD[NSL][2 * FR];         // Delta: token block kb, as the output's operand
  __shared__ int staged[NSL], consumed[NSL], done, broken;

  const int lg = xcd_logical_block(blockIdx.x, gridDim.x);
  const int slice = lg % NS, bh = lg / NS;
  const int b = bh / H, h = bh - b * H;
  const int v0 = slice * BV;
  // the wave index as a scalar: the role branch and the helper's LDS tiles are then wave-uniform
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
  const int lq = l & 15, g = l >> 4;
  const int nc = (T + kChunk - 1) / kChunk;
  const int rstride = H * DK;
  const size_t bh_base = ((size_t)b * T * H + h) * DK;

  // the A fragment of a row-major LDS row over one 32-wide k block in the natural k order: lane
  // group g holds k = 8 g .. 8 g + 7 (one 16-byte read)
  auto row_frag = [&](const E* arow) { return *reinterpret_cast<const bf16x8*>(arow + 8 * g); };
  auto frag_at = [&](const E* base, int f) { return *reinterpret_cast<const bf16x8*>(base + f * FR + 8 * l); };
  auto put_frag = [&](E* base, int f, const bf16x8& x) { *reinterpret_cast<bf16x8*>(base + f * FR + 8 * l) = x; };

  if (threadIdx.x < NSL) staged[threadIdx.x] = consumed[threadIdx.x] = -1;
  if (threadIdx.x == 0) {
    done = -1;
    broken = 0;
  }
  __syncthreads();
  // a bounded wait that gave up: the fault is recorded and the workgroup's later outputs are NaN
  auto await = [&](const int* f, int want) {
    if (!flag_wait<1>(f, want, wait_limit)) {
      record_fault(fault, FAULT_SCAN_CHAIN);
      flag_release(&broken, 1);
    }
  };
  auto await_slow = [&](const int* f, int want) {
    if (!flag_wait<4>(f, want, wait_limit)) {
      record_fault(fault, FAULT_SCAN_CHAIN);
      flag_release(&broken, 1);
    }
  };

  if (wave == 0) {
    // ---- the chain: Delta = U - W H, H <- H + K^T Delta per chunk ----
    __builtin_amdgcn_s_setprio(2);
    f32x4 hreg[HB];
#pragma unroll
    for (int m = 0; m < HB; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) hreg[m][r] = s_in[((size_t)bh * DK + 16 * m + 4 * g + r) * DK + v0 + lq];
    struct Ops {
      bf16x8 wf[4][KBF], kt[HB][2];
      f32x4 u[4];
    };
    auto read_ops = [&](int s, Ops& op) {
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) op.wf[ti][kb] = frag_at(sW[s], ti * KBF + kb);
        op.u[ti] = *reinterpret_cast<const f32x4*>(&sU[s][(ti * 64 + l) * 4]);
      }
#pragma unroll
      for (int m = 0; m < HB; ++m)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) op.kt[m][kb] = frag_at(sKt[s], m * 2 + kb);
    };
    // Chunk c may run once its operands are staged and its state slot has been read by the helper
    // of c - NSL. The flags of chunk c are fetched one step early; only when they are not yet set
    // does the chain poll.
    auto ready = [&](int c, int st, int cs) {
      const int s = c % NSL;
      if (st < c || cs < c - NSL) {
        await(&staged[s], c);
        await(&consumed[s], c - NSL);
      }
    };

    Ops cur;
    ready(0, -1, -1 - NSL);
    read_ops(0, cur);
    for (int it = 0; it < nc; ++it) {
      const int s = it % NSL, s2 = (it + 1) % NSL;
      const int st_next = flag_peek(&staged[s2]), cs_next = flag_peek(&consumed[s2]);
      bf16x8 hb[KBF];
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) hb[kb] = pack_acc(hreg[2 * kb], hreg[2 * kb + 1]);
      if (hrec != nullptr) {
        // the state at the chunk's start for the backward, as bf16 accumulator tiles in pairs of
        // row tiles (tiles 2 kb and 2 kb + 1 of the slice: one 16-byte store a lane and pair)
        __bf16* rec = hrec + ((size_t)bh * nc + it) * (DK * DK) + (size_t)slice * KBF * FR + 8 * l;
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) *reinterpret_cast<bf16x8*>(rec + kb * FR) = hb[kb];
      }
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) {  // H^T rows: value column lq, dk 32 kb + 4 g (+16)
        *reinterpret_cast<bf16x4*>(&sHo[s][lq * PK + 32 * kb + 4 * g]) = __builtin_shufflevector(hb[kb], hb[kb], 0, 1, 2, 3);
        *reinterpret_cast<bf16x4*>(&sHo[s][lq * PK + 32 * kb + 16 + 4 * g]) =
            __builtin_shufflevector(hb[kb], hb[kb], 4, 5, 6, 7);
      }
      f32x4 dt[4];
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        f32x4 acc = cur.u[ti];
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) acc = mfma_bf16(cur.wf[ti][kb], hb[kb], acc);
        dt[ti] = acc;
      }
      const bf16x8 db[2] = {pack_acc(dt[0], dt[1]), pack_acc(dt[2], dt[3])};
      put_frag(sD[s], 0, db[0]);
      put_frag(sD[s], 1, db[1]);
      bf16x8 kt[HB][2];
#pragma unroll
      for (int m = 0; m < HB; ++m)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) kt[m][kb] = cur.kt[m][kb];
      flag_release(&done, it);
      // the next chunk's operands load while this chunk's state update runs
      if (it + 1 < nc) {
        ready(it + 1, st_next, cs_next);
        read_ops(s2, cur);
      }
#pragma unroll
      for (int m = 0; m < HB; ++m)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) hreg[m] = mfma_bf16(kt[m][kb], db[kb], hreg[m]);
    }
    const bool bad = flag_peek(&broken) != 0;
#pragma unroll
    for (int m = 0; m < HB; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        s_out[((size_t)bh * DK + 16 * m + 4 * g + r) * DK + v0 + lq] = bad ? __builtin_nanf("") : hreg[m][r];
    return;
  }

  // ---- helpers: one chunk each, NH chunks in flight ----
  const int hj = wave - 1;
  E* myK = hK[hj];
  E* myV = hV[hj];
  // Buffer resources over this (b, h)'s rows: 32-bit offsets from a scalar base; reads past the
  // sequence's last token return zeros and stores there are dropped.
  const unsigned head_bytes = (unsigned)(((size_t)(T - 1) * rstride + DK) * sizeof(TIn));
  auto rsrc = [](const void* base, unsigned bytes) { return buffer_rsrc(base, bytes); };
  const __amdgpu_buffer_rsrc_t rq = rsrc(q + bh_base, head_bytes), rk = rsrc(k + bh_base, head_bytes);
  const __amdgpu_buffer_rsrc_t rv = rsrc(v + bh_base + v0, head_bytes - v0 * (unsigned)sizeof(TIn));
  const __amdgpu_buffer_rsrc_t ro = rsrc(o + bh_base + v0, head_bytes - v0 * (unsigned)sizeof(TIn));
  const __amdgpu_buffer_rsrc_t rt = rsrc(tmat + (size_t)bh * nc * kChunkT, (unsigned)(nc * kChunkT * 2));
  const __amdgpu_buffer_rsrc_t ra = rsrc(active != nullptr ? active + (size_t)b * T : active, (unsigned)T);
  const unsigned row_bytes = (unsigned)(rstride * sizeof(TIn));
  // K rows: 64 / KSEG rows per wave instruction, lane l on row l / KSEG, physical segment l % KSEG
  auto kswz = [](int row) { return KSEG == 8 ? ((((row >> 1) & 3) << 1) | ((row >> 3) & 1)) : ((row >> 2) & 3); };
  // lane offsets: row lq, features 4 g (q, o); row lq, T tile columns 4 g; the direct-load segments
  // (K: for even and odd instructions, whose rows differ in the swizzle's row-bit 3)
  const unsigned off_q = (unsigned)lq * row_bytes + 8u * g;    // the output's row lq, columns 4 g
  const unsigned off_qn = (unsigned)lq * row_bytes + 16u * g;  // Q row lq, features 8 g (16-byte pieces)
  const unsigned off_t = (unsigned)(lq * 16 + 4 * g) * 2u;
  const unsigned off_k0 = (unsigned)(l / KSEG) * row_bytes + 16u * (unsigned)((l % KSEG) ^ kswz(l / KSEG));
  const unsigned off_k1 = (unsigned)(l / KSEG) * row_bytes + 16u * (unsigned)((l % KSEG) ^ kswz(64 / KSEG + l / KSEG));
  const unsigned off_v = (unsigned)(l >> 1) * row_bytes + 16u * (unsigned)(l & 1);

  // Q as B fragments in the natural k order, qa[J][kb] = Q[16 J + lq][32 kb + 8 g .. + 7] (each a
  // 16-byte load: a wave instruction covers 16 rows in 64-byte runs), for two chunks: the one being
  // formed and written, and the one whose loads are in flight. The K and H^T fragments it meets in
  // the products are read in the same k order.
  bf16x8 qa0[4][KBF], qa1[4][KBF];
  bf16x4 tl[kTiles];  // the compact T tiles: row lq, columns 4 g .. + 3
  uint8_t actraw[4];
  bf16x8 pt[6];       // P^T per (key block, query tile): (0,0) (0,1) (0,2) (1,2) (0,3) (1,3)
  uint8_t actk[4];
  // With carried inputs the flags of a chunk pick each K and V row's source when its loads are
  // issued, so they are loaded one chunk of the helper ahead (actnext: token l of the helper's
  // next chunk) and kept as a wave-uniform mask per chunk in flight.
  uint8_t actnext = 1;

  // K rows and the V slice go straight into the helper's LDS tiles; Q, T and the active flags into
  // registers. The tiles are zeroed once first, so no uninitialised LDS is ever read.
  for (int i = l; i < 64 * DK / 8; i += 64) *reinterpret_cast<bf16x8*>(&myK[8 * i]) = bf16x8{};
  for (int i = l; i < 64 * BV / 8; i += 64) *reinterpret_cast<bf16x8*>(&myV[8 * i]) = bf16x8{};
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zeros land before any direct load
  auto issue_loads = [&](int c, bf16x8 (&qa)[4][KBF], uint64_t mask) {
    const unsigned cb = (unsigned)c * kChunk * row_bytes;
    if (!CARRY || mask == ~0ull) {
#pragma unroll
      for (int j = 0; j < KSEG; ++j)
        buffer_load_lds16(rk, &myK[512 * j], (j & 1) ? off_k1 : off_k0, cb + (unsigned)j * (64 / KSEG) * row_bytes);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        buffer_load_lds16(rv, &myV[512 * j], off_v, cb + (unsigned)j * 32 * row_bytes);
    } else {
      // each lane's row from the fresh or the carried tensor by a per-lane address (global direct
      // loads: a buffer resource chosen per lane would need a loop over lanes). Rows past the end
      // re-read row T - 1 (from that token's own source, so the row is finite) instead of reading
      // zeros: their T rows and columns are zero, so they add nothing, and their outputs are dropped.
      const char* kf = reinterpret_cast<const char*>(k + bh_base);
      const char* kh = reinterpret_cast<const char*>(carried.k + bh_base);
      const char* vf = reinterpret_cast<const char*>(v + bh_base + v0);
      const char* vh = reinterpret_cast<const char*>(carried.v + bh_base + v0);
#pragma unroll
      for (int j = 0; j < KSEG; ++j) {
        const int t = min(c * kChunk + l / KSEG + j * (64 / KSEG), T - 1);
        const unsigned seg = ((j & 1) ? off_k1 : off_k0) - (unsigned)(l / KSEG) * row_bytes;
        const char* src = (((mask >> (t - c * kChunk)) & 1) ? kf : kh) + (size_t)t * row_bytes + seg;
        load_lds16(src, &myK[512 * j]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = min(c * kChunk + (l >> 1) + 32 * j, T - 1);
        const char* src = (((mask >> (t - c * kChunk)) & 1) ? vf : vh) + (size_t)t * row_bytes + 16u * (l & 1);
        load_lds16(src, &myV[512 * j]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb)
        qa[i][kb] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, off_qn + 64u * kb, cb + 16u * i * row_bytes, 0));
    const unsigned tb = (unsigned)c * kChunkT * 2u;
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
      tl[t] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(rt, off_t + 512u * t, tb, 0));
    if constexpr (CARRY) {
      if (c + NH < nc) actnext = __builtin_amdgcn_raw_buffer_load_b8(ra, (unsigned)l, (unsigned)(c + NH) * kChunk, 0);
    } else if (active != nullptr) {
#pragma unroll
      for (int i = 0; i < 4; ++i) actraw[i] = __builtin_amdgcn_raw_buffer_load_b8(ra, (unsigned)(16 * i + lq), (unsigned)c * kChunk, 0);
    }
  };

  // element offset of (row, column) in a helper's K tile: unpadded rows, 16-byte segments XOR-swizzled
  // by row bits so that both the row-fragment and the transposed reads spread over the 64 banks
  auto kat = [&](int row, int col) { return row * DK + (((col >> 3) ^ kswz(row)) << 3) + (col & 7); };
  auto kfrag = [&](int row, int kb) {  // the A fragment of K row `row`, dk block kb, natural k order
    return *reinterpret_cast<const bf16x8*>(&myK[kat(row, 32 * kb + 8 * g)]);
  };
  auto ktr = [&](int r0, int m) {  // column 16 m + lq of token rows r0 + 4 g .. + 3 (transposed read)
    return read_tr16<bf16x4>(&myK[kat(r0 + 4 * g + (lq >> 2), 16 * m + 4 * (lq & 3))]);
  };

  // Chunk c's operands into state slot c % NSL (once the chain is done with the slot's previous
  // chunk); P^T kept in registers for the output
  auto form = [&](int c, const bf16x8 (&qa)[4][KBF], uint64_t mask, uint64_t& next_mask) {
    const int nvc = min(kChunk, T - c * kChunk);
    const int s = c % NSL;
    // The direct loads of K and V count as outstanding vector memory operations until they have
    // written LDS. Buffer loads and stores of a wave complete in issue order, and the only ones
    // issued after this chunk's loads are the previous chunk's four output stores: waiting for
    // all but the last four lets those stores drain meanwhile (the helper's first chunk has none;
    // the carried variant's per-lane global loads wait for everything).
    if (CARRY || c == hj)
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    else
      __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4)
    wave_sync();
    if constexpr (CARRY) {
#pragma unroll
      for (int i = 0; i < 4; ++i) actk[i] = (16 * i + lq < nvc && ((mask >> (16 * i + lq)) & 1)) ? 1 : 0;
      next_mask = __builtin_amdgcn_ballot_w64(actnext != 0);  // the helper's next chunk (arrived above)
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) actk[i] = (16 * i + lq < nvc && (active == nullptr || actraw[i] != 0)) ? 1 : 0;
    }
    // token-major operands: ktf[m][kb] = column 16 m + lq of token rows 32 kb + 4 g (+16)
    bf16x8 ktf[HB][2], vtf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int m = 0; m < HB; ++m) ktf[m][kb] = join4(ktr(32 * kb, m), ktr(32 * kb + 16, m));
      vtf[kb] = join4(read_tr16_rows<bf16x4>(myV, BV, 32 * kb, 0), read_tr16_rows<bf16x4>(myV, BV, 32 * kb + 16, 0));
    }
    // P^T = tril(K Q^T)^T tiles (key tile jj, query tile ii); only diagonal tiles hold keys after the query
    auto ptile = [&](int jj, int ii) {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) acc = mfma_bf16(kfrag(16 * jj + lq, kb), qa[ii][kb], acc);
      if (jj == ii) {
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = (4 * g + r <= lq) ? acc[r] : 0.f;
      }
      return acc;
    };
    pt[0] = pack_acc(ptile(0, 0), zero4());
    pt[1] = pack_acc(ptile(0, 1), ptile(1, 1));
    pt[2] = pack_acc(ptile(0, 2), ptile(1, 2));
    pt[3] = pack_acc(ptile(2, 2), zero4());
    pt[4] = pack_acc(ptile(0, 3), ptile(1, 3));
    pt[5] = pack_acc(ptile(2, 3), ptile(3, 3));
    // T's operand fragments (row tile, token block): (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
    const bf16x4 z4{};
    const bf16x8 tf[6] = {join4(tl[0], z4), join4(tl[1], tl[2]), join4(tl[3], tl[4]),
                          join4(tl[5], z4), join4(tl[6], tl[7]), join4(tl[8], tl[9])};
    await_slow(&done, c - NSL);  // the chain is done with the slot's previous chunk
    // W^T = K^T T^T (dk tile m, token tile ti): its tile pairs over dk are the chain's -W operand
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int f0 = ti == 0 ? 0 : (ti == 1 ? 1 : (ti == 2 ? 2 : 4));
      f32x4 wt[HB];
#pragma unroll
      for (int m = 0; m < HB; ++m) {
        wt[m] = mfma_bf16(ktf[m][0], tf[f0], zero4());
        if (ti >= 2) wt[m] = mfma_bf16(ktf[m][1], tf[f0 + 1], wt[m]);
      }
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) put_frag(sW[s], ti * KBF + kb, pack_acc(wt[2 * kb], wt[2 * kb + 1], -1.f));
      // U = T V (token tile ti), in the accumulator layout of Delta
      f32x4 u = mfma_bf16(tf[f0], vtf[0], zero4());
      if (ti >= 2) u = mfma_bf16(tf[f0 + 1], vtf[1], u);
      *reinterpret_cast<f32x4*>(&sU[s][(ti * 64 + l) * 4]) = u;
    }
#pragma unroll
    for (int m = 0; m < HB; ++m)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) put_frag(sKt[s], m * 2 + kb, ktf[m][kb]);
    flag_release(&staged[s], c);
  };

  // O^T = H^T Q^T + Delta^T P^T for chunk c, from state slot c % NSL; rows past the sequence's end
  // fall outside the output's buffer range and are dropped
  auto write_output = [&](int c, const bf16x8 (&qa)[4][KBF]) {
    const int s = c % NSL;
    bf16x8 hf[KBF];
#pragma unroll
    for (int kb = 0; kb < KBF; ++kb) hf[kb] = row_frag(&sHo[s][lq * PK + 32 * kb]);
    const bf16x8 d0 = frag_at(sD[s], 0), d1 = frag_at(sD[s], 1);
    flag_release(&consumed[s], c);  // after the reads above: the chain may reuse the slot
    const bool bad = flag_peek(&broken) != 0;
    const unsigned cb = (unsigned)c * kChunk * row_bytes;
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      const int p0 = J == 0 ? 0 : (J == 1 ? 1 : (J == 2 ? 2 : 4));
      f32x4 acc = mfma_bf16(d0, pt[p0], zero4());
      if (J >= 2) acc = mfma_bf16(d1, pt[p0 + 1], acc);
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) acc = mfma_bf16(hf[kb], qa[J][kb], acc);
      const bool on = actk[J] != 0;
      typedef TIn O4 __attribute__((ext_vector_type(4)));
      O4 w4;
#pragma unroll
      for (int r = 0; r < 4; ++r) w4[r] = from_f32<TIn>(bad ? __builtin_nanf("") : (on ? acc[r] : 0.f));
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, w4), ro, off_q, cb + 16u * J * row_bytes, 0);
    }
  };

  // chunk c: form its operands, issue the loads of chunk c + NH (their latency hidden behind the
  // wait for the chain), then write its output
  auto run = [&](int c, const bf16x8 (&qc)[4][KBF], bf16x8 (&qn)[4][KBF], uint64_t mc, uint64_t& mn) {
    form(c, qc, mc, mn);
    if (c + NH < nc) issue_loads(c + NH, qn, mn);
    await_slow(&done, c);
    write_output(c, qc);
  };
  uint64_t m0 = ~0ull, m1 = ~0ull;  // the flags of the chunks whose loads are in flight
  if constexpr (CARRY) {
    if (hj < nc) m0 = __builtin_amdgcn_ballot_w64(__builtin_amdgcn_raw_buffer_load_b8(ra, (unsigned)l, (unsigned)hj * kChunk, 0) != 0);
  }
  if (hj < nc) issue_loads(hj, qa0, m0);
  for (int c = hj; c < nc; c += 2 * NH) {
    run(c, qa0, qa1, m0, m1);
    if (c + NH < nc) run(c + NH, qa1, qa0, m1, m0);
  }
}

#include "scan_segments.h"

// --------------------------------------------------------------------------------------------
// host side
// --------------------------------------------------------------------------------------------
// beta given as write-strength logits (with an optional per-token modulator), turned into beta in the
// kernels' loads (recurrence.py:34-88)
struct Strength {
  const float* m = nullptr;
  float alpha = 0.f;
  int logits = 0;
};

bool chunked_width(int D, bool fp32) { return D == 16 || D == 32 || D == 64 || (D == 128 && !fp32); }
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
                  const uint8_t* active, Carried<TIn> carried, int B, int T, int H, int D, hipStream_t stream,
                  const char* who, Strength strength = {}) {
  const int groups = (D + 63) / 64;
  dim3 grid((unsigned)(B * H), (unsigned)groups);
  hipLaunchKernelGGL(delta_serial_kernel<TIn>, grid, dim3(64 * groups), 0, stream, q, k, v, beta, s_in, s_out, o,
                     active, carried.k, carried.v, carried.beta, T, H, D, groups, strength.m, strength.alpha,
                     strength.logits, (float*)nullptr);
  return check_launch(who);
}

size_t workspace_bytes(int B, int T, int H, int D, bool fp32) {
  if (B <= 0 || H <= 0 || T < kSerialBelow || !chunked_width(D, fp32)) return 0;
  if ((size_t)T * H * D >= ((size_t)1 << 31)) return 0;  // 32-bit row offsets in the chain kernel
  const size_t nc = (size_t)(T + kChunk - 1) / kChunk;
  size_t bytes = (size_t)B * H * nc * kChunkT * (fp32 ? sizeof(float) : sizeof(uint16_t));
  if (!fp32 && D == 64) {  // the segmented scan's maps and the copies of S0 follow the UT factors
    const SegShape sh = seg_shape(B, H, T);
    if (sh.nseg > 1) bytes += (size_t)B * H * ((sh.nseg - 1) * kSegMapBytes + 64 * 64 * sizeof(float));
  }
  return bytes;
}

// The segmented scan (bf16, head width 64): the map pass over every segment but the last, then the
// output pass over all of them. tmat is the workspace's start; the maps follow the UT factors.
template <bool CARRY>
void launch_segments(const __bf16* q, const __bf16* k, const __bf16* v, const float* s_in, float* s_out, __bf16* o,
                     __bf16* tmat, const uint8_t* active, Carried<__bf16> carried, int B, int T, int H,
                     hipStream_t stream, __bf16* hrec) {
  const SegShape sh = seg_shape(B, H, T);
  const size_t nc = (size_t)(T + kChunk - 1) / kChunk;
  float* maps = reinterpret_cast<float*>(tmat + (size_t)B * H * nc * kChunkT);
  float* s0copy = maps + (size_t)B * H * (sh.nseg - 1) * (kSegMapBytes / sizeof(float));
  if (sh.nseg > 1)
    hipLaunchKernelGGL((delta_seg_kernel<kSegMaps, CARRY>), dim3((unsigned)(B * H * (sh.nseg - 1))), dim3(512), 0,
                       stream, q, k, v, tmat, s_in, s_out, o, active, maps, s0copy, T, H, sh.nseg, sh.seglen,
                       (__bf16*)nullptr, fault_record(), wait_limit(), carried.k, carried.v);
  hipLaunchKernelGGL((delta_seg_kernel<kSegOutputs, CARRY>), dim3((unsigned)(B * H * sh.nseg)), dim3(512), 0, stream,
                     q, k, v, tmat, s_in, s_out, o, active, maps, s0copy, T, H, sh.nseg, sh.seglen, hrec,
                     fault_record(), wait_limit(), carried.k, carried.v);
}

template <typename TIn, typename E, int DK, bool CARRY>
void launch_chunked(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, float* s_out, TIn* o,
                    E* tmat, const uint8_t* active, Carried<TIn> carried, int B, int T, int H, hipStream_t stream,
                    Strength strength, __bf16* hrec) {
  const int nc = (T + kChunk - 1) / kChunk;
  const int total = B * H * nc;
  hipLaunchKernelGGL((delta_prep_kernel<TIn, E, DK, CARRY>), dim3((unsigned)((total + 3) / 4)), dim3(256), 0, stream, k,
                     beta, tmat, active, carried.k, carried.v, carried.beta, T, H, total, strength.m, strength.alpha,
                     strength.logits);
  if constexpr (std::is_same<TIn, __bf16>::value && DK == 64) {
    // by shape: the value-slice chains while they fit one workgroup a CU (B H D/16 <= kSegBlocks),
    // where their four CUs a head outrun one whole-head workgroup a segment; the segments beyond
    const int form = scan_segments();
    if (form == 1 || (form == 2 && B * H * (DK / 16) > kSegBlocks)) {
      launch_segments<CARRY>(q, k, v, s_in, s_out, o, tmat, active, carried, B, T, H, stream, hrec);
      return;
    }
  }
  if constexpr (sizeof(E) == 2 && DK >= 32 && DK <= 64) {  // (at 128 the staging registers would spill)
    hipLaunchKernelGGL((delta_chain_bf16_kernel<TIn, DK, CARRY>), dim3((unsigned)(B * H * (DK / 16))), dim3(512), 0,
                       stream, q, k, v, tmat, s_in, s_out, o, active, carried.k, carried.v, carried.beta, T, H,
                       hrec, fault_record(), wait_limit());
  } else {
    hipLaunchKernelGGL((delta_chain_kernel<TIn, E, DK, CARRY>), dim3((unsigned)(B * H * (DK / 16))),
                       dim3(64 * (ChainShape<E, DK>::NH + 1)), 0, stream, q, k, v, tmat, s_in, s_out, o, active,
                       carried.k, carried.v, carried.beta, T, H);
  }
}

template <typename TIn, typename E, int DK>
void launch_chunked(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, float* s_out, TIn* o,
                    E* tmat, const uint8_t* active, Carried<TIn> carried, int B, int T, int H, hipStream_t stream,
                    Strength strength, __bf16* hrec) {
  if (carried.k != nullptr)
    launch_chunked<TIn, E, DK, true>(q, k, v, beta, s_in, s_out, o, tmat, active, carried, B, T, H, stream, strength,
                                     hrec);
  else
    launch_chunked<TIn, E, DK, false>(q, k, v, beta, s_in, s_out, o, tmat, active, carried, B, T, H, stream, strength,
                                      hrec);
}

template <typename TIn, typename E>
int delta_scan(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, TIn* o, float* s_out,
               void* workspace, size_t ws_bytes, const uint8_t* active, Carried<TIn> carried, int B, int T, int H, int D,
               void* stream_ptr, const char* who, Strength strength = {}, __bf16* hrec = nullptr) {
  int st = check_common(q, k, v, beta, s_in, s_out, o, B, T, H, D, who);
  if (st != OK || B == 0 || H == 0) return st;
  if (carried.k != nullptr || carried.v != nullptr || carried.beta != nullptr) {
    if (!carried.k || !carried.v || !carried.beta)
      return fail(ERR_ARG, "%s: the carried k, v and beta come together", who);
    if (!active) return fail(ERR_ARG, "%s: carried inputs need the active flags", who);
    if ((reinterpret_cast<uintptr_t>(carried.k) | reinterpret_cast<uintptr_t>(carried.v)) & 15)
      return fail(ERR_ARG, "%s: the carried k and v must be 16-byte aligned", who);
  }
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  if (T == 0) {
    if (s_in != s_out) {
      hipError_t err = hipMemcpyAsync(s_out, s_in, (size_t)B * H * D * D * sizeof(float), hipMemcpyDeviceToDevice, stream);
      if (err != hipSuccess) return fail(ERR_LAUNCH, "%s: state copy failed: %s", who, hipGetErrorString(err));
    }
    return OK;
  }
  const size_t need = workspace_bytes(B, T, H, D, sizeof(E) == 4);
  if (need == 0)
    return launch_serial<TIn>(q, k, v, beta, s_in, s_out, o, active, carried, B, T, H, D, stream, who, strength);
  if (workspace == nullptr || ws_bytes < need)
    return fail(ERR_ARG, "%s: workspace of %zu bytes given, %zu needed", who, workspace ? ws_bytes : (size_t)0, need);
  // the chunked kernels move q, k, v, o rows and the workspace in 16-byte pieces
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
       reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(workspace)) & 15)
    return fail(ERR_ARG, "%s: q, k, v, o and the workspace must be 16-byte aligned", who);
  E* tmat = reinterpret_cast<E*>(workspace);
  switch (D) {
    case 16: launch_chunked<TIn, E, 16>(q, k, v, beta, s_in, s_out, o, tmat, active, carried, B, T, H, stream, strength, hrec); break;
    case 32: launch_chunked<TIn, E, 32>(q, k, v, beta, s_in, s_out, o, tmat, active, carried, B, T, H, stream, strength, hrec); break;
    case 64: launch_chunked<TIn, E, 64>(q, k, v, beta, s_in, s_out, o, tmat, active, carried, B, T, H, stream, strength, hrec); break;
    default:
      if constexpr (sizeof(E) == 2)
        launch_chunked<TIn, E, 128>(q, k, v, beta, s_in, s_out, o, tmat, active, carried, B, T, H, stream, strength, hrec);
      break;
  }
  return check_launch(who);
}

template <typename TIn>
int delta_step(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* s_in, float* s_out, TIn* o,
               const uint8_t* active, int B, int H, int D, void* stream_ptr, const char* who) {
  int st = check_common(q, k, v, beta, s_in, s_out, o, B, 1, H, D, who);
  if (st != OK || B == 0 || H == 0) return st;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  bool fast;
  if constexpr (sizeof(TIn) == 4) {
    fast = delta_step_fast_f32(q, k, v, beta, s_in, s_out, o, active, B, H, D, stream);
  } else {
    fast = delta_step_fast_bf16(q, k, v, beta, s_in, s_out, o, active, B, H, D, stream);
  }
  if (fast) return check_launch(who);
  return launch_serial<TIn>(q, k, v, beta, s_in, s_out, o, active, Carried<TIn>{}, B, 1, H, D, stream, who);
}

}  // namespace

// The states at every 64-token chunk's start (ckpt: [B, H, ceil(T / 64), D, D] fp32), from the
// token-serial forward with its outputs dropped; s_out receives the final state. For the backward
// at head widths the chunked kernels do not tile.
int delta_scan_checkpoints_bf16(const __bf16* q, const __bf16* k, const __bf16* v, const __bf16* beta,
                                const float* s_in, float* s_out, float* ckpt, int B, int T, int H, int D,
                                hipStream_t stream) {
  const int groups = (D + 63) / 64;
  hipLaunchKernelGGL(delta_serial_kernel<__bf16>, dim3((unsigned)(B * H), (unsigned)groups), dim3(64 * groups), 0,
                     stream, q, k, v, beta, s_in, s_out, (__bf16*)nullptr, (const uint8_t*)nullptr,
                     (const __bf16*)nullptr, (const __bf16*)nullptr, (const __bf16*)nullptr, T, H, D, groups,
                     (const float*)nullptr, 0.f, 0, ckpt);
  return OK;
}
int delta_scan_checkpoints_f32(const float* q, const float* k, const float* v, const float* beta, const float* s_in,
                               float* s_out, float* ckpt, int B, int T, int H, int D, hipStream_t stream) {
  const int groups = (D + 63) / 64;
  hipLaunchKernelGGL(delta_serial_kernel<float>, dim3((unsigned)(B * H), (unsigned)groups), dim3(64 * groups), 0,
                     stream, q, k, v, beta, s_in, s_out, (float*)nullptr, (const uint8_t*)nullptr,
                     (const float*)nullptr, (const float*)nullptr, (const float*)nullptr, T, H, D, groups,
                     (const float*)nullptr, 0.f, 0, ckpt);
  return OK;
}

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
                                    static_cast<__bf16*>(o), state_out, workspace, workspace_bytes, active,
                                    vsp::Carried<__bf16>{}, B, T, H, D, stream, "vsp_delta_scan_bf16");
}

// The chunk-start states the bf16 forward can record for the backward: widths 32 and 64 on the
// chunked path, one [D x D] bf16 block a (b, h, chunk) in the backward's accumulator-pair order.
extern "C" size_t vsp_delta_scan_records_bytes(int B, int T, int H, int D) {
  if (!(D == 32 || D == 64) || vsp::workspace_bytes(B, T, H, D, false) == 0) return 0;
  const size_t nc = (size_t)(T + vsp::kChunk - 1) / vsp::kChunk;
  return (size_t)B * H * nc * D * D * sizeof(uint16_t);
}

extern "C" int vsp_delta_scan_record_bf16(const void* q, const void* k, const void* v, const void* beta,
                                          const float* state_in, void* o, float* state_out, void* workspace,
                                          size_t workspace_bytes, const uint8_t* active, void* records,
                                          size_t records_bytes, int B, int T, int H, int D, void* stream) {
  const char* who = "vsp_delta_scan_record_bf16";
  const size_t need = vsp_delta_scan_records_bytes(B, T, H, D);
  if (need == 0)
    return vsp::fail(vsp::ERR_UNSUPPORTED, "%s: no records at B=%d T=%d H=%d D=%d (widths 32 and 64, T >= %d)", who, B,
                     T, H, D, vsp::kSerialBelow);
  if (records == nullptr || records_bytes < need || (reinterpret_cast<uintptr_t>(records) & 15))
    return vsp::fail(vsp::ERR_ARG, "%s: records of %zu bytes (16-byte aligned) needed, %zu given", who, need,
                     records ? records_bytes : (size_t)0);
  return delta_scan<__bf16, __bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                                    static_cast<const __bf16*>(v), static_cast<const __bf16*>(beta), state_in,
                                    static_cast<__bf16*>(o), state_out, workspace, workspace_bytes, active,
                                    vsp::Carried<__bf16>{}, B, T, H, D, stream, who, vsp::Strength{},
                                    static_cast<__bf16*>(records));
}

extern "C" int vsp_delta_scan_carried_bf16(const void* q, const void* k, const void* v, const void* beta,
                                           const void* k_carried, const void* v_carried, const void* beta_carried,
                                           const float* state_in, void* o, float* state_out, void* workspace,
                                           size_t workspace_bytes, const uint8_t* active, int B, int T, int H, int D,
                                           void* stream) {
  using T16 = __bf16;
  const vsp::Carried<T16> carried{static_cast<const T16*>(k_carried), static_cast<const T16*>(v_carried),
                                  static_cast<const T16*>(beta_carried)};
  return delta_scan<T16, T16>(static_cast<const T16*>(q), static_cast<const T16*>(k), static_cast<const T16*>(v),
                              static_cast<const T16*>(beta), state_in, static_cast<T16*>(o), state_out, workspace,
                              workspace_bytes, active, carried, B, T, H, D, stream, "vsp_delta_scan_carried_bf16");
}

extern "C" int vsp_delta_scan_f32(const float* q, const float* k, const float* v, const float* beta,
                                  const float* state_in, float* o, float* state_out, void* workspace,
                                  size_t workspace_bytes, const uint8_t* active, int B, int T, int H, int D,
                                  void* stream) {
  return delta_scan<float, float>(q, k, v, beta, state_in, o, state_out, workspace, workspace_bytes, active,
                                  vsp::Carried<float>{}, B, T, H, D, stream, "vsp_delta_scan_f32");
}

extern "C" int vsp_delta_scan_carried_f32(const float* q, const float* k, const float* v, const float* beta,
                                          const float* k_carried, const float* v_carried, const float* beta_carried,
                                          const float* state_in, float* o, float* state_out, void* workspace,
                                          size_t workspace_bytes, const uint8_t* active, int B, int T, int H, int D,
                                          void* stream) {
  return delta_scan<float, float>(q, k, v, beta, state_in, o, state_out, workspace, workspace_bytes, active,
                                  vsp::Carried<float>{k_carried, v_carried, beta_carried}, B, T, H, D, stream,
                                  "vsp_delta_scan_carried_f32");
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

extern "C" int vsp_delta_scan_logits_bf16(const void* q, const void* k, const void* v, const void* logits,
                                          const float* m, float alpha, const float* state_in, void* o,
                                          float* state_out, void* workspace, size_t workspace_bytes,
                                          const uint8_t* active, int B, int T, int H, int D, void* stream) {
  if (!(alpha >= 0.f) || alpha == __builtin_inff())
    return vsp::fail(vsp::ERR_ARG, "vsp_delta_scan_logits_bf16: alpha %g is not finite and non-negative", alpha);
  vsp::Strength strength;
  strength.m = m;
  strength.alpha = alpha;
  strength.logits = 1;
  return delta_scan<__bf16, __bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                                    static_cast<const __bf16*>(v), static_cast<const __bf16*>(logits), state_in,
                                    static_cast<__bf16*>(o), state_out, workspace, workspace_bytes, active,
                                    vsp::Carried<__bf16>{}, B, T, H, D, stream, "vsp_delta_scan_logits_bf16", strength);
}

extern "C" int vsp_delta_scan_logits_f32(const float* q, const float* k, const float* v, const float* logits,
                                         const float* m, float alpha, const float* state_in, float* o,
                                         float* state_out, void* workspace, size_t workspace_bytes,
                                         const uint8_t* active, int B, int T, int H, int D, void* stream) {
  if (!(alpha >= 0.f) || alpha == __builtin_inff())
    return vsp::fail(vsp::ERR_ARG, "vsp_delta_scan_logits_f32: alpha %g is not finite and non-negative", alpha);
  vsp::Strength strength;
  strength.m = m;
  strength.alpha = alpha;
  strength.logits = 1;
  return delta_scan<float, float>(q, k, v, logits, state_in, o, state_out, workspace, workspace_bytes, active,
                                  vsp::Carried<float>{}, B, T, H, D, stream, "vsp_delta_scan_logits_f32", strength);
}
