// The delta-rule scan's backward on CDNA4 (gfx950): d q, d k, d v, d beta and d state.
//
// The gradients of the chunked scan (reference vesper/recurrence.py:166-217, run on CUDA by fla-core
// behind vesper/kernels/delta_scan.py:132-187 with its backward). Per chunk of C = 64 tokens, with H
// the state at its start, G the gradient of the state at its end, A = tril(diag(beta) K K^T, -1),
// L = (I + A)^-1, T = L diag(beta), R = V - K H, Delta = T R, P = tril(Q K^T) (diagonal included):
//   dDelta = K G + P^T dO,  dR = T^T dDelta (= dV),  dQ = dO H^T + tril(dO Delta^T) K,
//   dT = dDelta R^T,  dA = tril(-L^T (dT diag(beta)) L^T, -1),  M = diag(beta) dA,
//   dK = Delta G^T + tril(dO Delta^T)^T Q - dR H^T + (M + M^T) K,
//   dbeta_j = sum_i dT_ij L_ij + sum_m dA_jm k_j . k_m,
// and the state's gradient at the chunk's start G + Q^T dO - K^T dR = G - W^T (K G) + Y with
// W = T K, Y = Q^T dO - W^T P^T dO.
//
// Both chains are one matrix product per chunk: with U = T V, N = -K^T W and B = K^T U,
//   H_next = H + N H + B        (forward: the state at the next chunk's start),
//   G_start = G + N^T G + Y     (reverse: the state's gradient at the chunk's start).
// Three kernels, no atomics (fp32 arithmetic; bf16 inputs multiply on bf16 MFMA):
// - scan_bwd_prep_kernel, per (b, h, chunk): L, N and N^T (bf16, in the chains' MFMA operand
//   order), B and Y (fp32, in the chains' accumulator order) into the workspace;
// - scan_bwd_chains_kernel, one wave per (b, h, 16 value columns) and direction (value columns
//   evolve independently): the states at the chunk starts and the state's gradients at the
//   chunk ends, and the initial state's gradient; the state slice stays in MFMA accumulators and
//   N's fragments come straight from global memory into a register ring, several chunks ahead;
// - scan_bwd_chunk_kernel, per (b, h, chunk): every token gradient of the chunk.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kC = 64;       // tokens per chunk
constexpr int kPC = kC + 4;  // pitch (floats) of a [.][64] LDS matrix

// mm16 over the k blocks kb0 .. kb1 - 1 of 16 (k = 16 kb0 .. 16 kb1 - 1): the part of a product
// that a triangular operand leaves nonzero. Same operand conventions as mm16.
template <bool TA, bool TB, bool BF = false>
__device__ __forceinline__ f32x4 mm16k(const float* X, int ldx, const float* Y, int ldy, int kb0, int kb1, f32x4 acc,
                                       const float* yscale = nullptr) {
  for (int kb = kb0; kb < kb1; ++kb) {
    const int k0 = 16 * kb;
    acc = mm16<TA, TB, BF>(TA ? X + k0 * ldx : X + k0, ldx, TB ? Y + k0 : Y + k0 * ldy, ldy, 16, acc,
                       yscale != nullptr ? yscale + k0 : nullptr);
  }
  return acc;
}

// Within a wave, LDS writes of any lane are visible to later LDS reads of any lane.
__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// element (row, col) of an accumulator tile for register r of this lane
__device__ __forceinline__ int tile_row(int r) { return 4 * ((threadIdx.x & 63) >> 4) + r; }
__device__ __forceinline__ int tile_col() { return threadIdx.x & 15; }

// Staging into LDS is split in two: fetch() issues a workgroup's global loads into registers,
// put() converts and writes them to LDS. A kernel fetches every operand before it puts the first,
// so all its loads are in flight together: with one workgroup per CU nothing else hides a load's
// latency. Loads are unconditional (rows past N re-read row N - 1, selected to zero in put()), so
// none sits behind a per-lane branch, which would make it wait for every earlier load. The kernels
// run 256 threads a workgroup.
constexpr int kThreads = 256;

template <typename TIn>
__device__ __forceinline__ void load4_f32(const TIn* p, float (&x)[4]) {
  if constexpr (sizeof(TIn) == 2) {
    typedef TIn V4 __attribute__((ext_vector_type(4)));
    const V4 v = *reinterpret_cast<const V4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = to_f32(v[j]);
  } else {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = v[j];
  }
}

// chunk rows t0 .. t0 + 63 of a [B, N, H, D] tensor (head h of batch row b) into LDS [64][ld] as
// fp32; rows past N are zero, and with `active` so are inactive tokens' rows
template <typename TIn, int D, int NTH = kThreads>
struct ChunkRows {
  typedef TIn V4 __attribute__((ext_vector_type(4)));
  static constexpr int kN = kC * D / 4, kIt = (kN + NTH - 1) / NTH;
  V4 raw[kIt];
  uint8_t act[kIt];  // the token's flag; without `active` a byte of src, not looked at
  bool masked;
  __device__ __forceinline__ void fetch(const TIn* src, int b, int h, int t0, int N, int H,
                                        const uint8_t* active = nullptr) {
    masked = active != nullptr;
    const uint8_t* flags = masked ? active + (size_t)b * N : reinterpret_cast<const uint8_t*>(src);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = min((int)threadIdx.x + NTH * it, kN - 1), row = e / (D / 4), c = 4 * (e % (D / 4));
      const int tc = min(t0 + row, N - 1);
      raw[it] = *reinterpret_cast<const V4*>(src + (((size_t)b * N + tc) * H + h) * D + c);
      act[it] = flags[masked ? tc : 0];
    }
  }
  __device__ __forceinline__ void put(float* dst, int ld, int t0, int N) const {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = threadIdx.x + NTH * it, row = e / (D / 4), c = 4 * (e % (D / 4));
      const bool ok = t0 + row < N && (!masked || act[it] != 0);
      f32x4 x;
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = ok ? to_f32(raw[it][j]) : 0.f;
      if (kN % NTH == 0 || e < kN) *reinterpret_cast<f32x4*>(dst + row * ld + c) = x;
    }
  }
};

// beta of the chunk's tokens (zero past N) into LDS [64]
template <typename TIn>
struct ChunkBeta {
  TIn raw;
  __device__ __forceinline__ void fetch(const TIn* beta, int b, int h, int t0, int N, int H) {
    raw = beta[((size_t)b * N + min(t0 + (int)(threadIdx.x & (kC - 1)), N - 1)) * H + h];
  }
  __device__ __forceinline__ void put(float* dst, int t0, int N) const {
    const int r = threadIdx.x;
    if (r < kC) dst[r] = t0 + r < N ? to_f32(raw) : 0.f;
  }
};

// a [R][D] fp32 global matrix (row pitch D) into LDS [R][ld]
template <int R, int D, int NTH = kThreads>
struct MatRows {
  static constexpr int kN = R * D / 4, kIt = (kN + NTH - 1) / NTH;
  f32x4 raw[kIt];
  __device__ __forceinline__ void fetch(const float* src) {
#pragma unroll
    for (int it = 0; it < kIt; ++it)
      raw[it] = *reinterpret_cast<const f32x4*>(src + 4 * min((int)threadIdx.x + NTH * it, kN - 1));
  }
  __device__ __forceinline__ void put(float* dst, int ld) const {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = threadIdx.x + NTH * it;
      if (kN % NTH == 0 || e < kN) *reinterpret_cast<f32x4*>(dst + (4 * e / D) * ld + 4 * e % D) = raw[it];
    }
  }
};

// a [D][D] fp32 matrix stored in accumulator order (accfrag: value slice s = column tile) into
// LDS [D][ld], row-major
template <int D, int NTH = kThreads>
struct AccRows {
  static constexpr int NT = D / 16, kN = D * D / 4, kIt = (kN + NTH - 1) / NTH;
  f32x4 raw[kIt];
  __device__ __forceinline__ void fetch(const float* src) {
#pragma unroll
    for (int it = 0; it < kIt; ++it)
      raw[it] = *reinterpret_cast<const f32x4*>(src + 4 * min((int)threadIdx.x + NTH * it, kN - 1));
  }
  __device__ __forceinline__ void put(float* dst, int ld) const {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = threadIdx.x + NTH * it;  // = (s NT + rt) 64 + lane
      if (kN % NTH == 0 || e < kN) {
        const int lane = e & 63, st = e >> 6, sl = st / NT, rt = st - sl * NT;
        const int row = 16 * rt + 4 * (lane >> 4), col = 16 * sl + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[(row + r) * ld + col] = raw[it][r];
      }
    }
  }
};

// workspace layout, per (b, h, chunk), in floats: L [64][64]; NF, NR [D][D] (the chains' A
// operands); B, Y, Hs, dHs [D][D] in accumulator order. On the bf16 entry NF, NR, B and Y hold
// bf16, and so do L, Hs and dHs at head widths 32 and 64 (in the first half of their blocks).
template <int D> struct Ws {
  static constexpr size_t kL = (size_t)kC * kC, kS = (size_t)D * D;
  static constexpr size_t kPer = kL + 6 * kS;
  __device__ __forceinline__ static float* L(float* ws, size_t chunk) { return ws + chunk * kPer; }
  // N's A-operand fragments for the forward chain (NF) and N^T's for the reverse one (NR)
  __device__ __forceinline__ static float* NF(float* ws, size_t chunk) { return ws + chunk * kPer + kL; }
  __device__ __forceinline__ static float* NR(float* ws, size_t chunk) { return ws + chunk * kPer + kL + kS; }
  __device__ __forceinline__ static float* B(float* ws, size_t chunk) { return ws + chunk * kPer + kL + 2 * kS; }
  __device__ __forceinline__ static float* Y(float* ws, size_t chunk) { return ws + chunk * kPer + kL + 3 * kS; }
  __device__ __forceinline__ static float* Hs(float* ws, size_t chunk) { return ws + chunk * kPer + kL + 4 * kS; }
  __device__ __forceinline__ static float* dHs(float* ws, size_t chunk) { return ws + chunk * kPer + kL + 5 * kS; }
};

typedef unsigned v4u32_t __attribute__((ext_vector_type(4)));
typedef unsigned v2u32_t __attribute__((ext_vector_type(2)));

// Chain operand orders (16x16x16 bf16 MFMA, or four 16x16x4 fp32 ones in k order 4 g + u: lane
// (i, g) of an A fragment holds row i, k = 4 g .. 4 g + 3; an accumulator's lane (j, g) holds rows
// 4 g .. 4 g + 3 of column j):
// - afrag: the four elements of A tile (rt, kt) for lane l; two k tiles of a row tile side by
//   side, so a lane reads a pair of bf16 tiles with one 16-byte load (D 16: one tile);
// - accfrag: the four floats of accumulator tile rt of value slice s for lane l.
template <int NT>
__device__ __forceinline__ size_t afrag(int rt, int kt, int l) {
  if constexpr (NT == 1) return (size_t)l * 4;
  else return ((size_t)(rt * (NT / 2) + kt / 2) * 64 + l) * 8 + (kt & 1) * 4;
}
template <int NT>
__device__ __forceinline__ size_t accfrag(int s, int rt, int l) { return ((size_t)(s * NT + rt) * 64 + l) * 4; }
// - accfrag2: the same for bf16 with two row tiles of a slice side by side (one 16-byte access for
//   a lane's pair; D 16: one tile): the chains' added terms and their records on the bf16 entry.
template <int NT>
__device__ __forceinline__ size_t accfrag2(int s, int rt, int l) {
  if constexpr (NT == 1) return (size_t)l * 4;
  else return ((size_t)(s * (NT / 2) + rt / 2) * 64 + l) * 8 + (rt & 1) * 4;
}

// Eight waves in the chunk kernel's arrangement: wave w owns row block rb (rb and 3 - rb on one
// SIMD) and every other column tile from ch = w / 4; triangular zeros are skipped.
constexpr int kPrepThreads = 512;

template <typename TIn, int D>
__global__ __launch_bounds__(kPrepThreads) void scan_bwd_prep_kernel(const TIn* __restrict__ q, const TIn* __restrict__ k,
                                                            const TIn* __restrict__ v, const TIn* __restrict__ beta,
                                                            const TIn* __restrict__ d_o,
                                                            const uint8_t* __restrict__ active,
                                                            float* __restrict__ ws, int N, int H, int NC) {
  constexpr int PD = D + 4;
  __shared__ __align__(16) float sK[kC * PD], sQ[kC * PD], sO[kC * PD], sV[kC * PD], sW[kC * PD], sU[kC * PD];
  __shared__ __align__(16) float sA[kC * kPC], sL[kC * kPC];
  __shared__ float sB[kC];
  const int c = blockIdx.x % NC, bh = blockIdx.x / NC;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kC;
  const size_t chunk = blockIdx.x;
  constexpr int NTH = kPrepThreads, NT = D / 16;
  constexpr bool BF = sizeof(TIn) == 2;  // bf16 inputs: the products on bf16 MFMA (fp32 accumulation)
  const int w = threadIdx.x >> 6, ch = w >> 2, rb = ch == 0 ? w : 7 - w, r0 = 16 * rb;
  {
    ChunkRows<TIn, D, NTH> rk, rq, ro, rv;
    ChunkBeta<TIn> rbeta;
    rk.fetch(k, b, h, t0, N, H);
    rq.fetch(q, b, h, t0, N, H);
    ro.fetch(d_o, b, h, t0, N, H, active);
    rv.fetch(v, b, h, t0, N, H);
    rbeta.fetch(beta, b, h, t0, N, H);
    rk.put(sK, PD, t0, N);
    rq.put(sQ, PD, t0, N);
    ro.put(sO, PD, t0, N);
    rv.put(sV, PD, t0, N);
    rbeta.put(sB, t0, N);
  }
  __syncthreads();
  // A = tril(diag(beta) K K^T, -1) (tiles above the diagonal: zeros)
  for (int ct = ch; ct < 4; ct += 2) {
    const f32x4 acc = ct <= rb ? mm16<false, true, BF>(sK + r0 * PD, PD, sK + 16 * ct * PD, PD, D, zero4()) : zero4();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      sA[i * kPC + j] = i > j ? sB[i] * acc[r] : 0.f;
    }
  }
  __syncthreads();
  // L = (I + A)^-1 by 16x16 blocks: the diagonal blocks (I + A_bb)^-1 by forward substitution (a
  // lane per column of a block), then L_ij = -L_ii sum_{m = j}^{i - 1} A_im L_mj level by level
  // (i - j = 1, 2, 3) on MFMA; the blocks above the diagonal are zero
#pragma unroll
  for (int e = threadIdx.x; e < kC * kC / 4; e += NTH) {  // four zeros a thread and step
    const int i = e / (kC / 4), j = 4 * (e % (kC / 4));
    if (i / 16 < j / 16) *reinterpret_cast<f32x4*>(sL + i * kPC + j) = zero4();
  }
  if (w == 0) {
    const int l = threadIdx.x & 63, blk = l >> 4, col = l & 15;
    const float* ab = sA + 16 * blk * kPC + 16 * blk;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sum = i == col ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) sum -= ab[i * kPC + m] * x[m];
      x[i] = sum;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sL[(16 * blk + i) * kPC + 16 * blk + col] = x[i];
  }
  __syncthreads();
  for (int lev = 1; lev < 4; ++lev) {
    const int i = w + lev, j = w;  // block (i, j) of this level, one per wave (waves 0 .. 2)
    if (i < 4) {
      f32x4 y = zero4();
      for (int m = j; m < i; ++m)
        y = mm16<false, false>(sA + 16 * i * kPC + 16 * m, kPC, sL + 16 * m * kPC + 16 * j, kPC, 16, y);
      // y is a register tile: stage it in the block's own (zero, not yet read) place of sL, then
      // L_ij = -L_ii y
      float* dst = sL + 16 * i * kPC + 16 * j;
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[tile_row(r) * kPC + tile_col()] = y[r];
      wave_sync_lds();  // every lane's y is in LDS before any lane reads it
      const f32x4 x = mm16<false, false>(sL + 16 * i * kPC + 16 * i, kPC, dst, kPC, 16, zero4());
      wave_sync_lds();  // every lane has read y before any lane overwrites it
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[tile_row(r) * kPC + tile_col()] = -x[r];
    }
    __syncthreads();
  }
  float* gL = Ws<D>::L(ws, chunk);
#pragma unroll
  for (int e = threadIdx.x; e < kC * kC / 4; e += NTH)
    *reinterpret_cast<f32x4*>(gL + 4 * e) = *reinterpret_cast<const f32x4*>(sL + (e / (kC / 4)) * kPC + 4 * (e % (kC / 4)));
  // W = L diag(beta) K and U = L diag(beta) V (L lower triangular: k blocks 0 .. rb)
  for (int ct = ch; ct < NT; ct += 2) {
    const f32x4 aw = mm16k<false, false, BF>(sL + r0 * kPC, kPC, sK + 16 * ct, PD, 0, rb + 1, zero4(), sB);
    const f32x4 au = mm16k<false, false, BF>(sL + r0 * kPC, kPC, sV + 16 * ct, PD, 0, rb + 1, zero4(), sB);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      sW[i * PD + j] = aw[r];
      sU[i * PD + j] = au[r];
    }
  }
  // P = tril(Q K^T), diagonal included, into sA (tiles above the diagonal: zeros)
  for (int ct = ch; ct < 4; ct += 2) {
    const f32x4 acc = ct <= rb ? mm16<false, true, BF>(sQ + r0 * PD, PD, sK + 16 * ct * PD, PD, D, zero4()) : zero4();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      sA[i * kPC + j] = j <= i ? acc[r] : 0.f;
    }
  }
  __syncthreads();  // sW, sA complete; sV's reads are done
  // Z = P^T dO into sV (P^T upper triangular: k blocks rb .. 3)
  for (int ct = ch; ct < NT; ct += 2) {
    const f32x4 acc = mm16k<true, false, BF>(sA + r0, kPC, sO + 16 * ct, PD, rb, 4, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) sV[(r0 + tile_row(r)) * PD + 16 * ct + tile_col()] = acc[r];
  }
  __syncthreads();
  // the chains' operands, tile (rt, ct) of each [D x D] product over the waves: Y = Q^T dO - W^T Z
  // and B = K^T U in accumulator order (value slice ct); N = -K^T W into NR and N^T = -W^T K into
  // NF, each accumulator tile (rt, ct) being A tile (ct, rt) of the other's transpose
  float* gY = Ws<D>::Y(ws, chunk);
  float* gB = Ws<D>::B(ws, chunk);
  float* gNF = Ws<D>::NF(ws, chunk);
  float* gNR = Ws<D>::NR(ws, chunk);
  const int l = threadIdx.x & 63;
  for (int tile = w; tile < NT * NT; tile += NTH / 64) {
    const int rt = tile / NT, ct = tile - rt * NT;
    const f32x4 qo = mm16<true, false, BF>(sQ + 16 * rt, PD, sO + 16 * ct, PD, kC, zero4());
    const f32x4 wz = mm16<true, false, BF>(sW + 16 * rt, PD, sV + 16 * ct, PD, kC, zero4());
    const f32x4 ku = mm16<true, false, BF>(sK + 16 * rt, PD, sU + 16 * ct, PD, kC, zero4());
    const f32x4 kw = mm16<true, false, BF>(sK + 16 * rt, PD, sW + 16 * ct, PD, kC, zero4());
    const f32x4 wk = mm16<true, false, BF>(sW + 16 * rt, PD, sK + 16 * ct, PD, kC, zero4());
    if constexpr (BF) {
      bf16x4 nr, nf, yb, bb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        nr[r] = (__bf16)(-kw[r]);
        nf[r] = (__bf16)(-wk[r]);
        yb[r] = (__bf16)(qo[r] - wz[r]);
        bb[r] = (__bf16)ku[r];
      }
      *reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(gY) + accfrag2<NT>(ct, rt, l)) = yb;
      *reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(gB) + accfrag2<NT>(ct, rt, l)) = bb;
      *reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(gNR) + afrag<NT>(ct, rt, l)) = nr;
      *reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(gNF) + afrag<NT>(ct, rt, l)) = nf;
    } else {
      *reinterpret_cast<f32x4*>(gY + accfrag<NT>(ct, rt, l)) = qo - wz;
      *reinterpret_cast<f32x4*>(gB + accfrag<NT>(ct, rt, l)) = ku;
      *reinterpret_cast<f32x4*>(gNR + afrag<NT>(ct, rt, l)) = -kw;
      *reinterpret_cast<f32x4*>(gNF + afrag<NT>(ct, rt, l)) = -wk;
    }
  }
}

// The chains, one wave each: logical blocks [0, S) walk the states forward, [S, 2 S) the state's
// gradient backward (S = B H D / 16 value slices). A step records the slice (the state at the
// chunk's start, or its gradient at the chunk's end) and applies X += A bf16(X) + C with the
// chunk's A (N or N^T) and C (B or Y): every B operand of the product is the lane's own
// accumulator, rounded, so the chain needs no data from other lanes. The operands of kRing chunks
// are in flight in registers: a slot is refilled with the chunk kRing later right after its use
// (unconditionally, the last chunk again past the end, so that no load sits behind a branch).
template <int D, bool BF>
struct ChainShape {
  static constexpr int NT = D / 16;
  // chunks of operands in flight: as many as the registers hold without spills
  static constexpr int kRing = BF ? (D >= 128 ? 2 : (D >= 64 ? 6 : 12)) : (D >= 64 ? 2 : (D >= 32 ? 8 : 12));
};

template <int NT, bool BF>
struct ChainOps {
  static constexpr int kA = BF ? 2 : 4;  // dwords per A tile and lane
  uint32_t a[kA * NT * NT];   // A tile (rt, kt): a[kA (rt NT + kt)] .. + kA - 1, four bf16 or fp32
  uint32_t add[kA * NT];      // the added term's accumulator tiles, four bf16 or fp32 a tile
  __device__ __forceinline__ f32x4 add_tile(int rt) const {
    if constexpr (BF) {
      const uint2 v = {add[2 * rt], add[2 * rt + 1]};
      const bf16x4 x = __builtin_bit_cast(bf16x4, v);
      return f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
    } else {
      const uint4 v = {add[4 * rt], add[4 * rt + 1], add[4 * rt + 2], add[4 * rt + 3]};
      return __builtin_bit_cast(f32x4, v);
    }
  }
};

// A chain's loads and stores go through one buffer resource over its (b, h) chunks: the chunk's
// offset is a scalar, a lane's offset within the chunk a constant.
template <int D, bool BF>
__device__ __forceinline__ void load_chain_ops(ChainOps<D / 16, BF>& o, __amdgpu_buffer_rsrc_t rs, unsigned a_off,
                                               unsigned add_off, unsigned chunk_off, int s, int l) {
  constexpr int NT = D / 16;
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (!BF) {
#pragma unroll
    for (int rt = 0; rt < NT; ++rt)
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, a_off + 4 * (unsigned)afrag<NT>(rt, kt, l), chunk_off, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) o.a[4 * (rt * NT + kt) + e] = v[e];
      }
  } else if constexpr (NT == 1) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, a_off + 2 * (unsigned)afrag<NT>(0, 0, l), chunk_off, 0);
    o.a[0] = v[0];
    o.a[1] = v[1];
  } else {
#pragma unroll
    for (int rt = 0; rt < NT; ++rt)
#pragma unroll
      for (int kt = 0; kt < NT; kt += 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, a_off + 2 * (unsigned)afrag<NT>(rt, kt, l), chunk_off, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) o.a[2 * (rt * NT + kt) + e] = v[e];
      }
  }
  if constexpr (BF && NT >= 2) {
#pragma unroll
    for (int rt = 0; rt < NT; rt += 2) {  // a pair of row tiles a load
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, add_off + 2 * (unsigned)accfrag2<NT>(s, rt, l), chunk_off, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) o.add[2 * rt + e] = v[e];
    }
  }
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    if constexpr (BF && NT >= 2) {
    } else if constexpr (BF) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, add_off + 2 * (unsigned)accfrag2<NT>(s, rt, l), chunk_off, 0);
      o.add[2 * rt] = v[0];
      o.add[2 * rt + 1] = v[1];
    } else {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, add_off + 4 * (unsigned)accfrag<NT>(s, rt, l), chunk_off, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) o.add[4 * rt + e] = v[e];
    }
  }
#endif
}

template <typename TIn, int D>
__global__ __launch_bounds__(64) void scan_bwd_chains_kernel(const float* __restrict__ state_in,
                                                             const float* __restrict__ d_state,
                                                             float* __restrict__ d_state_in, float* __restrict__ ws,
                                                             int NC, int S, int lg0) {
  constexpr bool BF = sizeof(TIn) == 2;  // bf16 A operands and 16x16x16 bf16 MFMA; else fp32 ones
  constexpr int NT = ChainShape<D, BF>::NT, R = ChainShape<D, BF>::kRing;
  // At D 128 the chunk kernel reads the records as MFMA fragments from global memory, in both
  // orientations: each step also records its slice transposed (through a 16x16 LDS tile), in
  // the second half of the record's block.
  constexpr bool kRowRec = BF && D >= 128;
  __shared__ __align__(16) __bf16 sTr[kRowRec ? NT * 16 * 16 : 1];
  constexpr unsigned kPerB = (unsigned)(Ws<D>::kPer * sizeof(float));  // bytes per chunk
  constexpr unsigned kLB = (unsigned)(Ws<D>::kL * sizeof(float)), kSB = (unsigned)(Ws<D>::kS * sizeof(float));
  // (lg0 = S: the reverse chains only, the states having been recorded by the forward)
  const int lg = xcd_logical_block(blockIdx.x, gridDim.x) + lg0;
  const bool rev = lg >= S;
  const int sl = rev ? lg - S : lg;
  const int s = sl % NT, bh = sl / NT;
  const int l = threadIdx.x & 63, j = l & 15, g = l >> 4;
  // offsets within a chunk: the A fragments (NF or NR), the added term (B or Y), the record (Hs or dHs)
  const unsigned a_off = rev ? kLB + kSB : kLB;
  const unsigned add_off = rev ? kLB + 3 * kSB : kLB + 2 * kSB;
  const unsigned rec_off = rev ? kLB + 5 * kSB : kLB + 4 * kSB;
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(ws + (size_t)bh * NC * Ws<D>::kPer, (unsigned)NC * kPerB);
  const float* init = rev ? d_state : state_in;  // (no gradient of the final state: zeros)
  f32x4 acc[NT];
#pragma unroll
  for (int rt = 0; rt < NT; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      acc[rt][r] = init != nullptr ? init[(size_t)bh * D * D + (16 * rt + 4 * g + r) * D + 16 * s + j] : 0.f;
  auto chunk_off = [&](int i) { return (unsigned)(rev ? NC - 1 - i : i) * kPerB; };  // the i-th chunk visited
  auto load = [&](ChainOps<NT, BF>& o, int i) {
    load_chain_ops<D, BF>(o, rs, a_off, add_off, chunk_off(min(i, NC - 1)), s, l);
  };
  ChainOps<NT, BF> ops[R];
#pragma unroll
  for (int p = 0; p < R; ++p) load(ops[p], p);
  auto step = [&](int i, ChainOps<NT, BF>& cur) {
    // the records' stores carry the chunk's offset in the vector offset (scalar offset 0): the
    // compiler puts no wait state after a wide buffer store with a scalar offset before its data
    // registers are written again, and on gfx950 such a store can then write the new value
    const unsigned co = chunk_off(i);
    s16x4_t xb[NT];
    f32x4 xf[NT];
    bf16x4 tprev;
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      xf[kt] = acc[kt];
      bf16x4 t;
#pragma unroll
      for (int r = 0; r < 4; ++r) t[r] = (__bf16)acc[kt][r];
      xb[kt] = __builtin_bit_cast(s16x4_t, t);
#if defined(__HIP_DEVICE_COMPILE__)
      if constexpr (BF && D >= 32) {  // the record as the bf16 chunk kernel multiplies it, a pair a store
        if (kt & 1) {
          const v4u32_t pr = {__builtin_bit_cast(v2u32_t, tprev)[0], __builtin_bit_cast(v2u32_t, tprev)[1],
                               __builtin_bit_cast(v2u32_t, t)[0], __builtin_bit_cast(v2u32_t, t)[1]};
          __builtin_amdgcn_raw_buffer_store_b128(pr, rs, co + rec_off + 2 * (unsigned)accfrag2<NT>(s, kt - 1, l), 0, 0);
        }
        tprev = t;
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, acc[kt]), rs,
                                               co + rec_off + 4 * (unsigned)accfrag<NT>(s, kt, l), 0, 0);
      }
#endif
      if constexpr (kRowRec) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sTr[kt * 256 + (4 * g + r) * 16 + j] = t[r];
      }
    }
    if constexpr (kRowRec) {
      // tile (kt, s) of the slice transposed: lane (j, g) takes row j, columns 4 g .. 4 g + 3
      wave_sync_lds();
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        const bf16x4 x = *reinterpret_cast<const bf16x4*>(sTr + kt * 256 + j * 16 + 4 * g);
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, x), rs,
                                              co + rec_off + kSB / 2 + 2 * (unsigned)accfrag<NT>(s, kt, l), 0, 0);
#endif
      }
      wave_sync_lds();
    }
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
      acc[rt] += cur.add_tile(rt);
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        const uint32_t* a = cur.a + ChainOps<NT, BF>::kA * (rt * NT + kt);
        if constexpr (BF) {
          const uint2 a2 = {a[0], a[1]};
          acc[rt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a2), xb[kt], acc[rt], 0, 0, 0);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u)
            acc[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(__builtin_bit_cast(float, a[u]), xf[kt][u], acc[rt], 0, 0, 0);
        }
      }
    }
    load(cur, i + R);
  };
  int i = 0;
  for (; i + R <= NC; i += R) {
#pragma unroll
    for (int p = 0; p < R; ++p) step(i + p, ops[p]);
  }
#pragma unroll
  for (int p = 0; p < R; ++p)
    if (i + p < NC) step(i + p, ops[p]);
  if (rev) {
#pragma unroll
    for (int rt = 0; rt < NT; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) d_state_in[(size_t)bh * D * D + (16 * rt + 4 * g + r) * D + 16 * s + j] = acc[rt][r];
  }
}

// Eight waves, two per SIMD, hiding each other's LDS and MFMA latency: wave w owns row block rb
// of every [64 x .] result and every other column tile from ch = w / 4. Waves w and w + 4 (one
// SIMD) own row blocks rb and 3 - rb: the triangular products (whose tiles and k ranges grow with
// the row block) then load every SIMD about evenly. Tiles that a triangular factor makes zero are
// not computed, and each product runs over the k blocks its triangular operand leaves nonzero.
constexpr int kChunkThreads = 512;

template <typename TIn, int D>
__global__ __launch_bounds__(kChunkThreads) void scan_bwd_chunk_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TIn* __restrict__ beta,
    const TIn* __restrict__ d_o, const uint8_t* __restrict__ active, const float* __restrict__ ws,
    TIn* __restrict__ dq, TIn* __restrict__ dk, TIn* __restrict__ dv, TIn* __restrict__ dbeta, int N, int H, int NC) {
  constexpr int P = kPC;  // every buffer is [64][68]
  constexpr int NT = D / 16, NTW = (NT + 1) / 2;  // column tiles of a [64 x D] result; a wave's share
  constexpr int NTH = kChunkThreads;
  constexpr bool BF = sizeof(TIn) == 2;  // bf16 inputs: the products on bf16 MFMA (fp32 accumulation)
  __shared__ __align__(16) float buf[9][kC * P];
  __shared__ float sB[kC], sPart[4 * kC], sRow[2 * kC];
  const int c = blockIdx.x % NC, bh = blockIdx.x / NC;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kC;
  const size_t chunk = blockIdx.x;
  const int w = threadIdx.x >> 6, ch = w >> 2, rb = ch == 0 ? w : 7 - w;
  float *Bq = buf[0], *Bk = buf[1], *Bo = buf[2], *Br = buf[3], *Bh = buf[4], *Bg = buf[5], *Bl = buf[6];
  float *Bd = buf[7], *Bp = buf[8];
  {
    ChunkRows<TIn, D, NTH> rq, rk, ro, rv;
    AccRows<D, NTH> mh, mg;
    MatRows<kC, kC, NTH> ml;
    ChunkBeta<TIn> rb_;
    rq.fetch(q, b, h, t0, N, H);
    rk.fetch(k, b, h, t0, N, H);
    ro.fetch(d_o, b, h, t0, N, H, active);
    rv.fetch(v, b, h, t0, N, H);
    mh.fetch(Ws<D>::Hs(const_cast<float*>(ws), chunk));
    mg.fetch(Ws<D>::dHs(const_cast<float*>(ws), chunk));
    ml.fetch(Ws<D>::L(const_cast<float*>(ws), chunk));
    rb_.fetch(beta, b, h, t0, N, H);
    rq.put(Bq, P, t0, N);
    rk.put(Bk, P, t0, N);
    ro.put(Bo, P, t0, N);
    rv.put(Br, P, t0, N);
    mh.put(Bh, P);
    mg.put(Bg, P);
    ml.put(Bl, P);
    rb_.put(sB, t0, N);
  }
  __syncthreads();
  const int r0 = 16 * rb;  // this wave's 16 rows of every [64 x .] result
  // R = V - K H, in place (each tile reads only its own V entries)
  for (int ct = ch; ct < NT; ct += 2) {
    const f32x4 acc = mm16<false, false, BF>(Bk + r0 * P, P, Bh + 16 * ct, P, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) Br[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] -= acc[r];
  }
  // P = tril(Q K^T), diagonal included (tiles above the diagonal: zeros)
  for (int ct = ch; ct < 4; ct += 2) {
    const f32x4 acc = ct <= rb ? mm16<false, true, BF>(Bq + r0 * P, P, Bk + 16 * ct * P, P, D, zero4()) : zero4();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      Bp[i * P + j] = j <= i ? acc[r] : 0.f;
    }
  }
  __syncthreads();
  // Delta = L diag(beta) R (L lower triangular: k blocks 0 .. rb)
  for (int ct = ch; ct < NT; ct += 2) {
    const f32x4 acc = mm16k<false, false, BF>(Bl + r0 * P, P, Br + 16 * ct, P, 0, rb + 1, zero4(), sB);
#pragma unroll
    for (int r = 0; r < 4; ++r) Bd[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] = acc[r];
  }
  __syncthreads();
  // dK accumulates in registers: the wave's rows r0, its column tiles ch, ch + 2
  f32x4 dka[NTW];
  // dDelta = K G + P^T dO (registers), dK = Delta G^T
  f32x4 ddl[NTW];
#pragma unroll
  for (int u = 0; u < NTW; ++u) {
    const int ct = ch + 2 * u;
    if (ct < NT) {
      ddl[u] = mm16<false, false, BF>(Bk + r0 * P, P, Bg + 16 * ct, P, D, zero4());
      ddl[u] = mm16k<true, false, BF>(Bp + r0, P, Bo + 16 * ct, P, rb, 4, ddl[u]);  // P^T: k blocks rb .. 3
      dka[u] = mm16<false, true, BF>(Bd + r0 * P, P, Bg + 16 * ct * P, P, D, zero4());
    }
  }
  __syncthreads();  // the reads of G are done: dDelta goes into its buffer
  float* Bdd = Bg;
#pragma unroll
  for (int u = 0; u < NTW; ++u) {
    const int ct = ch + 2 * u;
    if (ct < NT)
#pragma unroll
      for (int r = 0; r < 4; ++r) Bdd[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] = ddl[u][r];
  }
  __syncthreads();
  // dR = diag(beta) L^T dDelta into P's buffer (free now); dV = dR
  float* Bdr = Bp;
  for (int ct = ch; ct < NT; ct += 2) {
    const f32x4 acc = mm16k<true, false, BF>(Bl + r0, P, Bdd + 16 * ct, P, rb, 4, zero4());  // L^T: k blocks rb .. 3
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      const float x = sB[i] * acc[r];
      Bdr[i * P + j] = x;
      if (t0 + i < N) dv[(((size_t)b * N + t0 + i) * H + h) * D + j] = from_f32<TIn>(x);
    }
  }
  __syncthreads();
  // dK -= dR H^T
#pragma unroll
  for (int u = 0; u < NTW; ++u) {
    const int ct = ch + 2 * u;
    if (ct < NT) {
      const f32x4 acc = mm16<false, true, BF>(Bdr + r0 * P, P, Bh + 16 * ct * P, P, D, zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) dka[u][r] -= acc[r];
    }
  }
  __syncthreads();  // the reads of dR are done
  // S2 = tril(dO Delta^T), diagonal included, into dR's buffer (tiles above the diagonal: zeros)
  float* Bs = Bp;
  for (int ct = ch; ct < 4; ct += 2) {
    const f32x4 acc = ct <= rb ? mm16<false, true, BF>(Bo + r0 * P, P, Bd + 16 * ct * P, P, D, zero4()) : zero4();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      Bs[i * P + j] = j <= i ? acc[r] : 0.f;
    }
  }
  __syncthreads();
  // dQ = dO H^T + S2 K; dK += S2^T Q
#pragma unroll
  for (int u = 0; u < NTW; ++u) {
    const int ct = ch + 2 * u;
    if (ct < NT) {
      f32x4 acc = mm16<false, true, BF>(Bo + r0 * P, P, Bh + 16 * ct * P, P, D, zero4());
      acc = mm16k<false, false, BF>(Bs + r0 * P, P, Bk + 16 * ct, P, 0, rb + 1, acc);  // S2: k blocks 0 .. rb
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
        if (t0 + i < N) dq[(((size_t)b * N + t0 + i) * H + h) * D + j] = from_f32<TIn>(acc[r]);
      }
      dka[u] = mm16k<true, false, BF>(Bs + r0, P, Bq + 16 * ct, P, rb, 4, dka[u]);  // S2^T: k blocks rb .. 3
    }
  }
  __syncthreads();  // H, dO, Q, S2, Delta are done with
  // dT = dDelta R^T. dbeta_j gets sum_i dT_ij L_ij (L is zero above its diagonal): each wave sums
  // its 16 rows of its columns into sPart; dL = tril(dT) diag(beta) goes into H's buffer
  float* Bt = Bh;
  for (int ct = ch; ct < 4; ct += 2) {  // (tiles above the diagonal: dL is zero there, and so is L)
    const f32x4 acc = ct <= rb ? mm16<false, true, BF>(Bdd + r0 * P, P, Br + 16 * ct * P, P, D, zero4()) : zero4();
    const int j = 16 * ct + tile_col();
    float part = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r);
      part += acc[r] * Bl[i * P + j];
      Bt[i * P + j] = j <= i ? acc[r] * sB[j] : 0.f;
    }
    part = sum_over_rows(part);
    if ((threadIdx.x & 63) < 16) sPart[rb * kC + j] = part;
  }
  __syncthreads();
  // X1 = L^T dL into Q's buffer (L^T upper, dL lower triangular: k blocks max(rb, ct) .. 3)
  float* Bx = Bq;
  for (int ct = ch; ct < 4; ct += 2) {
    const f32x4 acc = mm16k<true, false, BF>(Bl + r0, P, Bt + 16 * ct, P, max(rb, ct), 4, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) Bx[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] = acc[r];
  }
  __syncthreads();
  // dA = -tril(X1 L^T, -1); dbeta_i gets sum_{m < i} dA_im (k_i . k_m), each wave's columns into
  // sRow; M = diag(beta) dA goes into dO's buffer
  float* Ba = Bo;
  float rows[4] = {0.f, 0.f, 0.f, 0.f};
  for (int ct = ch; ct < 4; ct += 2) {
    if (ct > rb) {  // strictly above the diagonal: dA and M are zero
#pragma unroll
      for (int r = 0; r < 4; ++r) Ba[(r0 + tile_row(r)) * P + 16 * ct + tile_col()] = 0.f;
      continue;
    }
    // L^T column block ct: k blocks 0 .. ct
    const f32x4 acc = mm16k<false, true, BF>(Bx + r0 * P, P, Bl + 16 * ct * P, P, 0, ct + 1, zero4());
    const f32x4 gk = mm16<false, true, BF>(Bk + r0 * P, P, Bk + 16 * ct * P, P, D, zero4());
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      const float da = j < i ? -acc[r] : 0.f;
      rows[r] += da * gk[r];
      Ba[i * P + j] = da * sB[i];
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float x = group_sum<16>(rows[r]);
    if (tile_col() == 0) sRow[ch * kC + r0 + tile_row(r)] = x;
  }
  __syncthreads();
  // dK += M K + M^T K, then store
#pragma unroll
  for (int u = 0; u < NTW; ++u) {
    const int ct = ch + 2 * u;
    if (ct < NT) {
      dka[u] = mm16k<false, false, BF>(Ba + r0 * P, P, Bk + 16 * ct, P, 0, rb + 1, dka[u]);  // M: k blocks 0 .. rb
      dka[u] = mm16k<true, false, BF>(Ba + r0, P, Bk + 16 * ct, P, rb, 4, dka[u]);         // M^T: k blocks rb .. 3
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
        if (t0 + i < N) dk[(((size_t)b * N + t0 + i) * H + h) * D + j] = from_f32<TIn>(dka[u][r]);
      }
    }
  }
  const int i = threadIdx.x;
  if (i < kC && t0 + i < N) {
    const float x = ((sPart[i] + sPart[kC + i]) + (sPart[2 * kC + i] + sPart[3 * kC + i])) + (sRow[i] + sRow[kC + i]);
    dbeta[((size_t)b * N + t0 + i) * H + h] = from_f32<TIn>(x);
  }
}

// ---- the chunk kernel on bf16 LDS tiles (bf16 entry, head widths 32 and 64) ------------------
// Operands live in LDS as bf16 row-major tiles and feed 16x16x32 MFMAs in one of two forms, with
// the same k order (k0 + 8 g + e for lane group g, element e) so that any two combine:
// - frow(X, ld, r0, k0): row r0 + lq of X, k along its columns (one 16-byte read);
// - fcol(X, ld, c0, k0): column c0 + lq of X, k along its rows (two transposed 8-byte reads).
// A product's A operand is frow(X) for X or fcol(X) for X^T; its B operand fcol(Y) for Y or
// frow(Y) for Y^T. Results (lane (j, g) holds rows 4 g .. 4 g + 3 of column j) go back to LDS as
// bf16, the rounding the fp32-staged kernel applied when it multiplied them.
__device__ __forceinline__ bf16x8 frow(const __bf16* X, int ld, int r0, int k0) {
  const int l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  return *reinterpret_cast<const bf16x8*>(X + (r0 + lq) * ld + k0 + 8 * g);
}
__device__ __forceinline__ bf16x8 fcol(const __bf16* X, int ld, int c0, int k0) {
  const int l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  const __bf16* p = X + (k0 + 8 * g + (lq >> 2)) * ld + c0 + 4 * (lq & 3);
  const bf16x4 lo = read_tr16<bf16x4>(p), hi = read_tr16<bf16x4>(p + 4 * ld);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
// the A operand in the k order of a pair of 16-row accumulator tiles (k0 + 4 g .. + 3, then
// k0 + 16 + 4 g .. + 3): row r0 + lq of X by two 8-byte reads
__device__ __forceinline__ bf16x8 frow2(const __bf16* X, int ld, int r0, int k0) {
  const int l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  const __bf16* p = X + (r0 + lq) * ld + k0 + 4 * g;
  const bf16x4 lo = *reinterpret_cast<const bf16x4*>(p), hi = *reinterpret_cast<const bf16x4*>(p + 16);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <int N> using vec_u32 = unsigned __attribute__((ext_vector_type(N)));
// An accumulator tile in bf16 as 32-bit pairs of columns: lane (j, g) holds rows 4 g .. 4 g + 3 of
// column j; after one exchange with the lane of column j ^ 1 (a DPP swap) the even lane holds rows
// 4 g, 4 g + 1 and the odd lane rows 4 g + 2, 4 g + 3 of columns j & ~1 and (j & ~1) + 1, so a
// tile goes out in two 4-byte writes a lane instead of four 2-byte ones (in LDS: no two lanes in
// one 32-bit word, and the 64 lanes of a write on 64 distinct banks at the tiles' pitches).
// Returns the two words and sets `row` to the first one's row within the tile. pair_words takes the
// lane's four bf16 values as two words (rows 4 g, 4 g + 1 and rows 4 g + 2, 4 g + 3).
__device__ __forceinline__ uint2 pair_words(uint32_t lo, uint32_t hi, int& row) {
  const int l = threadIdx.x & 63, odd = l & 1;
  const uint32_t own = odd ? hi : lo, send = odd ? lo : hi;
  // quad_perm [1, 0, 3, 2]: the word of the neighbouring column
  const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xB1, 0xF, 0xF, false);
  const uint32_t first = odd ? recv : own, second = odd ? own : recv;
  row = 4 * (l >> 4) + 2 * odd;
  return uint2{__builtin_amdgcn_perm(second, first, 0x05040100u), __builtin_amdgcn_perm(second, first, 0x07060302u)};
}
__device__ __forceinline__ uint2 pair_cols(f32x4 acc, int& row) {
  const bf16x2_t lo2 = {(__bf16)acc[0], (__bf16)acc[1]}, hi2 = {(__bf16)acc[2], (__bf16)acc[3]};
  return pair_words(__builtin_bit_cast(uint32_t, lo2), __builtin_bit_cast(uint32_t, hi2), row);
}
// an accumulator tile into a bf16 tile at (r0, c0) (ld and c0 even)
__device__ __forceinline__ void put_tile(__bf16* X, int ld, int r0, int c0, f32x4 acc) {
  int row;
  const uint2 w = pair_cols(acc, row);
  __bf16* p = X + (r0 + row) * ld + c0 + (tile_col() & ~1);
  *reinterpret_cast<uint32_t*>(p) = w.x;
  *reinterpret_cast<uint32_t*>(p + ld) = w.y;
}
// an accumulator tile into rows t0 + r0 .. of a [B, N, H, D] tensor (rows past N skipped)
template <typename TIn, int D>
__device__ __forceinline__ void store_rows(TIn* dst, int b, int h, int t0, int N, int H, int r0, int c0, f32x4 acc) {
  if constexpr (sizeof(TIn) == 2) {
    int row;
    const uint2 w = pair_cols(acc, row);
    const int t = t0 + r0 + row;
    TIn* p = dst + (((size_t)b * N + t) * H + h) * D + c0 + (tile_col() & ~1);
    if (t < N) *reinterpret_cast<uint32_t*>(p) = w.x;
    if (t + 1 < N) *reinterpret_cast<uint32_t*>(p + (size_t)H * D) = w.y;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + r0 + tile_row(r);
      if (t < N) dst[(((size_t)b * N + t) * H + h) * D + c0 + tile_col()] = from_f32<TIn>(acc[r]);
    }
  }
}

// chunk rows t0 .. t0 + 63 of a [B, N, H, D] bf16 tensor into LDS [64][ld] bf16; rows past N,
// and with `active` inactive tokens' rows, are zero. 16 bytes a thread and step.
template <int D, int NTH>
struct ChunkRows16 {
  static constexpr int kN = kC * D / 8, kIt = (kN + NTH - 1) / NTH;
  bf16x8 raw[kIt];
  bool ok[kIt];
  __device__ __forceinline__ void fetch(const __bf16* src, int b, int h, int t0, int N, int H,
                                        const uint8_t* active = nullptr) {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = min((int)threadIdx.x + NTH * it, kN - 1), row = e / (D / 8), c = 8 * (e % (D / 8));
      const int tc = min(t0 + row, N - 1);
      raw[it] = *reinterpret_cast<const bf16x8*>(src + (((size_t)b * N + tc) * H + h) * D + c);
      ok[it] = t0 + row < N && (active == nullptr || active[(size_t)b * N + tc] != 0);
    }
  }
  __device__ __forceinline__ void put(__bf16* dst, int ld) const {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = threadIdx.x + NTH * it, row = e / (D / 8), c = 8 * (e % (D / 8));
      const uint4 x = __builtin_bit_cast(uint4, raw[it]);  // zeros selected as four 32-bit words
      const bool o = ok[it];
      const uint4 y = {o ? x.x : 0u, o ? x.y : 0u, o ? x.z : 0u, o ? x.w : 0u};
      if (kN % NTH == 0 || e < kN) *reinterpret_cast<uint4*>(dst + row * ld + c) = y;
    }
  }
};

// a [D][D] bf16 record in accumulator order (accfrag2: pairs of row tiles) into LDS [D][ld] bf16,
// row-major (column pairs exchanged as put_tile does: a lane's units are the record's lane's)
template <int D, int NTH>
struct AccRows16 {
  static constexpr int NT = D / 16, NP = NT >= 2 ? NT / 2 : 1, EU = NT >= 2 ? 8 : 4;  // elements a unit
  static constexpr int kN = D * D / EU, kIt = (kN + NTH - 1) / NTH;
  typedef __bf16 U __attribute__((ext_vector_type(EU)));
  U raw[kIt];
  __device__ __forceinline__ void fetch(const __bf16* src) {
#pragma unroll
    for (int it = 0; it < kIt; ++it) raw[it] = *reinterpret_cast<const U*>(src + EU * min((int)threadIdx.x + NTH * it, kN - 1));
  }
  __device__ __forceinline__ void put(__bf16* dst, int ld) const {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = threadIdx.x + NTH * it;  // = (slice NP + pair) 64 + lane
      if (kN % NTH == 0 || e < kN) {
        const int lane = e & 63, st = e >> 6, sl = st / NP, m = st - sl * NP;
        const auto words = __builtin_bit_cast(vec_u32<EU / 2>, raw[it]);
#pragma unroll
        for (int u = 0; u < EU / 4; ++u) {
          int row;
          const uint2 w = pair_words(words[2 * u], words[2 * u + 1], row);
          __bf16* p = dst + (16 * (2 * m + u) + row) * ld + 16 * sl + ((lane & 15) & ~1);
          *reinterpret_cast<uint32_t*>(p) = w.x;
          *reinterpret_cast<uint32_t*>(p + ld) = w.y;
        }
      }
    }
  }
};

// Eight waves: wave w owns row block rb of every [64 x .] result (rb and 3 - rb on one SIMD) and
// every other column tile from ch = w / 4. Products run over their full k range, unrolled: the
// triangular factors hold exact zeros where they vanish, and straight-line code lets the compiler
// issue a stage's LDS reads ahead of its MFMAs.
// Threads of the bf16 chunk kernel: eight waves (two a SIMD, two tiles of every [64 x 64] product
// each). Sixteen at width 64 (four a SIMD, one tile each) measured slower: the 128-register bound
// of four waves a SIMD spilled (chunk kernel 115 -> 139 us at B8 T4096 H8 d64).
template <int D> struct ChunkShape {
  static constexpr int NTH = 512;
  static constexpr int NW = NTH / 64;
  static constexpr int NCH = NW / 4;  // column groups: a wave's column tiles are ch, ch + NCH, ...
};

template <int D>
__global__ __launch_bounds__(ChunkShape<D>::NTH) void scan_bwd_chunk_bf16_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const __bf16* __restrict__ beta, const __bf16* __restrict__ d_o, const uint8_t* __restrict__ active,
    const float* __restrict__ ws, const __bf16* __restrict__ hrec, __bf16* __restrict__ dq, __bf16* __restrict__ dk,
    __bf16* __restrict__ dv, __bf16* __restrict__ dbeta, int N, int H, int NC, int total) {
  using T = __bf16;
  constexpr int NT = D / 16;  // column tiles of a [64 x D] result
  constexpr int NTH = ChunkShape<D>::NTH, NCH = ChunkShape<D>::NCH;
  // pitches: [64][D] and [D][D], [64][64]; up to D 64 rows 40 banks apart (the row fragments'
  // 16-byte reads then meet no bank twice: each two groups of eight lanes in one cycle cover the 64
  // banks), at D 128 (LDS-bound) 68
  constexpr int LD = D <= 64 ? D + 16 : D + 8, L6 = D <= 64 ? kC + 16 : kC + 8;
  // Up to D 64 the states H and G are LDS tiles. At D 128 they would not fit: their fragments come
  // from the chains' records in global memory (column order for H and G as B operands, the
  // transposed records for H^T and G^T), whose k order within 32 is 4 g .. 4 g + 3 of each 16-row
  // tile, so the A operands they meet are read in that order too (frow2); and -dR goes over R.
  constexpr bool kHGinLDS = D <= 64;
  __shared__ __align__(16) T sQ[kC * LD], sK[kC * LD], sO[kC * LD], sR[kC * LD], sD[kC * LD], sDD[kC * LD];
  __shared__ __align__(16) T sDRx[kHGinLDS ? kC * LD : 1];
  __shared__ __align__(16) T sH[kHGinLDS ? D * LD : 1], sG[kHGinLDS ? D * LD : 1];
  T* sDR = kHGinLDS ? sDRx : sR;
  constexpr int kU = kHGinLDS ? NT / NCH : 1;  // column tiles unrolled (D 128: one, for the registers)
  __shared__ __align__(16) T sT[kC * L6], sL[kC * L6], sP[kC * L6], sM[kC * L6];
  __shared__ float sB[kC], sPart[4 * kC], sRow[NCH * kC];
  T* sX1 = sT;   // X1 = L^T dL once T is done with
  T* sS2 = sP;   // S2 = tril(dO Delta^T) once P is done with
  T* sDL = sM;   // dL, then M = diag(beta) dA
  // wave w: column group ch = w / 4 and row block rb; the waves of one SIMD (w, w + 4, ...) take
  // row blocks rb and 3 - rb in turn, which evens out the triangular products' work
  const int w = threadIdx.x >> 6, ch = w >> 2, rb = (ch & 1) == 0 ? (w & 3) : 3 - (w & 3), r0 = 16 * rb;
  // A workgroup walks chunks blockIdx.x, + gridDim.x, ...: the next chunk's operands are loaded
  // into registers while the current one is computed.
  ChunkRows16<D, NTH> rq, rk, ro, rv;
  AccRows16<kHGinLDS ? D : 16, NTH> mh, mg;
  ChunkBeta<T> rbeta;
  bf16x8 lraw;
  auto fetch = [&](int cid) {
    const int c = cid % NC, bh = cid / NC;
    const int b = bh / H, h = bh - b * H;
    const int t0 = c * kC;
    const T* gL = reinterpret_cast<const T*>(Ws<D>::L(const_cast<float*>(ws), cid));
    lraw = *reinterpret_cast<const bf16x8*>(gL + 8 * min((int)threadIdx.x, kC * kC / 8 - 1));  // [64][64]: 8 a thread
    rq.fetch(q, b, h, t0, N, H);
    rk.fetch(k, b, h, t0, N, H);
    ro.fetch(d_o, b, h, t0, N, H, active);
    rv.fetch(v, b, h, t0, N, H);
    if constexpr (kHGinLDS) {
      // the chunk's starting state: the forward's record when it kept one, else the chain's
      mh.fetch(hrec != nullptr ? hrec + (size_t)cid * (D * D)
                               : reinterpret_cast<const T*>(Ws<D>::Hs(const_cast<float*>(ws), cid)));
      mg.fetch(reinterpret_cast<const T*>(Ws<D>::dHs(const_cast<float*>(ws), cid)));
    }
    rbeta.fetch(beta, b, h, t0, N, H);
  };
  // (at D 128 the registers go to the states' fragments: each chunk loads its own operands)
  if constexpr (kHGinLDS) fetch(blockIdx.x);
  for (int cid = blockIdx.x; cid < total; cid += gridDim.x) {
  if constexpr (!kHGinLDS) fetch(cid);
  const int c = cid % NC, bh = cid / NC;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kC;
  // the states' fragments: B operands of X H (hcol) and X H^T (hrow), and the A operands they meet
  const T* gH = reinterpret_cast<const T*>(Ws<D>::Hs(const_cast<float*>(ws), cid));
  const T* gG = reinterpret_cast<const T*>(Ws<D>::dHs(const_cast<float*>(ws), cid));
  const int lane = threadIdx.x & 63;
  auto bcol = [&](const T* rec, const T* tile, int ct, int kk) -> bf16x8 {
    if constexpr (kHGinLDS) {
      return fcol(tile, LD, 16 * ct, kk);
    } else {
      return *reinterpret_cast<const bf16x8*>(rec + accfrag2<NT>(ct, kk / 16, lane));  // tiles kk/16, +1
    }
  };
  auto brow = [&](const T* rec, const T* tile, int ct, int kk) -> bf16x8 {
    if constexpr (kHGinLDS) {
      return frow(tile, LD, 16 * ct, kk);
    } else {
      const T* rr = rec + Ws<D>::kS;  // the transposed record
      const bf16x4 lo = *reinterpret_cast<const bf16x4*>(rr + accfrag<NT>(kk / 16, ct, lane));
      const bf16x4 hi = *reinterpret_cast<const bf16x4*>(rr + accfrag<NT>(kk / 16 + 1, ct, lane));
      return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };
  auto arow = [&](const T* X, int kk) -> bf16x8 { return kHGinLDS ? frow(X, LD, r0, kk) : frow2(X, LD, r0, kk); };
  {
    rq.put(sQ, LD);
    rk.put(sK, LD);
    ro.put(sO, LD);
    rv.put(sR, LD);
    if constexpr (kHGinLDS) {
      mh.put(sH, LD);
      mg.put(sG, LD);
    }
    if (threadIdx.x < kC * kC / 8) *reinterpret_cast<bf16x8*>(sL + (threadIdx.x >> 3) * L6 + 8 * (threadIdx.x & 7)) = lraw;
    rbeta.put(sB, t0, N);
  }
  static_assert(NTH * 8 >= kC * kC, "one 16-byte piece of L a thread at most");
  __syncthreads();
  if constexpr (kHGinLDS) fetch(min(cid + (int)gridDim.x, total - 1));  // (the last chunk again past the end)
  // T = L diag(beta)
  for (int e = threadIdx.x; e < kC * kC / 8; e += NTH) {
    const int i = e / (kC / 8), j = 8 * (e % (kC / 8));
    bf16x8 x = *reinterpret_cast<const bf16x8*>(sL + i * L6 + j);
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = (T)((float)x[u] * sB[j + u]);
    *reinterpret_cast<bf16x8*>(sT + i * L6 + j) = x;
  }
  // R = V - K H in place (each lane reads only its own V entries)
#pragma unroll kU
  for (int u_ = 0; u_ < NT / NCH; ++u_) {
    const int ct = ch + NCH * u_;
    f32x4 acc = zero4();
    #pragma unroll
    for (int kk = 0; kk < D; kk += 32) acc = mma32(arow(sK, kk), bcol(gH, sH, ct, kk), acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      T& x = sR[(r0 + tile_row(r)) * LD + 16 * ct + tile_col()];
      x = (T)((float)x - acc[r]);
    }
  }
  // P = tril(Q K^T), diagonal included
  #pragma unroll
  for (int u_ = 0; u_ < 4 / NCH; ++u_) {
    const int ct = ch + NCH * u_;
    f32x4 acc = zero4();
    if (ct <= rb)
      #pragma unroll
      for (int kk = 0; kk < D; kk += 32) acc = mma32(frow(sQ, LD, r0, kk), frow(sK, LD, 16 * ct, kk), acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = 16 * ct + tile_col() <= r0 + tile_row(r) ? acc[r] : 0.f;
    put_tile(sP, L6, r0, 16 * ct, acc);
  }
  __syncthreads();
  // Delta = T R; dDelta = K G + P^T dO
#pragma unroll kU
  for (int u_ = 0; u_ < NT / NCH; ++u_) {
    const int ct = ch + NCH * u_;
    f32x4 d = zero4(), dd = zero4();
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32) d = mma32(frow(sT, L6, r0, kk), fcol(sR, LD, 16 * ct, kk), d);
    #pragma unroll
    for (int kk = 0; kk < D; kk += 32) dd = mma32(arow(sK, kk), bcol(gG, sG, ct, kk), dd);
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32) dd = mma32(fcol(sP, L6, r0, kk), fcol(sO, LD, 16 * ct, kk), dd);
    put_tile(sD, LD, r0, 16 * ct, d);
    put_tile(sDD, LD, r0, 16 * ct, dd);
  }
  __syncthreads();
  // S2 = tril(dO Delta^T) over P; dT = dDelta R^T: dbeta_j gets sum_i dT_ij L_ij (column sums per
  // row block into sPart), dL = tril(dT) diag(beta); then dR = T^T dDelta (= dV; kept negated for
  // dK, over R at D 128 once every dT tile has read R)
  #pragma unroll
  for (int u_ = 0; u_ < 4 / NCH; ++u_) {
    const int ct = ch + NCH * u_;
    f32x4 s2 = zero4(), dt = zero4();
    if (ct <= rb) {
      #pragma unroll
      for (int kk = 0; kk < D; kk += 32) {
        s2 = mma32(frow(sO, LD, r0, kk), frow(sD, LD, 16 * ct, kk), s2);
        dt = mma32(frow(sDD, LD, r0, kk), frow(sR, LD, 16 * ct, kk), dt);
      }
    }
    const int j = 16 * ct + tile_col();
    float part = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r);
      part += dt[r] * (float)sL[i * L6 + j];
      s2[r] = j <= i ? s2[r] : 0.f;
      dt[r] = j <= i ? dt[r] * sB[j] : 0.f;
    }
    part = sum_over_rows(part);
    if ((threadIdx.x & 63) < 16) sPart[rb * kC + j] = part;
    put_tile(sS2, L6, r0, 16 * ct, s2);
    put_tile(sDL, L6, r0, 16 * ct, dt);
  }
  if constexpr (!kHGinLDS) __syncthreads();
#pragma unroll kU
  for (int u_ = 0; u_ < NT / NCH; ++u_) {
    const int ct = ch + NCH * u_;
    f32x4 acc = zero4();
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32) acc = mma32(fcol(sT, L6, r0, kk), fcol(sDD, LD, 16 * ct, kk), acc);
    store_rows<T, D>(dv, b, h, t0, N, H, r0, 16 * ct, acc);
    put_tile(sDR, LD, r0, 16 * ct, -acc);
  }
  __syncthreads();
  // dQ = dO H^T + S2 K; X1 = L^T dL over T (L^T upper, dL lower: k from max(rb, ct))
#pragma unroll kU
  for (int u_ = 0; u_ < NT / NCH; ++u_) {
    const int ct = ch + NCH * u_;
    f32x4 acc = zero4();
    #pragma unroll
    for (int kk = 0; kk < D; kk += 32) acc = mma32(arow(sO, kk), brow(gH, sH, ct, kk), acc);
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32) acc = mma32(frow(sS2, L6, r0, kk), fcol(sK, LD, 16 * ct, kk), acc);
    store_rows<T, D>(dq, b, h, t0, N, H, r0, 16 * ct, acc);
  }
  #pragma unroll
  for (int u_ = 0; u_ < 4 / NCH; ++u_) {  // (T was last read before the previous barrier)
    const int ct = ch + NCH * u_;
    f32x4 x1 = zero4();
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32)
      x1 = mma32(fcol(sL, L6, r0, kk), fcol(sDL, L6, 16 * ct, kk), x1);
    put_tile(sX1, L6, r0, 16 * ct, x1);
  }
  __syncthreads();
  // dA = -tril(X1 L^T, -1) (L^T[k][j] nonzero for k <= j); dbeta_i gets sum_m dA_im (k_i . k_m)
  // (row sums per column half into sRow); M = diag(beta) dA over dL
  float rows[4] = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
  for (int u_ = 0; u_ < 4 / NCH; ++u_) {
    const int ct = ch + NCH * u_;
    f32x4 da = zero4(), gk = zero4();
    if (ct <= rb) {
      #pragma unroll
      for (int kk = 0; kk < kC; kk += 32) da = mma32(frow(sX1, L6, r0, kk), frow(sL, L6, 16 * ct, kk), da);
      #pragma unroll
      for (int kk = 0; kk < D; kk += 32) gk = mma32(frow(sK, LD, r0, kk), frow(sK, LD, 16 * ct, kk), gk);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      da[r] = j < i ? -da[r] : 0.f;
      rows[r] += da[r] * gk[r];
      da[r] *= sB[i];
    }
    put_tile(sM, L6, r0, 16 * ct, da);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float x = group_sum<16>(rows[r]);
    if (tile_col() == 0) sRow[ch * kC + r0 + tile_row(r)] = x;
  }
  __syncthreads();
  // dK = Delta G^T + S2^T Q - dR H^T + M K + M^T K
#pragma unroll kU
  for (int u_ = 0; u_ < NT / NCH; ++u_) {
    const int ct = ch + NCH * u_;
    f32x4 acc = zero4();
    #pragma unroll
    for (int kk = 0; kk < D; kk += 32) {
      acc = mma32(arow(sD, kk), brow(gG, sG, ct, kk), acc);
      acc = mma32(arow(sDR, kk), brow(gH, sH, ct, kk), acc);
    }
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32) {
      acc = mma32(fcol(sS2, L6, r0, kk), fcol(sQ, LD, 16 * ct, kk), acc);
      acc = mma32(fcol(sM, L6, r0, kk), fcol(sK, LD, 16 * ct, kk), acc);
    }
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32) acc = mma32(frow(sM, L6, r0, kk), fcol(sK, LD, 16 * ct, kk), acc);
    store_rows<T, D>(dk, b, h, t0, N, H, r0, 16 * ct, acc);
  }
  const int i = threadIdx.x;
  if (i < kC && t0 + i < N) {
    float rs = sRow[i];
#pragma unroll
    for (int c2 = 1; c2 < NCH; ++c2) rs += sRow[c2 * kC + i];
    const float x = ((sPart[i] + sPart[kC + i]) + (sPart[2 * kC + i] + sPart[3 * kC + i])) + rs;
    dbeta[((size_t)b * N + t0 + i) * H + h] = (T)x;
  }
  __syncthreads();  // every read of this chunk's LDS is done before the next one is put
  }
}

// The prep kernel on bf16 LDS tiles (bf16 entry, head widths 32, 64 and 128). The UT solve stays
// in fp32; once it is done its two fp32 buffers hold the bf16 T and P, and (up to D 64) W and U,
// so that the kernel's LDS (about 74 KB at D 64) lets two workgroups share a CU.
template <int D, bool REC>
__global__ __launch_bounds__(kPrepThreads) void scan_bwd_prep_bf16_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const __bf16* __restrict__ beta, const __bf16* __restrict__ d_o, const uint8_t* __restrict__ active,
    float* __restrict__ ws, int N, int H, int NC) {
  using T = __bf16;
  constexpr int NT = D / 16, NTH = kPrepThreads;
  constexpr int LD = D + 8, L6 = kC + 8, PF = kC + 8;  // pitches: [64][D] bf16, [64][64] bf16, [64][64] fp32
  static_assert(2 * kC * L6 * sizeof(T) == kC * PF * sizeof(float), "T and P fit the fp32 buffer of A");
  constexpr bool kWUinL = 2 * kC * LD * sizeof(T) <= kC * PF * sizeof(float);  // W and U fit L's (D <= 64)
  __shared__ __align__(16) T sQ[kC * LD], sK[kC * LD], sV[kC * LD], sO[kC * LD];
  __shared__ __align__(16) float sA[kC * PF], sL[kC * PF];
  __shared__ __align__(16) T sWU[kWUinL ? 1 : 2 * kC * LD];
  __shared__ float sB[kC];
  T* sT = reinterpret_cast<T*>(sA);  // T = L diag(beta), then P beside it, once A is done with
  T* sP = sT + kC * L6;
  T* sW = kWUinL ? reinterpret_cast<T*>(sL) : sWU;  // W and U, over L once L is in bf16 (T) and saved
  T* sU = sW + kC * LD;
  T* sZ = sV;                        // Z = P^T dO once U is done
  const int c = blockIdx.x % NC, bh = blockIdx.x / NC;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * kC;
  const size_t chunk = blockIdx.x;
  const int w = threadIdx.x >> 6, ch = w >> 2, rb = ch == 0 ? w : 7 - w, r0 = 16 * rb;
  {
    ChunkRows16<D, NTH> rq, rk, rv, ro;
    ChunkBeta<T> rbeta;
    rk.fetch(k, b, h, t0, N, H);
    rq.fetch(q, b, h, t0, N, H);
    ro.fetch(d_o, b, h, t0, N, H, active);
    if constexpr (!REC) rv.fetch(v, b, h, t0, N, H);  // V only for U = T V and B = K^T U (the state chain)
    rbeta.fetch(beta, b, h, t0, N, H);
    rk.put(sK, LD);
    rq.put(sQ, LD);
    ro.put(sO, LD);
    if constexpr (!REC) rv.put(sV, LD);
    rbeta.put(sB, t0, N);
  }
  __syncthreads();
  // A = tril(diag(beta) K K^T, -1) in fp32
  #pragma unroll
  for (int u_ = 0; u_ < 2; ++u_) {
    const int ct = ch + 2 * u_;
    f32x4 acc = zero4();
    if (ct <= rb)
      #pragma unroll
      for (int kk = 0; kk < D; kk += 32) acc = mma32(frow(sK, LD, r0, kk), frow(sK, LD, 16 * ct, kk), acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + tile_row(r), j = 16 * ct + tile_col();
      sA[i * PF + j] = i > j ? sB[i] * acc[r] : 0.f;
    }
  }
  __syncthreads();
  // L = (I + A)^-1: the diagonal 16x16 blocks by forward substitution (a lane per column of a
  // block), then L_ij = -L_ii sum_{m = j}^{i - 1} A_im L_mj level by level on fp32 MFMA
#pragma unroll
  for (int e = threadIdx.x; e < kC * kC / 4; e += NTH) {
    const int i = e / (kC / 4), j = 4 * (e % (kC / 4));
    if (i / 16 < j / 16) *reinterpret_cast<f32x4*>(sL + i * PF + j) = zero4();
  }
  if (w == 0) {
    const int l = threadIdx.x & 63, blk = l >> 4, col = l & 15;
    const float* ab = sA + 16 * blk * PF + 16 * blk;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sum = i == col ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) sum -= ab[i * PF + m] * x[m];
      x[i] = sum;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sL[(16 * blk + i) * PF + 16 * blk + col] = x[i];
  }
  __syncthreads();
  #pragma unroll
  for (int lev = 1; lev < 4; ++lev) {
    const int i = w + lev, j = w;
    if (i < 4) {
      f32x4 y = zero4();
      #pragma unroll
      for (int m = j; m < i; ++m)
        y = mm16<false, false>(sA + 16 * i * PF + 16 * m, PF, sL + 16 * m * PF + 16 * j, PF, 16, y);
      float* dst = sL + 16 * i * PF + 16 * j;
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[tile_row(r) * PF + tile_col()] = y[r];
      wave_sync_lds();
      const f32x4 x = mm16<false, false>(sL + 16 * i * PF + 16 * i, PF, dst, PF, 16, zero4());
      wave_sync_lds();
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[tile_row(r) * PF + tile_col()] = -x[r];
    }
    __syncthreads();
  }
  // L into the workspace in bf16 (as the chunk kernel multiplies it); T = L diag(beta) in bf16 over A
  T* gL = reinterpret_cast<T*>(Ws<D>::L(ws, chunk));
  for (int e = threadIdx.x; e < kC * kC / 4; e += NTH) {
    const int i = e / (kC / 4), j = 4 * (e % (kC / 4));
    const f32x4 x = *reinterpret_cast<const f32x4*>(sL + i * PF + j);
    bf16x4 lb, t;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      lb[u] = (T)x[u];
      t[u] = (T)((float)lb[u] * sB[j + u]);
    }
    *reinterpret_cast<bf16x4*>(gL + 4 * e) = lb;
    *reinterpret_cast<bf16x4*>(sT + i * L6 + j) = t;
  }
  __syncthreads();
  // W = T K and (for the state chain) U = T V over L; P = tril(Q K^T) beside T
  #pragma unroll
  for (int u_ = 0; u_ < NT / 2; ++u_) {
    const int ct = ch + 2 * u_;
    f32x4 aw = zero4(), au = zero4();
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32) {
      const bf16x8 a = frow(sT, L6, r0, kk);
      aw = mma32(a, fcol(sK, LD, 16 * ct, kk), aw);
      if constexpr (!REC) au = mma32(a, fcol(sV, LD, 16 * ct, kk), au);
    }
    put_tile(sW, LD, r0, 16 * ct, aw);
    if constexpr (!REC) put_tile(sU, LD, r0, 16 * ct, au);
  }
  #pragma unroll
  for (int u_ = 0; u_ < 2; ++u_) {
    const int ct = ch + 2 * u_;
    f32x4 acc = zero4();
    if (ct <= rb)
      #pragma unroll
      for (int kk = 0; kk < D; kk += 32) acc = mma32(frow(sQ, LD, r0, kk), frow(sK, LD, 16 * ct, kk), acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = 16 * ct + tile_col() <= r0 + tile_row(r) ? acc[r] : 0.f;
    put_tile(sP, L6, r0, 16 * ct, acc);
  }
  __syncthreads();
  // Z = P^T dO over V (P^T upper triangular)
  #pragma unroll
  for (int u_ = 0; u_ < NT / 2; ++u_) {
    const int ct = ch + 2 * u_;
    f32x4 acc = zero4();
    #pragma unroll
    for (int kk = 0; kk < kC; kk += 32) acc = mma32(fcol(sP, L6, r0, kk), fcol(sO, LD, 16 * ct, kk), acc);
    put_tile(sZ, LD, r0, 16 * ct, acc);
  }
  __syncthreads();
  // the chains' operands, tile (rt, ct) of each [D x D] product: Y = Q^T dO - W^T Z and B = K^T U
  // in accumulator order, N = -K^T W into NR and N^T = -W^T K into NF (A tile (ct, rt) of each);
  // with the forward's records (REC) only the reverse chain runs, so B and N^T are not formed
  float* gY = Ws<D>::Y(ws, chunk);
  float* gB = Ws<D>::B(ws, chunk);
  __bf16* gNF = reinterpret_cast<__bf16*>(Ws<D>::NF(ws, chunk));
  __bf16* gNR = reinterpret_cast<__bf16*>(Ws<D>::NR(ws, chunk));
  const int l = threadIdx.x & 63;
  // a wave takes row tiles of one column tile, two at a time: each column fragment it reads (of
  // dO, Z, U, W, K) then serves both
  constexpr int RPW = NT * NT >= 8 ? NT * NT / 8 : 1;  // row tiles a wave
  constexpr int RSTEP = NT >= 8 ? 1 : 8 / NT;          // between a wave's row tiles
  constexpr int RG = RPW >= 2 ? 2 : 1;                 // row tiles at a time
  if (NT * NT >= 8 || w < NT * NT) {
    const int ct = w % NT, rt0 = w / NT;
#pragma unroll
    for (int j0 = 0; j0 < RPW; j0 += RG) {
      f32x4 y[RG], bb[RG], kw[RG], wk[RG];
#pragma unroll
      for (int j = 0; j < RG; ++j) y[j] = bb[j] = kw[j] = wk[j] = zero4();
#pragma unroll
      for (int kk = 0; kk < kC; kk += 32) {
        const bf16x8 ob = fcol(sO, LD, 16 * ct, kk), zb = -fcol(sZ, LD, 16 * ct, kk);
        const bf16x8 ub = REC ? bf16x8{} : fcol(sU, LD, 16 * ct, kk);
        const bf16x8 wb = fcol(sW, LD, 16 * ct, kk), kb = REC ? bf16x8{} : fcol(sK, LD, 16 * ct, kk);
#pragma unroll
        for (int j = 0; j < RG; ++j) {
          const int rt = rt0 + RSTEP * (j0 + j);
          const bf16x8 qa = fcol(sQ, LD, 16 * rt, kk), wa = fcol(sW, LD, 16 * rt, kk), ka = fcol(sK, LD, 16 * rt, kk);
          y[j] = mma32(qa, ob, y[j]);
          y[j] = mma32(wa, zb, y[j]);
          kw[j] = mma32(ka, wb, kw[j]);
          if constexpr (!REC) {
            bb[j] = mma32(ka, ub, bb[j]);
            wk[j] = mma32(wa, kb, wk[j]);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < RG; ++j) {
        const int rt = rt0 + RSTEP * (j0 + j);
        bf16x4 nr, nf, yb, bbb;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          nr[r] = (T)(-kw[j][r]);
          nf[r] = (T)(-wk[j][r]);
          yb[r] = (T)y[j][r];
          bbb[r] = (T)bb[j][r];
        }
        *reinterpret_cast<bf16x4*>(reinterpret_cast<T*>(gY) + accfrag2<NT>(ct, rt, l)) = yb;
        *reinterpret_cast<bf16x4*>(gNR + afrag<NT>(ct, rt, l)) = nr;
        if constexpr (!REC) {
          *reinterpret_cast<bf16x4*>(reinterpret_cast<T*>(gB) + accfrag2<NT>(ct, rt, l)) = bbb;
          *reinterpret_cast<bf16x4*>(gNF + afrag<NT>(ct, rt, l)) = nf;
        }
      }
    }
  }
}

size_t workspace_floats(int B, int N, int H, int D) {
  const size_t nc = (size_t)(N + kC - 1) / kC;
  const size_t per = (size_t)kC * kC + 6 * (size_t)D * D;
  return (size_t)B * H * nc * per;
}

// workgroups that stay resident at `per_cu` a CU on the current device
unsigned persistent_blocks(int per_cu) {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256u * per_cu;
  if (cus[dev] == 0 && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 256;
  return (unsigned)cus[dev] * per_cu;
}

// hrec: the chunk-start states the forward recorded (bf16, widths 32 and 64), or null: then the
// forward chain runs here as well.
template <typename TIn, int D>
void launch(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* state_in, const TIn* d_o,
            const float* d_state, const uint8_t* active, TIn* dq, TIn* dk, TIn* dv, TIn* dbeta, float* d_state_in,
            float* ws, int B, int N, int H, hipStream_t stream, const __bf16* hrec = nullptr) {
  const int NC = (N + kC - 1) / kC;
  const unsigned chunks = (unsigned)((size_t)B * H * NC), slices = (unsigned)((size_t)B * H * (D / 16));
  if constexpr (sizeof(TIn) == 2 && D >= 32) {
    if (hrec != nullptr)
      hipLaunchKernelGGL((scan_bwd_prep_bf16_kernel<D, true>), dim3(chunks), dim3(kPrepThreads), 0, stream, q, k, v,
                         beta, d_o, active, ws, N, H, NC);
    else
      hipLaunchKernelGGL((scan_bwd_prep_bf16_kernel<D, false>), dim3(chunks), dim3(kPrepThreads), 0, stream, q, k, v,
                         beta, d_o, active, ws, N, H, NC);
  } else {
    hipLaunchKernelGGL((scan_bwd_prep_kernel<TIn, D>), dim3(chunks), dim3(kPrepThreads), 0, stream, q, k, v, beta, d_o,
                       active, ws, N, H, NC);
  }
  hipLaunchKernelGGL((scan_bwd_chains_kernel<TIn, D>), dim3(hrec != nullptr ? slices : 2 * slices), dim3(64), 0, stream,
                     state_in, d_state, d_state_in, ws, NC, (int)slices, hrec != nullptr ? (int)slices : 0);
  if constexpr (sizeof(TIn) == 2 && D >= 32)
    hipLaunchKernelGGL((scan_bwd_chunk_bf16_kernel<D>), dim3(min(chunks, persistent_blocks(1))),
                       dim3(ChunkShape<D>::NTH), 0, stream, q, k, v, beta, d_o, active, ws, hrec, dq, dk, dv, dbeta, N, H,
                       NC, (int)chunks);
  else
    hipLaunchKernelGGL((scan_bwd_chunk_kernel<TIn, D>), dim3(chunks), dim3(kChunkThreads), 0, stream, q, k, v, beta, d_o,
                       active, ws, dq, dk, dv, dbeta, N, H, NC);
}

template <typename TIn>
int scan_backward(const TIn* q, const TIn* k, const TIn* v, const TIn* beta, const float* state_in, const TIn* d_o,
                  const float* d_state, const uint8_t* active, TIn* dq, TIn* dk, TIn* dv, TIn* dbeta,
                  float* d_state_in, void* workspace, size_t workspace_bytes, int B, int N, int H, int D,
                  void* stream_ptr, const char* who, const __bf16* hrec = nullptr) {
  if (B < 0 || N < 0 || H < 1) return fail(ERR_ARG, "%s: bad sizes B=%d N=%d H=%d", who, B, N, H);
  constexpr bool bf16 = sizeof(TIn) == 2;
  if (!(D == 16 || D == 32 || D == 64 || (D == 128 && bf16))) {
    // widths the chunked kernels do not tile: the wide backward (multiples of 16 up to 256)
    if (hrec != nullptr) return fail(ERR_UNSUPPORTED, "%s: head dimension %d with records", who, D);
    if constexpr (bf16)
      return scan_backward_wide_bf16(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in,
                                     workspace, workspace_bytes, B, N, H, D, static_cast<hipStream_t>(stream_ptr), who);
    else
      return scan_backward_wide_f32(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in,
                                    workspace, workspace_bytes, B, N, H, D, static_cast<hipStream_t>(stream_ptr), who);
  }
  if (B == 0 || N == 0) return OK;  // no token: the caller's state gradient passes through
  if (!q || !k || !v || !beta || !state_in || !d_o || !dq || !dk || !dv || !dbeta || !d_state_in)
    return fail(ERR_ARG, "%s: null pointer", who);
  // the chains address one (b, h)'s chunks of the workspace with 32-bit byte offsets
  if ((size_t)((N + kC - 1) / kC) * ((size_t)kC * kC + 6 * (size_t)D * D) * sizeof(float) >= ((size_t)1 << 32))
    return fail(ERR_UNSUPPORTED, "%s: %d tokens of width %d exceed the 4 GiB workspace a head", who, N, D);
  const size_t need = workspace_floats(B, N, H, D) * sizeof(float);
  if (!workspace || workspace_bytes < need)
    return fail(ERR_ARG, "%s: workspace of %zu bytes, %zu needed", who, workspace_bytes, need);
  if ((reinterpret_cast<uintptr_t>(workspace) | reinterpret_cast<uintptr_t>(state_in) |
       reinterpret_cast<uintptr_t>(d_state) | reinterpret_cast<uintptr_t>(d_state_in)) & 15)
    return fail(ERR_ARG, "%s: the states, their gradients and the workspace must be 16-byte aligned", who);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  float* ws = static_cast<float*>(workspace);
  switch (D) {
    case 16: launch<TIn, 16>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, ws, B, N, H, stream); break;
    case 32: launch<TIn, 32>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, ws, B, N, H, stream, hrec); break;
    case 64: launch<TIn, 64>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, ws, B, N, H, stream, hrec); break;
    default:
      if constexpr (bf16)
        launch<TIn, 128>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in, ws, B, N, H, stream);
      break;
  }
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" size_t vsp_delta_scan_backward_workspace_bytes(int B, int N, int H, int D) {
  if (B <= 0 || N <= 0 || H <= 0 || D <= 0) return 0;
  const size_t tiled = vsp::workspace_floats(B, N, H, D) * sizeof(float);
  if (D == 16 || D == 32 || D == 64) return tiled;
  const size_t wide = vsp::wide_backward_workspace_bytes(B, N, H, D);  // 0 where it does not run
  return D == 128 ? (tiled > wide ? tiled : wide) : wide;  // 128: tiled for bf16, wide for fp32
}

extern "C" int vsp_delta_scan_backward_bf16(const void* q, const void* k, const void* v, const void* beta,
                                            const float* state_in, const void* d_o, const float* d_state,
                                            const uint8_t* active, void* dq, void* dk, void* dv, void* dbeta,
                                            float* d_state_in, void* workspace, size_t workspace_bytes, int B, int N,
                                            int H, int D, void* stream) {
  using T = __bf16;
  return vsp::scan_backward<T>(static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                               static_cast<const T*>(beta), state_in, static_cast<const T*>(d_o), d_state, active,
                               static_cast<T*>(dq), static_cast<T*>(dk), static_cast<T*>(dv), static_cast<T*>(dbeta),
                               d_state_in, workspace, workspace_bytes, B, N, H, D, stream,
                               "vsp_delta_scan_backward_bf16");
}

extern "C" int vsp_delta_scan_backward_f32(const float* q, const float* k, const float* v, const float* beta,
                                           const float* state_in, const float* d_o, const float* d_state,
                                           const uint8_t* active, float* dq, float* dk, float* dv, float* dbeta,
                                           float* d_state_in, void* workspace, size_t workspace_bytes, int B, int N,
                                           int H, int D, void* stream) {
  return vsp::scan_backward<float>(q, k, v, beta, state_in, d_o, d_state, active, dq, dk, dv, dbeta, d_state_in,
                                   workspace, workspace_bytes, B, N, H, D, stream, "vsp_delta_scan_backward_f32");
}

extern "C" int vsp_delta_scan_backward_recorded_bf16(const void* q, const void* k, const void* v, const void* beta,
                                                     const float* state_in, const void* d_o, const float* d_state,
                                                     const uint8_t* active, const void* records, size_t records_bytes,
                                                     void* dq, void* dk, void* dv, void* dbeta, float* d_state_in,
                                                     void* workspace, size_t workspace_bytes, int B, int N, int H,
                                                     int D, void* stream) {
  using T = __bf16;
  const char* who = "vsp_delta_scan_backward_recorded_bf16";
  if (B > 0 && N > 0 && H > 0) {
    if (D != 32 && D != 64) return vsp::fail(vsp::ERR_UNSUPPORTED, "%s: head dimension %d (records: 32, 64)", who, D);
    const size_t need = (size_t)B * H * ((N + vsp::kC - 1) / vsp::kC) * D * D * sizeof(T);
    if (records == nullptr || records_bytes < need || (reinterpret_cast<uintptr_t>(records) & 15))
      return vsp::fail(vsp::ERR_ARG, "%s: records of %zu bytes (16-byte aligned) needed, %zu given", who, need,
                       records ? records_bytes : (size_t)0);
  }
  return vsp::scan_backward<T>(static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                               static_cast<const T*>(beta), state_in, static_cast<const T*>(d_o), d_state, active,
                               static_cast<T*>(dq), static_cast<T*>(dk), static_cast<T*>(dv), static_cast<T*>(dbeta),
                               d_state_in, workspace, workspace_bytes, B, N, H, D, stream, who,
                               static_cast<const T*>(records));
}
