// Sliding-window causal attention on CDNA4 (gfx950): the prefill kernel.
//
// Semantics (reference vesper/kernels/window_attn.py:27-39): q [B, N, H, D] against keys, values
// [B, M + N, HKV, D] whose first M rows are the cache; query i sits at key index M + i and attends
// key indices [M + i - W + 1, M + i]; scale 1/sqrt(D); query head h reads KV head h / (H / HKV).
//
// One workgroup = 128 queries of one (b, h): four waves of 32 queries, each as two 16-query
// blocks, so every K or V fragment read from LDS feeds two MFMAs. Key tiles of 64 rows walk the
// window through double-buffered LDS (one barrier per tile; the next tile's global loads are in
// flight while the current one is used). Per tile and query block a wave computes the transposed
// score tile S^T = K Q^T (16x16x32 MFMA, K rows from LDS as the A operand, Q in registers as the
// B operand), so a lane holds 16 keys of one query: the row maximum needs two lane swaps
// (v_permlane16/32_swap) and the probabilities are already laid out as the B operand of
// O^T += V^T P^T. V stays row-major in LDS; its transposed A fragments come from ds_read_b64_tr_b16.
// At D >= 64 the tiles go from global memory straight into LDS (global_load_lds_dwordx4), with no
// staging registers; K rows carry one 16-byte pad segment and V rows two, against bank conflicts.
//
// Softmax: exp2 with the scale folded into one FMA per score; the running maximum is only moved
// when a tile's maximum exceeds it by more than kLazy (log2 units), so the O rescale runs about
// once per query instead of once per tile (probabilities then reach at most 2^kLazy, which bf16
// P and the fp32 sums hold exactly as well). Only tiles that cross the causal diagonal, the
// window's lower edge or the end of the keys are masked.
#include "attn_mma.h"
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr float kLazy = 8.f;

// Where the key rows come from (SRC):
//  * kSrcPlain: keys / values [B, M + N, HKV, D], the cache's M rows first;
//  * kSrcCarried (copy-forward): as plain, but key rows M + t of an inactive token t come from
//    keys_c / values_c row t ([B, N, HKV, D], the carried keys and values);
//  * kSrcCached: rows below M from keys / values as the cache alone ([B, M, HKV, D]) and rows M + t
//    from keys_c / values_c row t (the chunk's own keys and values, [B, N, HKV, D]), so a chunk
//    attends over a cache without the two being copied into one tensor first. Whole tiles on either
//    side go through a buffer resource over their tensor; the one tile across row M picks each
//    row's source by a per-lane address.
// The per-lane 64-bit source addresses need more registers: three workgroups per CU at D 64
// instead of four.
constexpr int kSrcPlain = 0, kSrcCarried = 1, kSrcCached = 2;
template <typename T, int D, int SRC>
__global__ __launch_bounds__(256, D >= 256 ? 1 : (D >= 128 ? 2 : (SRC != kSrcPlain && D == 64 ? 3 : 4))) void window_attn_kernel(const T* __restrict__ q, const T* __restrict__ keys,
                                                             const T* __restrict__ values, T* __restrict__ o,
                                                             float* __restrict__ lse,
                                                             const uint8_t* __restrict__ active, const T* keys_c,
                                                             const T* values_c, int N, int M, int H,
                                                             int HKV, int W, float scale_log2, int nqt) {
  using V8 = typename Mma<T>::V8;
  using V4 = typename Mma<T>::V4;
  constexpr bool CARRY = SRC == kSrcCarried, CACHED = SRC == kSrcCached;
  constexpr int QT = 128;              // queries per workgroup
  constexpr int QB = 2;                // 16-query blocks per wave
  constexpr int KT = 64;               // keys per tile
  constexpr int DP = D < 32 ? 32 : D;  // feature extent padded to the MFMA k step
  constexpr int DT = DP / 16;          // 16-row tiles of O^T
  constexpr int KSQ = DP / 32;         // k steps over features
  constexpr int SEG = DP / 8;          // 16-byte segments per row
  // LDS layouts against bank conflicts on the 64 banks. A 16-byte row-fragment read serves lanes
  // 0-7 and 16-23 (then 8-15 and 24-31, ...) in one pass: at D 64 the K rows are unpadded and
  // their 16-byte segments XOR-swizzled by row (segment s of row r at s ^ 2 ((r >> 1) & 3)), so
  // the 16 lanes of a pass, rows 0-7 at two segments each, meet every bank once; a 36-bank pitch
  // (one pad segment, kept at other widths) costs these reads a second pass. V rows carry two pad
  // segments (the 8 rows of a transposed read start 8, 24 or 40 banks apart and cover all 64).
  constexpr bool kSwzK = D == 64;
  constexpr int PK = kSwzK ? DP : DP + 8, PSEG = kSwzK ? SEG : SEG + 1;
  constexpr int PV = DP + 16, PSEGV = SEG + 2;
  // At D >= 64 the tiles go from global memory straight into LDS: a wave instruction fills 1 KiB
  // of consecutive segments (pad segments re-read a real one and are never used); narrower heads,
  // whose rows need zero padding up to the MFMA k step, stage through registers.
  constexpr bool kDirect = D >= 64;
  constexpr int NINS = KT * PSEG / 64, NINSV = KT * PSEGV / 64;  // wave instructions per K, V tile
  constexpr int NI = kDirect ? (NINSV + 3) / 4 : (KT * SEG + 255) / 256;
  // Separate variables per buffer, each tile's buffers fixed at compile time (the tile loop runs
  // two tiles an iteration): the compiler then tells the direct loads into one buffer from the
  // reads of the other and does not wait for the next tile's loads before reading this one.
  __shared__ __align__(16) T sK0[KT * PK], sK1[KT * PK];
  __shared__ __align__(16) T sV0[KT * PV], sV1[KT * PV];

  auto kswz = [](int row) { return kSwzK ? 2 * ((row >> 1) & 3) : 0; };  // K's segment swizzle
  const int lg = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qt = lg % nqt, bh = lg / nqt;
  const int b = bh / H, h = bh - b * H;
  const int kvh = h / (H / HKV);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lq = l & 15, g = l >> 4;
  const int S = M + N;
  const int qbase = qt * QT;
  const int wq0 = qbase + 32 * w;  // the wave's first query

  bool qok[QB], act[QB];
  bool any = false;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int myq = wq0 + 16 * qb + lq;
    qok[qb] = myq < N;
    act[qb] = qok[qb] && (active == nullptr || active[(size_t)b * N + myq] != 0);
    any |= act[qb];
  }
  if (!__syncthreads_or(any)) {  // every query of the tile is inactive (or past N): zeros
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int myq = wq0 + 16 * qb + lq;
      if (qok[qb] && g == 0) {
        T* dst = o + (((size_t)b * N + myq) * H + h) * D;
        for (int d = 0; d < D; ++d) dst[d] = from_f32<T>(0.f);
        if (lse != nullptr) lse[((size_t)b * H + h) * N + myq] = INFINITY;
      }
    }
    return;
  }

  V8 qf[QB][KSQ];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int myq = wq0 + 16 * qb + lq;
#pragma unroll
    for (int s = 0; s < KSQ; ++s) {
      const int f = 32 * s + 8 * g;
      if (qok[qb] && f < D) {
        qf[qb][s] = *reinterpret_cast<const V8*>(q + (((size_t)b * N + myq) * H + h) * D + f);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) qf[qb][s][j] = from_f32<T>(0.f);
      }
    }
  }

  const int kfirst = max(0, M + qbase - W + 1);
  const int klast = min(S, M + qbase + QT);
  const int ntiles = (klast - kfirst + KT - 1) / KT;
  const size_t kv_row = (size_t)HKV * D;
  const T* kbase = keys + ((size_t)b * (CACHED ? M : S) * HKV + kvh) * D;
  const T* vbase = values + ((size_t)b * (CACHED ? M : S) * HKV + kvh) * D;
  // carried (or the chunk's own) rows, indexed by key index (valid from M on)
  const T* kcbase = CARRY || CACHED ? keys_c + ((size_t)b * N * HKV + kvh) * D - (size_t)M * kv_row : kbase;
  const T* vcbase = CARRY || CACHED ? values_c + ((size_t)b * N * HKV + kvh) * D - (size_t)M * kv_row : vbase;
  // cached: bit r of a tile's mask says key k0 + r is a cache row
  auto cache_rows = [&](int k0) -> uint64_t {
    return k0 >= M ? 0ull : (M - k0 >= 64 ? ~0ull : ((1ull << (M - k0)) - 1ull));
  };
  // With carried rows, each tile's 64 source flags (bit r: key k0 + r reads the fresh row) are
  // loaded one tile ahead (lane l: key k0 + l) and turned into a wave-uniform mask when issued.
  auto flag_of = [&](int k0) -> uint8_t {
    const int s = k0 + l;
    const uint8_t f = active[(size_t)b * N + min(max(s - M, 0), N - 1)];
    return (s < M || s >= S) ? (uint8_t)1 : f;  // cache rows and rows past the end: fresh
  };

  // staging of one 64-key tile. At D >= 64 through buffer resources over the (b, KV head) rows:
  // each lane's offset within a tile is fixed (computed once), rows past the last key read zeros,
  // and keys past klast that do load are masked in the scores (weight 0 in the output). Narrower
  // heads: keys past klast re-read key klast - 1.
  V8 kreg[kDirect ? 1 : NI], vreg[kDirect ? 1 : NI];
  const unsigned kv_bytes =
      CACHED ? (M > 0 ? (unsigned)(((size_t)(M - 1) * kv_row + D) * sizeof(T)) : 0u)
             : (unsigned)(((size_t)(S - 1) * kv_row + D) * sizeof(T));
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kbase, kv_bytes), rv = buffer_rsrc(vbase, kv_bytes);
  // cached: the chunk's rows, from key index M on
  const unsigned kvc_bytes = CACHED ? (unsigned)(((size_t)(N - 1) * kv_row + D) * sizeof(T)) : 0u;
  const __amdgpu_buffer_rsrc_t rkc = buffer_rsrc(kcbase + (size_t)M * kv_row, kvc_bytes);
  const __amdgpu_buffer_rsrc_t rvc = buffer_rsrc(vcbase + (size_t)M * kv_row, kvc_bytes);
  unsigned koff[kDirect ? NI : 1], voff[kDirect ? NI : 1];
#pragma unroll
  for (int j = 0; j < (kDirect ? NI : 1); ++j) {
    const int pos = (w + 4 * j) * 64 + l;  // padded segment position in the tile
    const int row = pos / PSEG, seg = pos - row * PSEG;  // LDS position: the segment it holds is seg ^ kswz(row)
    koff[j] = (unsigned)(row * kv_row + 8 * (seg < SEG ? seg ^ kswz(row) : 0)) * (unsigned)sizeof(T);
    const int rowv = pos / PSEGV, segv = pos - rowv * PSEGV;
    voff[j] = (unsigned)(rowv * kv_row + 8 * (segv < SEG ? segv : 0)) * (unsigned)sizeof(T);
  }
  auto fetch = [&](int k0, T* Kn, T* Vn, uint64_t fresh) {
    if constexpr (CACHED) fresh = cache_rows(k0);
    // cached: a whole tile on one side of row M loads through that tensor's buffer resource
    const bool whole = CACHED && (k0 >= M || k0 + KT <= M);
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      if constexpr (kDirect && CACHED) {
        if (whole) {
          const int ins = w + 4 * j;
          const bool chunk = k0 >= M;
          const unsigned toff = (unsigned)((size_t)(chunk ? k0 - M : k0) * kv_row * sizeof(T));
          if (ins < NINS) buffer_load_lds16(chunk ? rkc : rk, Kn + ins * 64 * 8, koff[j], toff);
          if (ins < NINSV) buffer_load_lds16(chunk ? rvc : rv, Vn + ins * 64 * 8, voff[j], toff);
          continue;
        }
      }
      if constexpr (kDirect && (CARRY || CACHED)) {
        // per-lane sources (global direct loads: a buffer resource cannot differ between lanes);
        // rows past the last key re-read key S - 1, from that key's own source (masked in the
        // scores, they must still be finite: probability 0 times the row)
        const int ins = w + 4 * j;
        const int pos = ins * 64 + l;
        const int row = pos / PSEG, seg = pos - row * PSEG;
        const int rowv = pos / PSEGV, segv = pos - rowv * PSEGV;
        const int key = min(k0 + row, S - 1), keyv = min(k0 + rowv, S - 1);
        const size_t sk = (size_t)key * kv_row + 8 * (seg < SEG ? seg ^ kswz(row) : 0);
        const size_t sv = (size_t)keyv * kv_row + 8 * (segv < SEG ? segv : 0);
        if (ins < NINS) load_lds16((((fresh >> (key - k0)) & 1) ? kbase : kcbase) + sk, Kn + ins * 64 * 8);
        if (ins < NINSV) load_lds16((((fresh >> (keyv - k0)) & 1) ? vbase : vcbase) + sv, Vn + ins * 64 * 8);
      } else if constexpr (kDirect) {
        const int ins = w + 4 * j;  // this wave's j-th instruction of the tile
        const unsigned toff = (unsigned)((size_t)k0 * kv_row * sizeof(T));
        if (ins < NINS) buffer_load_lds16(rk, Kn + ins * 64 * 8, koff[j], toff);
        if (ins < NINSV) buffer_load_lds16(rv, Vn + ins * 64 * 8, voff[j], toff);
      } else {
        const int sg = threadIdx.x + 256 * j;
        const int row = sg / SEG, part = sg - row * SEG;
        const int key = min(k0 + row, klast - 1);  // the key loaded, with its own source flag
        const size_t goff = (size_t)key * kv_row + 8 * part;
        const bool from_fresh = !(CARRY || CACHED) || ((fresh >> ((key - k0) & 63)) & 1);  // (key - k0 < 64 where it loads)
        if (sg < KT * SEG && 8 * part < D) {
          kreg[j] = *reinterpret_cast<const V8*>((from_fresh ? kbase : kcbase) + goff);
          vreg[j] = *reinterpret_cast<const V8*>((from_fresh ? vbase : vcbase) + goff);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            kreg[j][e] = from_f32<T>(0.f);
            vreg[j][e] = from_f32<T>(0.f);
          }
        }
      }
    }
  };
  auto stash = [&](T* Kn, T* Vn) {
    if constexpr (!kDirect) {
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int sg = threadIdx.x + 256 * j;
        if (sg < KT * SEG) {
          const int row = sg / SEG, part = sg - row * SEG;
          *reinterpret_cast<V8*>(Kn + row * PK + 8 * part) = kreg[j];
          *reinterpret_cast<V8*>(Vn + row * PV + 8 * part) = vreg[j];
        }
      }
    }
  };

  // lacc: the row sums of the probabilities as rounded for the P V product, by one more MFMA per
  // key step with an all-ones A operand (every lane then holds its query's sum, and no VALU adds)
  float m_used[QB];
  f32x4 oacc[QB][DT], lacc[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_used[qb] = -1e30f;  // finite: exp2 of a masked score minus it is exactly 0
    lacc[qb] = zero4();
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[qb][t] = zero4();
  }
  V8 ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = from_f32<T>(1.f);
  // the wave's queries in key-index space: [wlo, whi]
  const int wlo = M + wq0, whi = M + wq0 + 31;

  uint8_t fl = 1;  // CARRY: lane l's flag of the next tile to issue
  uint64_t fresh = ~0ull;
  if constexpr (CARRY) {
    fresh = __builtin_amdgcn_ballot_w64(flag_of(kfirst) != 0);
    fl = flag_of(kfirst + KT);
  }
  fetch(kfirst, sK0, sV0, fresh);
  stash(sK0, sV0);
  if constexpr (kDirect) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct loads
  __syncthreads();
  // one tile: K, V in Kt, Vt; the next tile's loads go to Kn, Vn (last read before the previous barrier)
  auto tile = [&](int it, const T* Kt, const T* Vt, T* Kn, T* Vn) {
    const int k0 = kfirst + it * KT;
    // a wave in the first half of its tiles issues ahead of those in their second half: the four
    // workgroups of a CU then finish closer together (issue goes oldest-first otherwise, and the
    // last workgroup would run its final tiles alone on the CU)
    if (2 * it < ntiles)
      __builtin_amdgcn_s_setprio(1);
    else
      __builtin_amdgcn_s_setprio(0);
    if (it + 1 < ntiles) {
      if constexpr (CARRY) {
        fresh = __builtin_amdgcn_ballot_w64(fl != 0);
        fl = flag_of(k0 + 2 * KT);
      }
      fetch(k0 + KT, Kn, Vn, fresh);
    }

    // skip a tile this wave's queries cannot see (wave-uniform)
    const bool seen = k0 <= whi && k0 + KT - 1 > wlo - W;
    if (seen) {
      // masks only where needed: the causal edge (some key after some query of the wave, or keys
      // past the last one) and the window's lower edge (some key too old for the wave's last query)
      const bool cmask = k0 + KT - 1 > wlo || k0 + KT > klast;
      const bool wmask = k0 <= whi - W;
      f32x4 sacc[QB][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = zero4();
#pragma unroll
        for (int st = 0; st < KSQ; ++st) {
          const V8 a = *reinterpret_cast<const V8*>(Kt + (16 * kb + lq) * PK + 8 * ((4 * st + g) ^ kswz(lq)));
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = Mma<T>::run(a, qf[qb][st], sacc[qb][kb]);
        }
      }
      V8 pb[QB][2];
      // both query blocks' maxima first, then one wave-uniform decision on rescaling, so that the
      // exponentials of the two blocks form one stretch of independent work
      float mt[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        // key k0 + 4 g + e (e = 16 kb + r) is visible to query qidx iff qidx - W < key <= qidx, that
        // is iff c - W < e <= c with c = qidx - k0 - 4 g (each test one compare with a constant);
        // every query that is stored has qidx < klast, so keys at or past klast fail the first
        const int c = wlo + 16 * qb + lq - k0 - 4 * g;
        if (cmask) {
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) sacc[qb][kb][r] = 16 * kb + r <= c ? sacc[qb][kb][r] : -INFINITY;
        }
        if (wmask) {
          const int cw = c - W;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) sacc[qb][kb][r] = 16 * kb + r > cw ? sacc[qb][kb][r] : -INFINITY;
        }
        mt[qb] = sacc[qb][0][0];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) mt[qb] = fmax_ieee(mt[qb], sacc[qb][kb][r]);
      }
      bool need[QB], any_need = false;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        mt[qb] = max_over_groups(mt[qb]) * scale_log2;
        need[qb] = mt[qb] > m_used[qb] + kLazy;
        any_need |= need[qb];
      }
      if (__builtin_amdgcn_ballot_w64(any_need)) {  // some query of the wave moves its maximum
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float mn = need[qb] ? mt[qb] : m_used[qb];
          const float alpha = __builtin_amdgcn_exp2f(m_used[qb] - mn);
          lacc[qb] *= alpha;
#pragma unroll
          for (int t = 0; t < DT; ++t) oacc[qb][t] *= alpha;
          m_used[qb] = mn;
        }
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float p[4][4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) p[kb][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][kb][r], scale_log2, -m_used[qb]));
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            pb[qb][ks][j] = from_f32<T>(p[2 * ks][j]);
            pb[qb][ks][4 + j] = from_f32<T>(p[2 * ks + 1][j]);
          }
      }
      // O^T += V^T P^T: A fragments of V^T by transposed LDS reads (lane (lq, g) gets column
      // 16 t + lq of key rows 32 ks + 4 g .. +3 and 32 ks + 16 + 4 g .. +3)
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const T* base = Vt + (32 * ks + 4 * g + (lq >> 2)) * PV + 16 * t + 4 * (lq & 3);
          const V4 lo = read_tr<T>(base);
          const V4 hi = read_tr<T>(base + 16 * PV);
          const V8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) oacc[qb][t] = Mma<T>::run(a, pb[qb][ks], oacc[qb][t]);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) lacc[qb] = Mma<T>::run(ones, pb[qb][ks], lacc[qb]);
    }
    if (it + 1 < ntiles) stash(Kn, Vn);
    if constexpr (kDirect) __builtin_amdgcn_s_waitcnt(0x0F70);  // the next tile's direct loads
    __syncthreads();
  };
  int it = 0;
  for (; it + 1 < ntiles; it += 2) {
    tile(it, sK0, sV0, sK1, sV1);
    tile(it + 1, sK1, sV1, sK0, sV0);
  }
  if (it < ntiles) tile(it, sK0, sV0, sK1, sV1);

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float lt = lacc[qb][0];
    const float inv = (act[qb] && lt > 0.f) ? 1.f / lt : 0.f;
    // the log-sum-exp in log2 units of the scaled scores, for the backward: P = exp2(s sl2 - lse);
    // +inf for an inactive query, whose probabilities (and gradients) are then exactly zero
    if (lse != nullptr && qok[qb] && g == 0)
      lse[((size_t)b * H + h) * N + wq0 + 16 * qb + lq] = inv > 0.f ? m_used[qb] + log2f(lt) : INFINITY;
    if (qok[qb]) {
      T* dst = o + (((size_t)b * N + wq0 + 16 * qb + lq) * H + h) * D;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int d = 16 * t + 4 * g;
        if (d < D) {
          V4 v;
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = from_f32<T>(oacc[qb][t][r] * inv);
          *reinterpret_cast<V4*>(dst + d) = v;
        }
      }
    }
  }
}

bool attn_width(int D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

template <typename T, int SRC>
void launch_window(dim3 grid, hipStream_t stream, const T* q, const T* keys, const T* values, T* o, float* lse,
                   const uint8_t* active, const T* kc, const T* vc, int N, int M, int H, int HKV, int D, int W,
                   float scale_log2, int nqt) {
  switch (D) {
    case 16: hipLaunchKernelGGL((window_attn_kernel<T, 16, SRC>), grid, dim3(256), 0, stream, q, keys, values, o, lse, active, kc, vc, N, M, H, HKV, W, scale_log2, nqt); break;
    case 32: hipLaunchKernelGGL((window_attn_kernel<T, 32, SRC>), grid, dim3(256), 0, stream, q, keys, values, o, lse, active, kc, vc, N, M, H, HKV, W, scale_log2, nqt); break;
    case 64: hipLaunchKernelGGL((window_attn_kernel<T, 64, SRC>), grid, dim3(256), 0, stream, q, keys, values, o, lse, active, kc, vc, N, M, H, HKV, W, scale_log2, nqt); break;
    case 128: hipLaunchKernelGGL((window_attn_kernel<T, 128, SRC>), grid, dim3(256), 0, stream, q, keys, values, o, lse, active, kc, vc, N, M, H, HKV, W, scale_log2, nqt); break;
    default: hipLaunchKernelGGL((window_attn_kernel<T, 256, SRC>), grid, dim3(256), 0, stream, q, keys, values, o, lse, active, kc, vc, N, M, H, HKV, W, scale_log2, nqt); break;
  }
}

template <typename T>
int window_attn(const T* q, const T* keys, const T* values, T* o, float* lse, const uint8_t* active, int B, int N, int M,
                int H, int HKV, int D, int W, float scale, void* stream_ptr, const char* who, const T* kc = nullptr,
                const T* vc = nullptr, bool cached = false) {
  if (B < 0 || N < 0 || M < 0 || H < 1 || HKV < 1) return fail(ERR_ARG, "%s: bad sizes B=%d N=%d M=%d H=%d HKV=%d", who, B, N, M, H, HKV);
  if (H % HKV != 0) return fail(ERR_ARG, "%s: %d query heads are not a multiple of %d KV heads", who, H, HKV);
  if (W < 1) return fail(ERR_ARG, "%s: window must be at least 1, got %d", who, W);
  if (!(scale > 0.f)) return fail(ERR_ARG, "%s: the score scale must be positive, got %g", who, (double)scale);
  if (!attn_width(D)) return fail(ERR_UNSUPPORTED, "%s: head dimension %d (kernels: 16, 32, 64, 128, 256)", who, D);
  if (B == 0 || N == 0) return OK;
  // (a cached call with no cache rows may pass null for them)
  if (!q || !o || ((!keys || !values) && !(cached && M == 0))) return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(values) |
       reinterpret_cast<uintptr_t>(o)) & 15)
    return fail(ERR_ARG, "%s: q, keys, values and o must be 16-byte aligned", who);
  if (reinterpret_cast<uintptr_t>(lse) & 3) return fail(ERR_ARG, "%s: lse must be 4-byte aligned", who);
  if (cached) {
    if (!kc || !vc) return fail(ERR_ARG, "%s: null pointer", who);
    if ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & 15)
      return fail(ERR_ARG, "%s: the chunk's keys and values must be 16-byte aligned", who);
  } else if (kc != nullptr || vc != nullptr) {
    if (!kc || !vc) return fail(ERR_ARG, "%s: the carried keys and values come together", who);
    if (!active) return fail(ERR_ARG, "%s: carried keys and values need the active flags", who);
    if ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & 15)
      return fail(ERR_ARG, "%s: the carried keys and values must be 16-byte aligned", who);
  }
  // one batch row's keys (all KV heads) are addressed with 32-bit byte offsets
  if ((size_t)(M + N) * HKV * D * sizeof(T) >= ((size_t)1 << 32))
    return fail(ERR_UNSUPPORTED, "%s: %d keys x %d KV heads x %d features exceed 4 GiB per batch row", who, M + N, HKV, D);
  const float scale_log2 = scale * 1.4426950408889634f;
  const int nqt = (N + 127) / 128;
  dim3 grid((unsigned)((size_t)nqt * H * B));
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  if (cached)
    launch_window<T, kSrcCached>(grid, stream, q, keys, values, o, lse, active, kc, vc, N, M, H, HKV, D, W, scale_log2,
                                 nqt);
  else if (kc != nullptr)
    launch_window<T, kSrcCarried>(grid, stream, q, keys, values, o, lse, active, kc, vc, N, M, H, HKV, D, W, scale_log2,
                                  nqt);
  else
    launch_window<T, kSrcPlain>(grid, stream, q, keys, values, o, lse, active, kc, vc, N, M, H, HKV, D, W, scale_log2,
                                nqt);
  return check_launch(who);
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_window_attn_bf16(const void* q, const void* keys, const void* values, void* o, const uint8_t* active,
                                    int B, int N, int M, int H, int HKV, int D, int window, float scale, void* stream) {
  return vsp::window_attn<__bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(keys),
                                  static_cast<const __bf16*>(values), static_cast<__bf16*>(o), nullptr, active, B, N, M,
                                  H, HKV, D, window, scale, stream, "vsp_window_attn_bf16");
}

extern "C" int vsp_window_attn_lse_bf16(const void* q, const void* keys, const void* values, void* o, float* lse,
                                        const uint8_t* active, int B, int N, int M, int H, int HKV, int D, int window,
                                        float scale, void* stream) {
  return vsp::window_attn<__bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(keys),
                                  static_cast<const __bf16*>(values), static_cast<__bf16*>(o), lse, active, B, N, M, H,
                                  HKV, D, window, scale, stream, "vsp_window_attn_lse_bf16");
}

extern "C" int vsp_window_attn_f16(const void* q, const void* keys, const void* values, void* o, const uint8_t* active,
                                   int B, int N, int M, int H, int HKV, int D, int window, float scale, void* stream) {
  return vsp::window_attn<_Float16>(static_cast<const _Float16*>(q), static_cast<const _Float16*>(keys),
                                    static_cast<const _Float16*>(values), static_cast<_Float16*>(o), nullptr, active, B,
                                    N, M, H, HKV, D, window, scale, stream, "vsp_window_attn_f16");
}

extern "C" int vsp_window_attn_lse_f16(const void* q, const void* keys, const void* values, void* o, float* lse,
                                       const uint8_t* active, int B, int N, int M, int H, int HKV, int D, int window,
                                       float scale, void* stream) {
  return vsp::window_attn<_Float16>(static_cast<const _Float16*>(q), static_cast<const _Float16*>(keys),
                                    static_cast<const _Float16*>(values), static_cast<_Float16*>(o), lse, active, B, N,
                                    M, H, HKV, D, window, scale, stream, "vsp_window_attn_lse_f16");
}

extern "C" int vsp_window_attn_carried_bf16(const void* q, const void* keys, const void* values, const void* keys_carried,
                                            const void* values_carried, void* o, const uint8_t* active, int B, int N,
                                            int M, int H, int HKV, int D, int window, float scale, void* stream) {
  using T = __bf16;
  return vsp::window_attn<T>(static_cast<const T*>(q), static_cast<const T*>(keys), static_cast<const T*>(values),
                             static_cast<T*>(o), nullptr, active, B, N, M, H, HKV, D, window, scale, stream,
                             "vsp_window_attn_carried_bf16", static_cast<const T*>(keys_carried),
                             static_cast<const T*>(values_carried));
}

extern "C" int vsp_window_attn_carried_f16(const void* q, const void* keys, const void* values, const void* keys_carried,
                                           const void* values_carried, void* o, const uint8_t* active, int B, int N,
                                           int M, int H, int HKV, int D, int window, float scale, void* stream) {
  using T = _Float16;
  return vsp::window_attn<T>(static_cast<const T*>(q), static_cast<const T*>(keys), static_cast<const T*>(values),
                             static_cast<T*>(o), nullptr, active, B, N, M, H, HKV, D, window, scale, stream,
                             "vsp_window_attn_carried_f16", static_cast<const T*>(keys_carried),
                             static_cast<const T*>(values_carried));
}

extern "C" int vsp_window_attn_cached_bf16(const void* q, const void* cache_keys, const void* cache_values,
                                           const void* keys, const void* values, void* o, const uint8_t* active, int B,
                                           int N, int M, int H, int HKV, int D, int window, float scale, void* stream) {
  using T = __bf16;
  return vsp::window_attn<T>(static_cast<const T*>(q), static_cast<const T*>(cache_keys),
                             static_cast<const T*>(cache_values), static_cast<T*>(o), nullptr, active, B, N, M, H, HKV, D,
                             window, scale, stream, "vsp_window_attn_cached_bf16", static_cast<const T*>(keys),
                             static_cast<const T*>(values), true);
}

extern "C" int vsp_window_attn_cached_f16(const void* q, const void* cache_keys, const void* cache_values,
                                          const void* keys, const void* values, void* o, const uint8_t* active, int B,
                                          int N, int M, int H, int HKV, int D, int window, float scale, void* stream) {
  using T = _Float16;
  return vsp::window_attn<T>(static_cast<const T*>(q), static_cast<const T*>(cache_keys),
                             static_cast<const T*>(cache_values), static_cast<T*>(o), nullptr, active, B, N, M, H, HKV, D,
                             window, scale, stream, "vsp_window_attn_cached_f16", static_cast<const T*>(keys),
                             static_cast<const T*>(values), true);
}
