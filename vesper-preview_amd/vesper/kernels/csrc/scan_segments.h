// Segmented chunk scan, bf16 inputs at head width 64 (included by delta_scan.hip inside its
// namespace, after the chain kernels whose fragment helpers it shares).
//
// One workgroup holds the whole 64 x 64 fp32 state of one (b, h) for one segment of consecutive
// 64-token chunks, so the state-independent products of a chunk (-W = -T K, K^T, U = T V,
// P^T = tril(Q K^T)^T) are formed once for all 64 value columns. The sequence of each head is cut
// into segments so that B * H * segments workgroups fill the chip. A segment's effect on the state
// is the affine map H -> X + M H (X: the state the segment leaves from a zero start, M: the product
// of its chunks' I - K^T W), so:
//
//  * delta_seg_kernel<kSegMaps> runs every segment but the last once without outputs, carrying
//    [X | M] through its chunks (M from I, X from zero; the first segment carries the true state
//    from S0 instead and needs no M), and writes X and M (fp32, row-major [64][64]) to the
//    workspace; its first segment also copies S0 there, so that the output pass may write the
//    final state over S0 (s_out == s_in) while its first segment still reads the copy;
//  * delta_seg_kernel<kSegOutputs> starts segment s from H = X_0, folded through the maps of
//    segments 1 .. s - 1 (H <- X_i + M_i H, three bf16 products per tile: hi*hi + hi*lo + lo*hi),
//    then runs its chunks with the outputs; the last segment writes the final state.
//
// Waves of a workgroup (512 threads):
//  * waves 0-3, the chain: wave j keeps value columns 16 j .. 16 j + 15 of the state in MFMA
//    accumulators and per chunk runs Delta = U - W H, H <- H + K^T Delta and writes
//    O^T = H^T Q^T + Delta^T P^T (the state before the update, the WY/UT form of
//    recurrence.py:202-216). In the map pass it carries the same columns of M (Delta_M = -W M);
//  * waves 4-7, the producers: producer p forms chunks p, p + 4, ... of the segment. K and V rows
//    go straight into the producer's LDS tiles (buffer_load ... lds, 16-byte segments XOR-swizzled
//    by row); Q (as the chain's B fragments) and the compact UT factor T (written by
//    delta_prep_kernel) into registers, the next chunk's loads issued as soon as the current
//    chunk's tiles have been read. It forms the chunk's operands on MFMA and stages them in one
//    of two LDS slots.
//
// Hand-over by LDS flags, never a workgroup barrier: staged[s] = i once chunk i's operands are in
// slot s = i % 2; consumed[s][j] = i once chain wave j has read them into registers. The producer
// of chunk i fills slot s after every chain wave has read chunk i - 2 from it; a chain wave runs
// chunk i once it is staged. Every wait is on an earlier step of the other side, so all end; each
// poll loop is bounded (a wait that gives up records the fault and the workgroup writes NaN).
// Ordering rests on the LDS performing one wave's DS instructions in issue order, as in
// delta_chain_bf16_kernel.
//
// Reads past the sequence's end return zeros and stores there are dropped (buffer resources over
// each (b, h)'s rows), so a partial last chunk needs no masking.
// With carried inputs (CARRY, copy-forward), the K and V rows of inactive tokens come from the
// carried tensors: the producer picks each row's source by its token's flag when it issues the
// loads, so the scan equals the one over the merged inputs bit for bit.

constexpr int kSegMaps = 0;
constexpr int kSegOutputs = 1;
constexpr int kSegBlocks = 256;  // workgroups the segment count aims at: one per CU of an MI355X
constexpr int kSegMinChunks = 4;  // shortest segment worth its map pass

struct SegShape {
  int nseg, seglen;
};
// Segments per head: enough for B * H * nseg to reach the CU count, none shorter than four chunks.
inline SegShape seg_shape(int B, int H, int T) {
  const int nc = (T + kChunk - 1) / kChunk;
  const long heads = (long)B * H;
  int s = heads >= kSegBlocks ? 1 : (int)(kSegBlocks / heads);
  s = s < nc / kSegMinChunks ? s : nc / kSegMinChunks;
  if (s < 1) s = 1;
  const int len = (nc + s - 1) / s;
  return SegShape{(nc + len - 1) / len, len};
}
constexpr size_t kSegMapBytes = 2 * 64 * 64 * sizeof(float);  // X and M of one (b, h, segment)

template <int MODE, bool CARRY>
__global__ __launch_bounds__(512) void delta_seg_kernel(const __bf16* __restrict__ q, const __bf16* __restrict__ k,
                                                        const __bf16* __restrict__ v,
                                                        const __bf16* __restrict__ tmat,
                                                        const float* __restrict__ s_in, float* __restrict__ s_out,
                                                        __bf16* __restrict__ o, const uint8_t* __restrict__ active,
                                                        float* __restrict__ maps, float* __restrict__ s0copy, int T,
                                                        int H, int nseg, int seglen,
                                                        __bf16* __restrict__ hrec, unsigned* fault, int wait_limit,
                                                        const __bf16* kc, const __bf16* vc) {
  using E = __bf16;
  constexpr int DK = 64;
  constexpr bool OUT = MODE == kSegOutputs;
  constexpr int NP = 4;     // producer waves
  constexpr int NSL = 2;    // operand slots
  constexpr int KBF = 2;    // 32-wide k blocks over dk
  constexpr int FR = 64 * 8;  // elements of one lane-linear bf16 fragment
  constexpr int KSEG = 8;   // 16-byte segments of a K row

  __shared__ __align__(16) E rK[NP][64 * DK];           // each producer's K rows (segments swizzled)
  __shared__ __align__(16) E rV[NP][64 * DK];           // each producer's V rows
  __shared__ __align__(16) E sW[NSL][8 * FR];           // -W: (token tile ti, dk block kb)
  __shared__ __align__(16) E sKt[NSL][8 * FR];          // K^T: (dk tile m, token block kb)
  __shared__ __align__(16) float sU[NSL][16 * 256];     // U: (value tile n, token tile ti), accumulator order
  __shared__ __align__(16) E sQ[OUT ? NSL : 1][8 * FR];  // Q^T: (query tile J, dk block kb)
  __shared__ __align__(16) E sP[OUT ? NSL : 1][6 * FR];  // P^T: (key block, query tile) pairs
  __shared__ uint64_t sMask[NSL];
  __shared__ int staged[NSL], broken;
  __shared__ __align__(16) int consumed[NSL][4];

  const int nmap = nseg - 1;
  const int per_head = OUT ? nseg : nmap;
  const int sg = blockIdx.x % per_head, bh = blockIdx.x / per_head;
  const int b = bh / H, h = bh - b * H;
  const int nc = (T + kChunk - 1) / kChunk;
  const int c0 = sg * seglen;
  const int L = min(nc, c0 + seglen) - c0;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
  const int lq = l & 15, g = l >> 4;
  const int rstride = H * DK;
  const size_t bh_base = ((size_t)b * T * H + h) * DK;
  const unsigned row_bytes = (unsigned)(rstride * sizeof(E));
  const unsigned head_bytes = (unsigned)(((size_t)(T - 1) * rstride + DK) * sizeof(E));

  auto frag_at = [&](const E* base, int f) { return *reinterpret_cast<const bf16x8*>(base + f * FR + 8 * l); };
  auto put_frag = [&](E* base, int f, const bf16x8& x) { *reinterpret_cast<bf16x8*>(base + f * FR + 8 * l) = x; };

  if (threadIdx.x < NSL) staged[threadIdx.x] = -1;
  if (threadIdx.x < NSL * 4) consumed[threadIdx.x / 4][threadIdx.x % 4] = -1;
  if (threadIdx.x == 0) broken = 0;
  __syncthreads();
  auto await = [&](const int* f, int want) {
    if (!flag_wait<1>(f, want, wait_limit)) {
      record_fault(fault, FAULT_SCAN_CHAIN);
      flag_release(&broken, 1);
    }
  };
  // the four chain waves' flags of a slot, read together (one 16-byte LDS read a poll)
  auto await_all4 = [&](const int* f, int want) {
    for (int spin = 0;; ++spin) {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      typedef int i32x4 __attribute__((ext_vector_type(4)));
      const i32x4 v = *reinterpret_cast<const volatile i32x4*>(f);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (min(min(v[0], v[1]), min(v[2], v[3])) >= want) return;
      if (spin >= wait_limit) {
        record_fault(fault, FAULT_SCAN_CHAIN);
        flag_release(&broken, 1);
        return;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  };

  if (wave < 4) {
    // ---------------------------------------------------------------- the chain, value slice j
    const int j = wave;
    __builtin_amdgcn_s_setprio(2);
    const float* s0 = s_in + (size_t)bh * DK * DK;
    const float* head_maps = maps + (size_t)bh * nmap * (kSegMapBytes / sizeof(float));
    float* head_s0 = s0copy + (size_t)bh * DK * DK;  // this head's copy of S0
    // accumulator tile m of a row-major [64][64] fp32 matrix, columns of slice j
    auto load_tile = [&](const float* mat, int m) {
      f32x4 t;
#pragma unroll
      for (int r = 0; r < 4; ++r) t[r] = mat[(16 * m + 4 * g + r) * DK + 16 * j + lq];
      return t;
    };
    f32x4 hreg[4], mreg[4];
    const bool with_m = !OUT && sg > 0;
    if (sg == 0) {
      // the first segment starts from S0; with later segments, from the copy of S0 that the map
      // pass's first segment takes (the last segment may write the final state over S0)
      const float* start = (OUT && nseg > 1) ? head_s0 : s0;
#pragma unroll
      for (int m = 0; m < 4; ++m) hreg[m] = load_tile(start, m);
      if (!OUT) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r) head_s0[(16 * m + 4 * g + r) * DK + 16 * j + lq] = hreg[m][r];
      }
    } else if (OUT) {
#pragma unroll
      for (int m = 0; m < 4; ++m) hreg[m] = load_tile(head_maps, m);  // X_0 = the state after segment 0
      for (int i = 1; i < sg; ++i) {
        const float* X = head_maps + (size_t)i * (kSegMapBytes / sizeof(float));
        const float* M = X + DK * DK;
        bf16x8 hhi[KBF], hlo[KBF];
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) {
          hhi[kb] = pack_acc(hreg[2 * kb], hreg[2 * kb + 1]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            hlo[kb][r] = (__bf16)(hreg[2 * kb][r] - (float)hhi[kb][r]);
            hlo[kb][4 + r] = (__bf16)(hreg[2 * kb + 1][r] - (float)hhi[kb][4 + r]);
          }
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          f32x4 acc = load_tile(X, m);
#pragma unroll
          for (int kb = 0; kb < KBF; ++kb) {
            // A fragment of M: row 16 m + lq, dk 32 kb + 4 g .. + 3 and 32 kb + 16 + 4 g .. + 3
            const f32x4 lo4 = *reinterpret_cast<const f32x4*>(M + (16 * m + lq) * DK + 32 * kb + 4 * g);
            const f32x4 hi4 = *reinterpret_cast<const f32x4*>(M + (16 * m + lq) * DK + 32 * kb + 16 + 4 * g);
            bf16x8 ahi, alo;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              ahi[r] = (__bf16)lo4[r];
              ahi[4 + r] = (__bf16)hi4[r];
              alo[r] = (__bf16)(lo4[r] - (float)ahi[r]);
              alo[4 + r] = (__bf16)(hi4[r] - (float)ahi[4 + r]);
            }
            acc = mfma_bf16(ahi, hhi[kb], acc);
            acc = mfma_bf16(ahi, hlo[kb], acc);
            acc = mfma_bf16(alo, hhi[kb], acc);
          }
          mreg[m] = acc;  // the folded state, moved to hreg once every tile has read the old one
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) hreg[m] = mreg[m];
      }
    } else {
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          hreg[m][r] = 0.f;
          mreg[m][r] = (16 * m + 4 * g + r == 16 * j + lq) ? 1.f : 0.f;
        }
    }

    const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(o + bh_base, head_bytes);
    for (int i = 0; i < L; ++i) {
      const int s = i % NSL;
      const int c = c0 + i;
      await(&staged[s], i);
      bf16x8 wf[4][KBF], kt[4][KBF];
      f32x4 u[4];
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) wf[ti][kb] = frag_at(sW[s], ti * KBF + kb);
        u[ti] = *reinterpret_cast<const f32x4*>(&sU[s][((j * 4 + ti) * 64 + l) * 4]);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) kt[m][kb] = frag_at(sKt[s], m * KBF + kb);
      bf16x8 qf[4][KBF], pt[6];
      uint64_t mask = ~0ull;
      if constexpr (OUT) {
#pragma unroll
        for (int J = 0; J < 4; ++J)
#pragma unroll
          for (int kb = 0; kb < KBF; ++kb) qf[J][kb] = frag_at(sQ[s], J * KBF + kb);
#pragma unroll
        for (int f = 0; f < 6; ++f) pt[f] = frag_at(sP[s], f);
        mask = sMask[s];
      }
      flag_release(&consumed[s][j], i);  // performed after the reads above: the slot may be refilled

      bf16x8 hb[KBF];
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) hb[kb] = pack_acc(hreg[2 * kb], hreg[2 * kb + 1]);
      if (OUT && hrec != nullptr) {
        // the chunk-start state for the backward, as in delta_chain_bf16_kernel's records
        __bf16* rec = hrec + ((size_t)bh * nc + c) * (DK * DK) + (size_t)j * KBF * FR + 8 * l;
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) *reinterpret_cast<bf16x8*>(rec + kb * FR) = hb[kb];
      }
      f32x4 dt[4];
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        f32x4 acc = u[ti];
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) acc = mfma_bf16(wf[ti][kb], hb[kb], acc);
        dt[ti] = acc;
      }
      const bf16x8 db[KBF] = {pack_acc(dt[0], dt[1]), pack_acc(dt[2], dt[3])};
      if (with_m) {
        bf16x8 mb[KBF];
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) mb[kb] = pack_acc(mreg[2 * kb], mreg[2 * kb + 1]);
        f32x4 dm[4];
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kb = 0; kb < KBF; ++kb) acc = mfma_bf16(wf[ti][kb], mb[kb], acc);
          dm[ti] = acc;
        }
        const bf16x8 dmb[KBF] = {pack_acc(dm[0], dm[1]), pack_acc(dm[2], dm[3])};
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int kb = 0; kb < KBF; ++kb) mreg[m] = mfma_bf16(kt[m][kb], dmb[kb], mreg[m]);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) hreg[m] = mfma_bf16(kt[m][kb], db[kb], hreg[m]);
      if constexpr (OUT) {
        // O^T (value columns of slice j, query tile J) = H^T Q^T + Delta^T P^T
        const bool bad = flag_peek(&broken) != 0;
        const unsigned cb = (unsigned)c * kChunk * row_bytes;
#pragma unroll
        for (int J = 0; J < 4; ++J) {
          const int p0 = J == 0 ? 0 : (J == 1 ? 1 : (J == 2 ? 2 : 4));
          f32x4 acc = mfma_bf16(db[0], pt[p0], zero4());
          if (J >= 2) acc = mfma_bf16(db[1], pt[p0 + 1], acc);
#pragma unroll
          for (int kb = 0; kb < KBF; ++kb) acc = mfma_bf16(hb[kb], qf[J][kb], acc);
          const bool on = ((mask >> (16 * J + lq)) & 1) != 0;
          bf16x4 w4;
#pragma unroll
          for (int r = 0; r < 4; ++r) w4[r] = (__bf16)(bad ? __builtin_nanf("") : (on ? acc[r] : 0.f));
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, w4), ro,
                                                (unsigned)(16 * J + lq) * row_bytes + (unsigned)(16 * j + 4 * g) * 2u,
                                                cb, 0);
        }
      }
    }
    const bool bad = flag_peek(&broken) != 0;
    auto store_tile = [&](float* mat, int m, const f32x4& t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) mat[(16 * m + 4 * g + r) * DK + 16 * j + lq] = bad ? __builtin_nanf("") : t[r];
    };
    if constexpr (OUT) {
      if (sg == nseg - 1) {
#pragma unroll
        for (int m = 0; m < 4; ++m) store_tile(s_out + (size_t)bh * DK * DK, m, hreg[m]);
      }
    } else {
      float* X = maps + ((size_t)bh * nmap + sg) * (kSegMapBytes / sizeof(float));
#pragma unroll
      for (int m = 0; m < 4; ++m) store_tile(X, m, hreg[m]);
      if (with_m) {
#pragma unroll
        for (int m = 0; m < 4; ++m) store_tile(X + DK * DK, m, mreg[m]);
      }
    }
    return;
  }

  // ------------------------------------------------------------------ producers
  const int p = wave - 4;
  E* myK = rK[p];
  E* myV = rV[p];
  const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(q + bh_base, head_bytes), rk = buffer_rsrc(k + bh_base, head_bytes);
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(v + bh_base, head_bytes);
  const __amdgpu_buffer_rsrc_t rt = buffer_rsrc(tmat + (size_t)bh * nc * kChunkT, (unsigned)(nc * kChunkT * 2));
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(active != nullptr ? active + (size_t)b * T : active, (unsigned)T);
  // K and V rows: 8 rows a wave instruction, lane l on row l / 8, physical segment l % 8 holding
  // the row's segment (l % 8) ^ kswz(row)
  auto kswz = [](int row) { return (((row >> 1) & 3) << 1) | ((row >> 3) & 1); };
  const unsigned off_k0 = (unsigned)(l / KSEG) * row_bytes + 16u * (unsigned)((l % KSEG) ^ kswz(l / KSEG));
  const unsigned off_k1 = (unsigned)(l / KSEG) * row_bytes + 16u * (unsigned)((l % KSEG) ^ kswz(8 + l / KSEG));
  const unsigned off_q = (unsigned)lq * row_bytes + 8u * g;  // Q row lq, features 4 g .. 4 g + 3
  const unsigned off_t = (unsigned)(lq * 16 + 4 * g) * 2u;
  auto kat = [&](int row, int col) { return row * DK + (((col >> 3) ^ kswz(row)) << 3) + (col & 7); };
  auto tr_read = [&](const E* tile, int r0, int m) {  // column 16 m + lq of rows r0 + 4 g .. + 3
    return read_tr16<bf16x4>(&tile[kat(r0 + 4 * g + (lq >> 2), 16 * m + 4 * (lq & 3))]);
  };

  bf16x8 qf[4][KBF];
  bf16x4 tl[kTiles];
  uint8_t act = 1;
  for (int i = l; i < 64 * DK / 8; i += 64) {
    *reinterpret_cast<bf16x8*>(&myK[8 * i]) = bf16x8{};
    *reinterpret_cast<bf16x8*>(&myV[8 * i]) = bf16x8{};
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zeros land before any direct load
  // the rows of chunk c: K and V into the producer's tiles, Q's B fragments and T into registers
  auto issue_tiles = [&](int c, uint64_t flags) {
    const unsigned cb = (unsigned)c * kChunk * row_bytes;
    if (!CARRY || flags == ~0ull) {
#pragma unroll
      for (int jj = 0; jj < KSEG; ++jj) {
        buffer_load_lds16(rk, &myK[512 * jj], (jj & 1) ? off_k1 : off_k0, cb + (unsigned)jj * 8 * row_bytes);
        buffer_load_lds16(rv, &myV[512 * jj], (jj & 1) ? off_k1 : off_k0, cb + (unsigned)jj * 8 * row_bytes);
      }
    } else {
      // copy-forward: each row from the fresh or the carried tensor by a per-lane address (bit r of
      // `flags`: token r of the chunk is active). Rows past the end re-read row T - 1 from that
      // token's own source: their T rows and columns are zero, so they add nothing.
      const char* kf = reinterpret_cast<const char*>(k + bh_base);
      const char* kh = reinterpret_cast<const char*>(kc + bh_base);
      const char* vf = reinterpret_cast<const char*>(v + bh_base);
      const char* vh = reinterpret_cast<const char*>(vc + bh_base);
#pragma unroll
      for (int jj = 0; jj < KSEG; ++jj) {
        const int t = min(c * kChunk + 8 * jj + l / KSEG, T - 1);
        const size_t at = (size_t)t * row_bytes + (((jj & 1) ? off_k1 : off_k0) - (unsigned)(l / KSEG) * row_bytes);
        const bool fresh = ((flags >> (t - c * kChunk)) & 1) != 0;
        load_lds16((fresh ? kf : kh) + at, &myK[512 * jj]);
        load_lds16((fresh ? vf : vh) + at, &myV[512 * jj]);
      }
    }
  };
  auto issue_regs = [&](int c) {
    const unsigned cb = (unsigned)c * kChunk * row_bytes;
    if constexpr (OUT) {
#pragma unroll
      for (int J = 0; J < 4; ++J)
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) {
          const unsigned so = cb + 16u * J * row_bytes;
          const bf16x4 lo = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(rq, off_q + 64u * kb, so, 0));
          const bf16x4 hi = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(rq, off_q + 64u * kb + 32u, so, 0));
          qf[J][kb] = join4(lo, hi);
        }
      if (!CARRY && active != nullptr) act = __builtin_amdgcn_raw_buffer_load_b8(ra, (unsigned)l, (unsigned)c * kChunk, 0);
    }
    const unsigned tb = (unsigned)c * kChunkT * 2u;
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
      tl[t] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(rt, off_t + 512u * t, tb, 0));
  };

  // with carried inputs, the flags of a chunk choose its rows' sources: they are loaded when the
  // producer starts its previous chunk, and kept as a wave-uniform mask
  uint64_t next_flags = ~0ull;
  uint8_t act_next = 1;
  if (p < L) {
    if constexpr (CARRY)
      next_flags = __builtin_amdgcn_ballot_w64(__builtin_amdgcn_raw_buffer_load_b8(ra, (unsigned)l, (unsigned)(c0 + p) * kChunk, 0) != 0);
    issue_tiles(c0 + p, next_flags);
    issue_regs(c0 + p);
  }
  for (int i = p; i < L; i += NP) {
    const int c = c0 + i;
    const int s = i % NSL;
    const uint64_t flags = next_flags;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this chunk's tiles and registers have arrived
    wave_sync();
    if constexpr (CARRY) {
      if (i + NP < L) act_next = __builtin_amdgcn_raw_buffer_load_b8(ra, (unsigned)l, (unsigned)(c + NP) * kChunk, 0);
    }
    // token-major fragments: ktf[m][kb] = column 16 m + lq of K rows 32 kb + 4 g (+16); V's likewise
    // once the slot is free
    bf16x8 ktf[4][KBF];
#pragma unroll
    for (int kb = 0; kb < KBF; ++kb)
#pragma unroll
      for (int m = 0; m < 4; ++m) ktf[m][kb] = join4(tr_read(myK, 32 * kb, m), tr_read(myK, 32 * kb + 16, m));
    // K row fragments in the chain's dk order (32 kb + 4 g .. + 3, then + 16)
    bf16x8 kr[4][KBF];
    if constexpr (OUT) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb)
          kr[jj][kb] = join4(*reinterpret_cast<const bf16x4*>(&myK[kat(16 * jj + lq, 32 * kb + 4 * g)]),
                             *reinterpret_cast<const bf16x4*>(&myK[kat(16 * jj + lq, 32 * kb + 16 + 4 * g)]));
    }
    uint64_t mask = ~0ull;
    bf16x8 pt[6];
    if constexpr (OUT) {
      const int nvc = min(kChunk, T - c * kChunk);
      mask = CARRY ? (flags & __builtin_amdgcn_ballot_w64(l < nvc))
                   : __builtin_amdgcn_ballot_w64(l < nvc && (active == nullptr || act != 0));
      auto ptile = [&](int jj, int ii) {
        f32x4 acc = zero4();
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) acc = mfma_bf16(kr[jj][kb], qf[ii][kb], acc);
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
    }
    // T's fragments (row tile, token block): (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
    const bf16x4 z4{};
    const bf16x8 tf[6] = {join4(tl[0], z4), join4(tl[1], tl[2]), join4(tl[3], tl[4]),
                          join4(tl[5], z4), join4(tl[6], tl[7]), join4(tl[8], tl[9])};
    // -W (the pairs over dk of W^T = K^T T^T, token tile ti) into registers first, so that once the
    // slot is free only U = T V and the stores remain
    bf16x8 wneg[4][KBF];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int f0 = ti == 0 ? 0 : (ti == 1 ? 1 : (ti == 2 ? 2 : 4));
      f32x4 wt[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        wt[m] = mfma_bf16(ktf[m][0], tf[f0], zero4());
        if (ti >= 2) wt[m] = mfma_bf16(ktf[m][1], tf[f0 + 1], wt[m]);
      }
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) wneg[ti][kb] = pack_acc(wt[2 * kb], wt[2 * kb + 1], -1.f);
    }
    // every chain wave has read chunk i - 2 from this slot
    await_all4(consumed[s], i - NSL);
    bf16x8 vtf[4][KBF];
#pragma unroll
    for (int kb = 0; kb < KBF; ++kb)
#pragma unroll
      for (int n = 0; n < 4; ++n) vtf[n][kb] = join4(tr_read(myV, 32 * kb, n), tr_read(myV, 32 * kb + 16, n));
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int f0 = ti == 0 ? 0 : (ti == 1 ? 1 : (ti == 2 ? 2 : 4));
      // U = T V (token tile ti, value tile n), in the accumulator order of Delta
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        f32x4 u = mfma_bf16(tf[f0], vtf[n][0], zero4());
        if (ti >= 2) u = mfma_bf16(tf[f0 + 1], vtf[n][1], u);
        *reinterpret_cast<f32x4*>(&sU[s][((n * 4 + ti) * 64 + l) * 4]) = u;
      }
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) put_frag(sW[s], ti * KBF + kb, wneg[ti][kb]);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb) put_frag(sKt[s], m * KBF + kb, ktf[m][kb]);
    if constexpr (OUT) {
#pragma unroll
      for (int J = 0; J < 4; ++J)
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb) put_frag(sQ[s], J * KBF + kb, qf[J][kb]);
#pragma unroll
      for (int f = 0; f < 6; ++f) put_frag(sP[s], f, pt[f]);
      if (l == 0) sMask[s] = mask;
    }
    flag_release(&staged[s], i);
    // the tiles have been read: the producer's next chunk may be loaded over them, and its Q and T
    // into the registers, free once staged
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (i + NP < L) {
      if constexpr (CARRY) next_flags = __builtin_amdgcn_ballot_w64(act_next != 0);
      issue_tiles(c + NP, next_flags);
      issue_regs(c + NP);
    }
  }
}
