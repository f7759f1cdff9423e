// The looped column's decode-step projections on CDNA4 (gfx950): residual add, RMSNorm and the
// small-batch product in one launch.
//
// Reference: each sublayer projects the RMS-normalized residual stream (vesper/column.py:146-188
// for the norm, :192-260 and vesper/attention.py:269-292 for the projections); the looped column
// stacks a sublayer's projections into one [p, d, h*dk] weight per pass. In a decode step the
// product has only M = batch rows, so a library GEMM tiles it into a few dozen 64x64 workgroups
// and the norm and the residual add run as launches of their own. Here one launch does all three:
//
//   s = x + r (float32; r in bf16 is the previous mixer's output, or absent)   -> sum_out
//   z = RMSNorm(s) in bf16, the arithmetic of vsp_rms_norm_bf16 (bitwise the same z)
//   y_j = z W_j for each block j of the stacked weight, only its first used_j columns
//
// Workgroup = 16 rows x 32 output columns of one block: eight waves each normalize two of the
// rows (one wave a row, as the norm kernel) into LDS, then each wave forms the 16x32 tile over
// every eighth 32-wide step of the d inputs (16x16x32 bf16 MFMA, the transposed weight
// [p, h*dk, d] giving the A fragments as 16-byte loads issued before the norm), and the eight
// partial tiles are summed in a fixed order through LDS. A block whose used width is narrow (the
// write strength's h columns) takes one column group. One block may have its outputs passed
// through the logistic function (the write strength, rounded to bf16 first as the separate
// sigmoid would see it), and blocks may be rotated as they are stored (the attention's q and k:
// a thread stores two adjacent columns of one token, a rotary pair, turned by the rotary kernel's
// own arithmetic, so the result is bitwise the separate launch's; its float64 cos and sin are
// formed while the loads are in flight). The launch is a chain of latencies (timestamps per phase
// in a timing copy, four waves: the loads 43 %, the norm of four rows a wave 36 %, the products
// 10 %, the float64 cos and sin a further 13 % on the attention's launch): eight waves halve the
// norm's rows a wave.
#include "common.h"
#include "rotary_math.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr float kProjRmsEps = 1e-6f;         // column.py:55
constexpr float kProjRmsScaleFloor = 1e-3f;  // column.py:56
constexpr int kMaxBlocks = 4;
constexpr int kProjWaves = 8;                   // waves a workgroup
constexpr int kProjRowsPerWave = 16 / kProjWaves;  // rows of the norm a wave takes

struct ProjBlocks {
  int nblk;
  int used[kMaxBlocks];           // columns written per block
  int start[kMaxBlocks + 1];      // first column group (workgroup along x) of each block
  __bf16* out[kMaxBlocks];        // [M, used] per block
};

template <int NSEG>
__global__ __launch_bounds__(64 * kProjWaves) void decode_proj_kernel(const float* __restrict__ x, const __bf16* __restrict__ res,
                                                          float* __restrict__ sum_out, const float* __restrict__ gain,
                                                          const __bf16* __restrict__ wt, int M, int d, int cols,
                                                          ProjBlocks blk, int sig_block,
                                                          const int64_t* __restrict__ pos,
                                                          const double* __restrict__ inv_freq, int rot_mask,
                                                          int rot_dk) {
  constexpr int PITCH = 512 * NSEG + 16;  // bf16 elements a row of z: rows 8 banks apart
  constexpr int KSMAX = 16 * NSEG / kProjWaves;  // k steps of 32 a wave takes, at most
  __shared__ __align__(16) __bf16 sz[16][PITCH];
  __shared__ f32x4 part[kProjWaves][2][64];

  const int gid = blockIdx.x, mb = blockIdx.y;
  int nb = 0;
#pragma unroll
  for (int j = 1; j < kMaxBlocks; ++j)
    if (j < blk.nblk && gid >= blk.start[j]) nb = j;
  const int c0 = (gid - blk.start[nb]) * 32;  // first output column of this workgroup in block nb
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  const int ksteps = d / 32;  // wave w takes the steps w, w + 8, w + 16, ...

  // the weight fragments first (they do not depend on x): A[n][k] = W_nb[k][c0 + 16 j + n] from the
  // transposed weight; columns past the block's width re-read its last row (never stored)
  bf16x8 af[2][KSMAX];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = min(c0 + 16 * j + lq, cols - 1);
    const __bf16* wr = wt + ((size_t)nb * cols + n) * d + 8 * g;
#pragma unroll
    for (int i = 0; i < KSMAX; ++i)
      if (w + kProjWaves * i < ksteps) af[j][i] = *reinterpret_cast<const bf16x8*>(wr + 32 * (w + kProjWaves * i));
  }

  // The store's thread: thread t < 256 stores two adjacent columns of one row (tile j = t / 128,
  // lane ln = (t % 128) / 2: row lq, columns 4 g .. 4 g + 3; pair p = t % 2). A rotated block's cos
  // and sin for that pair are formed now, while the loads are in flight.
  const int t = threadIdx.x, j = (t >> 7) & 1, ln = (t & 127) >> 1, p = t & 1;
  const int m = mb * 16 + (ln & 15);
  const int col = c0 + 16 * j + 4 * (ln >> 4) + 2 * p;
  const int used = blk.used[nb];
  const bool rot = (rot_mask >> nb) & 1;
  __bf16 rc = (__bf16)0.f, rs = (__bf16)0.f;
  if (rot && t < 256 && m < M && col < used) {  // columns col, col + 1: pair (col % dk) / 2 of a head
    const double angle = (double)pos[m] * inv_freq[(col % rot_dk) >> 1];
    rc = rot_from_f64<__bf16>(cos(angle));
    rs = rot_from_f64<__bf16>(sin(angle));
  }

  // the norm: wave w takes rows 2w, 2w + 1 of the 16 (one wave a row, lane segments 8 (lane + 64 j));
  // every row's loads are issued before the first row's reductions
  constexpr int RA = NSEG <= 2 ? kProjRowsPerWave : 1;  // rows whose loads are in flight together
  for (int i0 = 0; i0 < kProjRowsPerWave; i0 += RA) {
    float e[RA][NSEG][8];
#pragma unroll
    for (int ii = 0; ii < RA; ++ii) {
      const int m = mb * 16 + kProjRowsPerWave * w + i0 + ii;
      const size_t ro = (size_t)min(m, M - 1) * d;  // rows past M read row M - 1 (never used)
#pragma unroll
      for (int j = 0; j < NSEG; ++j) {
        const int f = 8 * (l + 64 * j);
        const int fs = f < d ? f : 0;
        const float4 a = reinterpret_cast<const float4*>(x + ro + fs)[0];
        const float4 b = reinterpret_cast<const float4*>(x + ro + fs)[1];
        e[ii][j][0] = a.x; e[ii][j][1] = a.y; e[ii][j][2] = a.z; e[ii][j][3] = a.w;
        e[ii][j][4] = b.x; e[ii][j][5] = b.y; e[ii][j][6] = b.z; e[ii][j][7] = b.w;
        if (res != nullptr) {
          const bf16x8 rv = *reinterpret_cast<const bf16x8*>(res + ro + fs);
#pragma unroll
          for (int k = 0; k < 8; ++k) e[ii][j][k] += (float)rv[k];
        }
      }
    }
#pragma unroll
    for (int ii = 0; ii < RA; ++ii) {
      const int rl = kProjRowsPerWave * w + i0 + ii, m = mb * 16 + rl;
      if (m >= M) {
#pragma unroll
        for (int j = 0; j < NSEG; ++j) {
          const int f = 8 * (l + 64 * j);
          if (f < d) *reinterpret_cast<bf16x8*>(&sz[rl][f]) = bf16x8{};
        }
        continue;
      }
      float v[NSEG][8];
      float peak = 0.f;
#pragma unroll
      for (int j = 0; j < NSEG; ++j) {
        const int f = 8 * (l + 64 * j);
        const bool ok = f < d;
        if (ok && sum_out != nullptr && gid == 0) {
          float* so = sum_out + (size_t)m * d + f;
          reinterpret_cast<float4*>(so)[0] = make_float4(e[ii][j][0], e[ii][j][1], e[ii][j][2], e[ii][j][3]);
          reinterpret_cast<float4*>(so)[1] = make_float4(e[ii][j][4], e[ii][j][5], e[ii][j][6], e[ii][j][7]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          v[j][k] = ok ? e[ii][j][k] : 0.f;
          peak = __builtin_fmaxf(peak, fabsf(v[j][k]));
        }
      }
      const float scale = __builtin_fmaxf(group_max<64>(peak), kProjRmsScaleFloor);
      const float inv_scale = __builtin_amdgcn_rcpf(scale);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < NSEG; ++j)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float s0 = v[j][k] * inv_scale;
          v[j][k] = __builtin_fmaf(__builtin_fmaf(-s0, scale, v[j][k]), inv_scale, s0);
          ss += v[j][k] * v[j][k];
        }
      const float mean = group_sum<64>(ss) / (float)d;
      const float inv_rms = 1.f / __builtin_sqrtf(mean + kProjRmsEps / (scale * scale));
#pragma unroll
      for (int j = 0; j < NSEG; ++j) {
        const int f = 8 * (l + 64 * j);
        if (f >= d) continue;
        bf16x8 o;
        if (gain != nullptr) {
          const float4 ga = reinterpret_cast<const float4*>(gain + f)[0];
          const float4 gb = reinterpret_cast<const float4*>(gain + f)[1];
          const float gg[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
          for (int k = 0; k < 8; ++k) o[k] = (__bf16)(v[j][k] * inv_rms * gg[k]);
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) o[k] = (__bf16)(v[j][k] * inv_rms);
        }
        *reinterpret_cast<bf16x8*>(&sz[rl][f]) = o;
      }
    }
  }
  __syncthreads();

  // y^T tile [32 columns x 16 rows] over this wave's steps of d: A = W^T rows, B = z^T
  f32x4 acc[2] = {zero4(), zero4()};
#pragma unroll
  for (int i = 0; i < KSMAX; ++i) {
    if (w + kProjWaves * i < ksteps) {
      const bf16x8 bz = *reinterpret_cast<const bf16x8*>(&sz[lq][32 * (w + kProjWaves * i) + 8 * g]);
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[j][i], bz, acc[j], 0, 0, 0);
    }
  }
  part[w][0][l] = acc[0];
  part[w][1][l] = acc[1];
  __syncthreads();

  // the waves' partial tiles summed in a fixed order by the store's threads
  if (t < 256 && m < M && col < used) {
    float y0 = 0.f, y1 = 0.f;
#pragma unroll
    for (int q = 0; q < kProjWaves; ++q) {
      y0 += part[q][j][ln][2 * p];
      y1 += part[q][j][ln][2 * p + 1];
    }
    __bf16 b0 = (__bf16)y0, b1 = (__bf16)y1;
    if (nb == sig_block) {
      b0 = (__bf16)(1.f / (1.f + expf(-(float)b0)));
      b1 = (__bf16)(1.f / (1.f + expf(-(float)b1)));
    }
    if (rot) rot_pair<__bf16>(b0, b1, rc, rs, b0, b1);
    __bf16* orow = blk.out[nb] + (size_t)m * used;
    orow[col] = b0;
    if (col + 1 < used) orow[col + 1] = b1;
  }
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_decode_proj_bf16(const float* x, const void* residual, float* sum_out, const float* gain,
                                    const void* weights_t, int nblk, int cols, int d, int M, int used0, int used1,
                                    int used2, int used3, void* out0, void* out1, void* out2, void* out3,
                                    int sigmoid_block, const int64_t* positions, const double* inv_freq,
                                    int rotate_mask, int rotary_dk, void* stream) {
  using namespace vsp;
  const char* who = "vsp_decode_proj_bf16";
  if (nblk < 1 || nblk > kMaxBlocks) return fail(ERR_ARG, "%s: %d weight blocks (1..%d)", who, nblk, kMaxBlocks);
  if (d < 32 || d > 2048 || d % 32 != 0) return fail(ERR_ARG, "%s: width %d (a multiple of 32 in 32..2048)", who, d);
  if (M < 0 || cols < 1) return fail(ERR_ARG, "%s: bad sizes M=%d cols=%d", who, M, cols);
  if (sigmoid_block < -1 || sigmoid_block >= nblk) return fail(ERR_ARG, "%s: sigmoid block %d", who, sigmoid_block);
  if (rotate_mask < 0 || rotate_mask >= (1 << nblk)) return fail(ERR_ARG, "%s: rotate mask %d", who, rotate_mask);
  if (rotate_mask != 0) {
    if (!positions || !inv_freq) return fail(ERR_ARG, "%s: rotation without positions or frequencies", who);
    if (rotary_dk < 2 || rotary_dk % 2 != 0) return fail(ERR_ARG, "%s: rotary head width %d", who, rotary_dk);
    if (sigmoid_block >= 0 && ((rotate_mask >> sigmoid_block) & 1))
      return fail(ERR_ARG, "%s: block %d both rotated and passed through the logistic", who, sigmoid_block);
  }
  const int used_in[kMaxBlocks] = {used0, used1, used2, used3};
  void* out_in[kMaxBlocks] = {out0, out1, out2, out3};
  ProjBlocks blk{};
  blk.nblk = nblk;
  int groups = 0;
  for (int j = 0; j < kMaxBlocks; ++j) {
    blk.start[j] = groups;
    if (j >= nblk) continue;
    if (used_in[j] < 1 || used_in[j] > cols)
      return fail(ERR_ARG, "%s: block %d uses %d of its %d columns", who, j, used_in[j], cols);
    if (out_in[j] == nullptr) return fail(ERR_ARG, "%s: null output for block %d", who, j);
    if (reinterpret_cast<uintptr_t>(out_in[j]) & 3) return fail(ERR_ARG, "%s: output %d must be 4-byte aligned", who, j);
    if (((rotate_mask >> j) & 1) && used_in[j] % rotary_dk != 0)
      return fail(ERR_ARG, "%s: rotated block %d's %d columns are not whole heads of %d", who, j, used_in[j], rotary_dk);
    blk.used[j] = used_in[j];
    blk.out[j] = static_cast<__bf16*>(out_in[j]);
    groups += (used_in[j] + 31) / 32;
  }
  blk.start[kMaxBlocks] = groups;
  if (M == 0) return OK;
  if (!x || !weights_t) return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(sum_out) |
       reinterpret_cast<uintptr_t>(gain) | reinterpret_cast<uintptr_t>(weights_t)) & 15)
    return fail(ERR_ARG, "%s: x, residual, sum_out, gain and the weights must be 16-byte aligned", who);
  const dim3 grid((unsigned)groups, (unsigned)((M + 15) / 16));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const __bf16* r = static_cast<const __bf16*>(residual);
  const __bf16* w = static_cast<const __bf16*>(weights_t);
  if (d <= 512)
    hipLaunchKernelGGL(decode_proj_kernel<1>, grid, dim3(64 * kProjWaves), 0, s, x, r, sum_out, gain, w, M, d, cols, blk, sigmoid_block,
                       positions, inv_freq, rotate_mask, rotary_dk);
  else if (d <= 1024)
    hipLaunchKernelGGL(decode_proj_kernel<2>, grid, dim3(64 * kProjWaves), 0, s, x, r, sum_out, gain, w, M, d, cols, blk, sigmoid_block,
                       positions, inv_freq, rotate_mask, rotary_dk);
  else
    hipLaunchKernelGGL(decode_proj_kernel<4>, grid, dim3(64 * kProjWaves), 0, s, x, r, sum_out, gain, w, M, d, cols, blk, sigmoid_block,
                       positions, inv_freq, rotate_mask, rotary_dk);
  return check_launch(who);
}
