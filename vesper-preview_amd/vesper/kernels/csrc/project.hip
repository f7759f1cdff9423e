// The looped column's prefill projections on CDNA4 (gfx950): every block of a pass's stacked weight
// in one launch.
//
// Reference: each sublayer projects its normalized input (vesper/column.py:192-260 for the recurrent
// q, z, v and the write strength, vesper/attention.py:269-292 for the attention's q, k, v); the looped
// column stacks a sublayer's projections into one weight per pass. A library GEMM over the
// zero-padded stack computes every padded column (the write strength's h columns padded to h*dk, the
// grouped keys and values to h*dk) and writes [p, M, cols]; here each block is computed over the
// columns it uses only, written as its own [M, used] tensor, and the write strength's block may pass
// through the logistic function as it is stored.
//
// y_j = z W_j with z [M, d] bf16 and the weights transposed and stacked, W^T [p, cols, d] (d
// contiguous). Workgroup = 256 rows (tokens) x 256 columns of one block, eight waves of 64 rows x 128
// columns, one workgroup a CU. Both operands go through LDS in stages of 64 inputs, double-buffered:
// global_load_lds_dwordx4 moves 8 rows of 128 bytes (whole cache lines) an instruction, and each
// row's 16-byte segments are XOR-swizzled by row so that the fragment reads meet each bank once.
// The product is formed transposed, y^T = W^T z^T (16x16x32 bf16 MFMA, the weight rows as the A
// operand: each weight fragment read feeds four MFMAs, each z fragment eight). The outputs go back
// through LDS so that they leave as whole rows (16-byte pieces, 256 bytes a row). Workgroups are
// numbered so that an XCD takes whole row tiles with all their column tiles: z comes from HBM once.
//
// Measured at the looped column's shape (M 8192, d 512, 512-column blocks; kernel alone, µs): the
// recurrent sublayer's q, z, v and 8-column write strength 21.9 (the library GEMM over the padded
// stack 25.5), the attention's q, k, v 20.9 (30.0). A stage's LDS traffic (the eight waves'
// fragment reads, 192 KiB, and the 64 KiB of direct loads) takes as many cycles at 128 bytes a
// clock as its MFMAs (2048), so the products run at half the MFMA peak at best; with the stores
// taken out (a timing copy, before the outputs went through LDS) the kernel took 16.1 of 24.8 µs.
#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kPrjMaxBlocks = 4;
constexpr int kPrjBM = 256;  // rows (tokens) a workgroup
constexpr int kPrjBN = 256;  // output columns a workgroup
constexpr int kPrjBK = 64;   // inputs a stage

struct PrjBlocks {
  int nblk;
  int used[kPrjMaxBlocks];       // columns written per block
  int start[kPrjMaxBlocks + 1];  // first column tile of each block
  __bf16* out[kPrjMaxBlocks];    // [M, used] per block
};

__global__ __launch_bounds__(512, 1) void project_kernel(const __bf16* __restrict__ z, const __bf16* __restrict__ wt,
                                                         int M, int d, int cols, PrjBlocks blk, int ctiles, int mtiles,
                                                         int sig_block) {
  // Two stages of the z rows and the weight rows, [256 rows][64 inputs] each: row r's 16-byte
  // segment s at s ^ 2 ((r >> 1) & 3), so that a fragment read (lanes 0-7 with 16-23: rows 0-7, two
  // segments each) meets every bank once. Separate variables: each stage's buffers are fixed at
  // compile time, and the compiler tells the direct loads into one from the reads of the other.
  __shared__ __align__(16) __bf16 sZ0[kPrjBM * kPrjBK], sZ1[kPrjBM * kPrjBK];
  __shared__ __align__(16) __bf16 sW0[kPrjBN * kPrjBK], sW1[kPrjBN * kPrjBK];

  const int lg = xcd_logical_block(blockIdx.x, gridDim.x);
  const int mt = lg / ctiles, ct = lg - mt * ctiles;
  if (mt >= mtiles) return;  // the grid is padded to whole XCD rounds; whole workgroups leave
  int nb = 0;
#pragma unroll
  for (int j = 1; j < kPrjMaxBlocks; ++j)
    if (j < blk.nblk && ct >= blk.start[j]) nb = j;
  const int c0 = (ct - blk.start[nb]) * kPrjBN;  // first output column of the tile in block nb
  const int used = blk.used[nb];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, lq = l & 15, g = l >> 4;
  const int wm = w & 3, wn = w >> 2;  // the wave's rows 64 wm .. + 63 and columns 128 wn .. + 127
  const bool live = c0 + 128 * wn < used;  // a wave whose columns are all unused forms no products
  const int stages = d / kPrjBK;

  // Buffer resources: weight rows past the block's `cols` and z rows past M read zeros.
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wt + (size_t)nb * cols * d, (unsigned)((size_t)cols * d * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(z, (unsigned)((size_t)M * d * 2));
  auto kswz = [](int row) { return 2 * ((row >> 1) & 3); };
  // direct loads: instruction j of wave w fills rows 8 (w + 8 j) .. + 7 of a stage, 128 bytes each
  // (whole cache lines); lane l brings row l / 8's logical segment (l % 8) ^ kswz(row), whose row
  // bits 1-2 are those of l / 8
  const int lrow = l >> 3, lseg = (l & 7) ^ kswz(lrow);
  const unsigned zoff = ((unsigned)(mt * kPrjBM + 8 * w + lrow) * (unsigned)d + 8u * (unsigned)lseg) * 2u;
  const unsigned woff = ((unsigned)(c0 + 8 * w + lrow) * (unsigned)d + 8u * (unsigned)lseg) * 2u;
  auto issue = [&](int st, __bf16* dz, __bf16* dw) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned so = ((unsigned)(64 * j) * (unsigned)d + (unsigned)(st * kPrjBK)) * 2u;
      buffer_load_lds16(rz, dz + (w + 8 * j) * 512, zoff, so);
      buffer_load_lds16(rw, dw + (w + 8 * j) * 512, woff, so);
    }
  };

  // acc[j][i]: y^T tile of the wave's output columns 16 j .. and rows 16 i ..; lane (lq, g) holds
  // columns 16 j + 4 g + r of row 16 i + lq
  f32x4 acc[8][4];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = zero4();
  auto compute = [&](const __bf16* sz, const __bf16* sw) {
    if (!live) return;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8 zf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 64 * wm + 16 * i + lq;
        zf[i] = *reinterpret_cast<const bf16x8*>(sz + row * kPrjBK + 8 * ((4 * s + g) ^ kswz(row)));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int row = 128 * wn + 16 * j + lq;
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(sw + row * kPrjBK + 8 * ((4 * s + g) ^ kswz(row)));
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, zf[i], acc[j][i], 0, 0, 0);
      }
    }
  };

  // Two stages an iteration. A stage's direct loads are issued before the previous stage's
  // products; the wait for them (vmcnt 0) and the barrier follow those products.
  issue(0, sZ0, sW0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  for (int st = 0; st < stages; st += 2) {
    if (st + 1 < stages) issue(st + 1, sZ1, sW1);
    compute(sZ0, sW0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (st + 1 < stages) {
      if (st + 2 < stages) issue(st + 2, sZ0, sW0);
      compute(sZ1, sW1);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
    }
  }
  if (!live) return;

  // The outputs through LDS (free once the last stage's barrier has passed): the wave's 64 x 128
  // tile in bf16 (row r's 16-byte segment s at s ^ (r & 15)), then written as whole rows, 16 lanes a
  // row and four rows a store instruction. The logistic function is applied to the stored columns
  // of the write strength's block only.
  __bf16* stile = (w >> 1) == 0 ? sZ0 : (w >> 1) == 1 ? sZ1 : (w >> 1) == 2 ? sW0 : sW1;
  stile += (w & 1) * 64 * 128;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * i + lq, c = 16 * j + 4 * g;  // tile column c: segment c / 8, half c % 8
      const bool sig = nb == sig_block && c0 + 128 * wn + c < used;
      bf16x4 y;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        __bf16 b = (__bf16)acc[j][i][r];
        if (sig) b = (__bf16)(1.f / (1.f + expf(-(float)b)));
        y[r] = b;
      }
      *reinterpret_cast<bf16x4*>(stile + row * 128 + 8 * ((c >> 3) ^ (row & 15)) + (c & 7)) = y;
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the tile is in LDS (only this wave reads it)
  __bf16* out = blk.out[nb];
  const int m0 = mt * kPrjBM + 64 * wm;
  const int seg = l & 15, col = c0 + 128 * wn + 8 * seg;
  const bool whole = (used & 7) == 0;  // rows of whole 16-byte pieces (the outputs are 16-byte aligned)
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int row = 4 * it + (l >> 4);
    const int m = m0 + row;
    if (m >= M || col >= used) continue;
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(stile + row * 128 + 8 * (seg ^ (row & 15)));
    __bf16* orow = out + (size_t)m * used + col;
    if (whole) {
      *reinterpret_cast<bf16x8*>(orow) = v;
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r)
        if (col + r < used) orow[r] = v[r];
    }
  }
}

}  // namespace
}  // namespace vsp

extern "C" int vsp_project_bf16(const void* z, const void* weights_t, int nblk, int cols, int d, int M, int used0,
                                int used1, int used2, int used3, void* out0, void* out1, void* out2, void* out3,
                                int sigmoid_block, void* stream) {
  using namespace vsp;
  const char* who = "vsp_project_bf16";
  if (nblk < 1 || nblk > kPrjMaxBlocks) return fail(ERR_ARG, "%s: %d weight blocks (1..%d)", who, nblk, kPrjMaxBlocks);
  if (d < kPrjBK || d > 16384 || d % kPrjBK != 0)
    return fail(ERR_ARG, "%s: width %d (a multiple of %d in %d..16384)", who, d, kPrjBK, kPrjBK);
  if (M < 0 || cols < 1) return fail(ERR_ARG, "%s: bad sizes M=%d cols=%d", who, M, cols);
  if (sigmoid_block < -1 || sigmoid_block >= nblk) return fail(ERR_ARG, "%s: sigmoid block %d", who, sigmoid_block);
  // 32-bit buffer offsets: z and each block's weights under 4 GiB
  if (((size_t)M + kPrjBM) * d * 2 >= ((size_t)1 << 32) || ((size_t)cols + kPrjBN) * d * 2 >= ((size_t)1 << 32))
    return fail(ERR_ARG, "%s: operands over 4 GiB (M=%d cols=%d d=%d)", who, M, cols, d);
  const int used_in[kPrjMaxBlocks] = {used0, used1, used2, used3};
  void* out_in[kPrjMaxBlocks] = {out0, out1, out2, out3};
  PrjBlocks blk{};
  blk.nblk = nblk;
  int tiles = 0;
  for (int j = 0; j < kPrjMaxBlocks; ++j) {
    blk.start[j] = tiles;
    if (j >= nblk) continue;
    if (used_in[j] < 1 || used_in[j] > cols)
      return fail(ERR_ARG, "%s: block %d uses %d of its %d columns", who, j, used_in[j], cols);
    if (M > 0 && out_in[j] == nullptr) return fail(ERR_ARG, "%s: null output for block %d", who, j);
    if (reinterpret_cast<uintptr_t>(out_in[j]) & 15) return fail(ERR_ARG, "%s: output %d must be 16-byte aligned", who, j);
    blk.used[j] = used_in[j];
    blk.out[j] = static_cast<__bf16*>(out_in[j]);
    tiles += (used_in[j] + kPrjBN - 1) / kPrjBN;
  }
  blk.start[kPrjMaxBlocks] = tiles;
  if (M == 0) return OK;
  if (!z || !weights_t) return fail(ERR_ARG, "%s: null pointer", who);
  if ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(weights_t)) & 15)
    return fail(ERR_ARG, "%s: z and the weights must be 16-byte aligned", who);
  const int mtiles = (M + kPrjBM - 1) / kPrjBM;
  const long long n = ((long long)tiles * mtiles + 7) / 8 * 8;  // whole rounds over the 8 XCDs
  if (n >= ((long long)1 << 31)) return fail(ERR_ARG, "%s: too many tiles", who);
  hipLaunchKernelGGL(project_kernel, dim3((unsigned)n), dim3(512), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const __bf16*>(z), static_cast<const __bf16*>(weights_t), M, d, cols, blk, tiles,
                     mtiles, sigmoid_block);
  return check_launch(who);
}
