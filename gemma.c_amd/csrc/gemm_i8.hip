// gemm_i8.hip -- prefill / SigLIP int8 GEMM on CDNA4 int8 MFMA
// (gemma.c:3937-4054 gemm_int8 and its tile/flush helpers 3847-3935).
//
//   dst[i][j] = (float)sum_l src[i][l]*mat[j][l] * (ssc[i]*matsc[j])
//
// Both operands are K-contiguous ("NT"), which is the layout MFMA wants: a
// lane feeds 16 consecutive int8 of one row to v_mfma_i32_32x32x32_i8.
// Workgroup: 256 threads = 4 waves in a 2x2 grid, block tile 128x128, K step
// 64 bytes, LDS double-buffered (one barrier per K step; the next step's
// global loads are in registers while the current step's MFMAs run).  Each
// wave owns a 64x64 sub-tile = 2x2 MFMA tiles of 32x32 with int32
// accumulators, so the sum is exact whatever order the hardware adds in.
// The epilogue fuses the reference's dequant flush (gemma.c:3854-3865): each
// accumulator is rescaled with the row and column scales and stored fp32.
//
// Operand layout: a lane supplies row (lane % 32) of its 32-row tile and the
// 16-byte K chunk (lane / 32) of each 32-byte K sub-step, for A and B alike.
// The A and B k-index maps therefore coincide, and an exact int32 dot product
// does not depend on which k the hardware pairs inside one instruction.
// Output layout (32x32 MFMA): accumulator r of lane l holds row
// 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "gh_arith.h"
#include "gh_kernels.h"

namespace gh {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;                   // bytes of K per step
constexpr int kRowChunks = kBK / 16 + 1;  // 16-byte chunks per LDS row (+1 pad)

// VEC-free requirement: k % 16 == 0 and every row 16-byte aligned (checked
// by the launcher); rows/columns beyond m/n and K beyond k load as zeros.
template <bool HEADS>
__global__ __launch_bounds__(kThreads) void gemm_i8_kernel(
    float *__restrict__ dst, int dstr, int hdim, const int8_t *__restrict__ mat,
    int mstr, const float *__restrict__ matsc, const int8_t *__restrict__ src,
    int sstr, const float *__restrict__ ssc, int m, int n, int k) {
  __shared__ v4i lds_a[2][kBM][kRowChunks];
  __shared__ v4i lds_b[2][kBN][kRowChunks];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;  // wave's 64-row half of the block tile
  const int wn = wave & 1;   // wave's 64-column half
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;

  // global -> register mapping: thread loads chunk (tid % 4) of rows
  // tid/4 and 64 + tid/4 of both the A and the B tile
  const int ld_row = tid >> 2;
  const int ld_chunk = tid & 3;

  v4i ra[2], rb[2];
  auto load_tiles = [&](int kt) {
    const int kb = kt * kBK + ld_chunk * 16;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = ld_row + 64 * h;
      const int gm = m0 + r;
      const int gn = n0 + r;
      ra[h] = (gm < m && kb < k)
                  ? *reinterpret_cast<const v4i *>(src + (size_t)gm * sstr + kb)
                  : v4i{0, 0, 0, 0};
      rb[h] = (gn < n && kb < k)
                  ? *reinterpret_cast<const v4i *>(mat + (size_t)gn * mstr + kb)
                  : v4i{0, 0, 0, 0};
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      lds_a[buf][ld_row + 64 * h][ld_chunk] = ra[h];
      lds_b[buf][ld_row + 64 * h][ld_chunk] = rb[h];
    }
  };

  v16i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16i{};

  const int nk = (k + kBK - 1) / kBK;
  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_chunk = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles(kt + 1);
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      v4i a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = lds_a[cur][wm * 64 + i * 32 + frag_row][ks * 2 + frag_chunk];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = lds_b[cur][wn * 64 + j * 32 + frag_row][ks * 2 + frag_chunk];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j],
                                                            acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // epilogue: rescale and store (gemma.c:3854-3865)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + wn * 64 + j * 32 + (lane & 31);
    if (col >= n) continue;
    const float wsc = matsc[col];
    float *out_col;
    size_t row_stride;
    if (HEADS) {
      out_col = dst + (size_t)(col / hdim) * m * hdim + (col % hdim);
      row_stride = hdim;
    } else {
      out_col = dst + col;
      row_stride = dstr;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row =
            m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < m)
          out_col[(size_t)row * row_stride] = rescale(acc[i][j][r], ssc[row], wsc);
      }
    }
  }
}

// Any shape, any alignment: one thread per output, byte loads.  Used only
// when k % 16 != 0 or a row is not 16-byte aligned.
template <bool HEADS>
__global__ __launch_bounds__(kThreads) void gemm_i8_generic_kernel(
    float *__restrict__ dst, int dstr, int hdim, const int8_t *__restrict__ mat,
    int mstr, const float *__restrict__ matsc, const int8_t *__restrict__ src,
    int sstr, const float *__restrict__ ssc, int m, int n, int k) {
  const int col = blockIdx.x * 64 + (threadIdx.x & 63);
  const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (row >= m || col >= n) return;
  const int8_t *a = src + (size_t)row * sstr;
  const int8_t *b = mat + (size_t)col * mstr;
  int32_t acc = 0;
  for (int l = 0; l < k; ++l) acc += (int32_t)a[l] * (int32_t)b[l];
  const float y = rescale(acc, ssc[row], matsc[col]);
  if (HEADS)
    dst[((size_t)(col / hdim) * m + row) * hdim + col % hdim] = y;
  else
    dst[(size_t)row * dstr + col] = y;
}

}  // namespace

hipError_t launch_gemm_i8(float *dst, int dstr, int hdim, const int8_t *mat,
                          int mstr, const float *matsc, const int8_t *src,
                          int sstr, const float *ssc, int m, int n, int k,
                          const DeviceInfo &dev, hipStream_t stream) {
  (void)dev;
  const bool fast = k % 16 == 0 && mstr % 16 == 0 && sstr % 16 == 0 &&
                    (uintptr_t)mat % 16 == 0 && (uintptr_t)src % 16 == 0;
  const bool heads = hdim > 0;
  if (fast) {
    const dim3 grid((n + kBN - 1) / kBN, (m + kBM - 1) / kBM);
    if (heads)
      gemm_i8_kernel<true><<<grid, kThreads, 0, stream>>>(
          dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k);
    else
      gemm_i8_kernel<false><<<grid, kThreads, 0, stream>>>(
          dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k);
  } else {
    const dim3 grid((n + 63) / 64, (m + 3) / 4);
    if (heads)
      gemm_i8_generic_kernel<true><<<grid, kThreads, 0, stream>>>(
          dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k);
    else
      gemm_i8_generic_kernel<false><<<grid, kThreads, 0, stream>>>(
          dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k);
  }
  return hipGetLastError();
}

}  // namespace gh
