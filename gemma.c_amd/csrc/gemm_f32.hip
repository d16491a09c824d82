// gemm_f32.hip -- fp32 fallback GEMM for unquantized model files
// (gemma.c:3304-3399 gemm_fpx), on fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
//   dst[i][j] = sum_l src[i][l]*mat[j][l]
//
// 256 threads, 2x2 waves, 128x128 or 64x64 block tiles, a K step of 16
// floats (64 bytes per row) double-buffered in LDS.  A lane
// owns 8 consecutive k of each step (lane / 32 picks the half) for A and B
// alike, so each of the 8 MFMA sub-steps pairs matching k.  The reference's
// fp32 sum has no fixed order (vectorised, KC-chunked, gemma.c:3287-3299), so
// parity for this path is a tolerance on |y - y_exact| / sum|a*b|.
#include <cstdlib>
#include <cstring>

#include "gh_arith.h"
#include "gh_kernels.h"

namespace gh {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 16;                   // floats of K per step
constexpr int kRowChunks = kBK / 4 + 1;   // float4 chunks per LDS row (+1 pad)

// WM x WN: each wave's sub-tile in 32x32 MFMA tiles; the 2x2 waves make a
// (64 WM) x (64 WN) block tile.
template <int WM, int WN>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(
    float *__restrict__ dst, int dstr, const float *__restrict__ mat, int mstr,
    const float *__restrict__ src, int sstr, int m, int n, int k, F32Epilogue ep) {
  constexpr int kBM = 64 * WM, kBN = 64 * WN;
  __shared__ v4f lds_a[2][kBM][kRowChunks];
  __shared__ v4f lds_b[2][kBN][kRowChunks];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;
  const int ld_row = tid >> 2;
  const int ld_chunk = tid & 3;

  v4f ra[WM], rb[WN];
  auto load_tiles = [&](int kt) {
    const int kb = kt * kBK + ld_chunk * 4;
#pragma unroll
    for (int h = 0; h < WM; ++h) {
      const int gm = m0 + ld_row + 64 * h;
      ra[h] = (gm < m && kb < k)
                  ? *reinterpret_cast<const v4f *>(src + (size_t)gm * sstr + kb)
                  : v4f{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int h = 0; h < WN; ++h) {
      const int gn = n0 + ld_row + 64 * h;
      rb[h] = (gn < n && kb < k)
                  ? *reinterpret_cast<const v4f *>(mat + (size_t)gn * mstr + kb)
                  : v4f{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int h = 0; h < WM; ++h) lds_a[buf][ld_row + 64 * h][ld_chunk] = ra[h];
#pragma unroll
    for (int h = 0; h < WN; ++h) lds_b[buf][ld_row + 64 * h][ld_chunk] = rb[h];
  };

  v16f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v16f{};

  const int nk = (k + kBK - 1) / kBK;
  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  const int frag_row = lane & 31;
  const int half = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles(kt + 1);
    v4f a[WM][2], b[WN][2];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      a[i][0] = lds_a[cur][wm * 32 * WM + i * 32 + frag_row][half * 2];
      a[i][1] = lds_a[cur][wm * 32 * WM + i * 32 + frag_row][half * 2 + 1];
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      b[j][0] = lds_b[cur][wn * 32 * WN + j * 32 + frag_row][half * 2];
      b[j][1] = lds_b[cur][wn * 32 * WN + j * 32 + frag_row][half * 2 + 1];
    }
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
              a[i][s >> 2][s & 3], b[j][s >> 2][s & 3], acc[i][j], 0, 0, 0);
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int col = n0 + wn * 32 * WN + j * 32 + (lane & 31);
    if (col >= n) continue;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row =
            m0 + wm * 32 * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < m) dst[(size_t)row * dstr + col] = ep.apply(acc[i][j][r], row, col, dstr);
      }
  }
}

// The same GEMM on the bf16 matrix cores in split precision: every fp32
// operand x is split into three bf16 pieces x = x0 + x1 + x2 (split3x2: each
// rounded to nearest from the remainder, together x's 24 significant bits)
// and each product summed from the six piece products whose orders add up
// to at most 2 (a2 b0, a1 b1, a0 b2, a1 b0, a0 b1, a0 b0, the small ones
// first), on v_mfma_f32_32x32x16_bf16 with fp32 accumulation: the dropped
// terms are below 3 * 2^-24 |a b| and bf16 x bf16 products are exact, so
// each product carries an fp32 rounding's error, and the sums are fp32 as in
// the fp32-MFMA kernel.  The six bf16 MFMAs cost ~0.4 of that kernel's fp32
// MFMA work.  Geometry as gemm_f32_kernel (2x2 waves of WM x WN 32x32 tiles,
// the same output layout: lane l, element r -> row 8 (r/4) + 4 (l/32) + r%4,
// column l%32; A and B fragments give lane l row l%32 and k 8 (l/32) .. + 7).
// Per 32-float K step the workgroup splits its A and B rows once into three
// bf16 planes each in LDS, while the next step's fp32 rows load into
// registers; one buffer (60 KB at 128x128), two workgroups per CU.
template <int WM, int WN>
__global__ __launch_bounds__(kThreads, 2) void gemm_bf3_kernel(
    float *__restrict__ dst, int dstr, const float *__restrict__ mat, int mstr,
    const float *__restrict__ src, int sstr, int m, int n, int k, F32Epilogue ep) {
  constexpr int kBM = 64 * WM, kBN = 64 * WN;
  constexpr int BK = 32;      // floats of K per step
  constexpr int RW = BK + 8;  // plane row (bf16): 8 consecutive rows in distinct banks
  constexpr int HA = kBM / 32, HB = kBN / 32;  // rows per thread and step
  __shared__ __attribute__((aligned(16))) uint16_t pa[3][kBM * RW];
  __shared__ __attribute__((aligned(16))) uint16_t pb[3][kBN * RW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;
  const int ld_row = tid >> 3, ld_c = tid & 7;  // float4 chunk ld_c of rows ld_row + 32 h

  v4f ra[HA], rb[HB];
  auto load = [&](int kt) {
    const int kb = kt * BK + 4 * ld_c;
#pragma unroll
    for (int h = 0; h < HA; ++h) {
      const int gm = m0 + ld_row + 32 * h;
      ra[h] = (gm < m && kb < k)
                  ? *reinterpret_cast<const v4f *>(src + (size_t)gm * sstr + kb)
                  : v4f{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const int gn = n0 + ld_row + 32 * h;
      rb[h] = (gn < n && kb < k)
                  ? *reinterpret_cast<const v4f *>(mat + (size_t)gn * mstr + kb)
                  : v4f{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto split_store = [&]() {
#pragma unroll
    for (int h = 0; h < HA; ++h) {
      const Bf3x2 lo = split3x2(ra[h][0], ra[h][1]), hi = split3x2(ra[h][2], ra[h][3]);
      const int at = (ld_row + 32 * h) * RW + 4 * ld_c;
      *reinterpret_cast<u2 *>(&pa[0][at]) = u2{lo.q0, hi.q0};
      *reinterpret_cast<u2 *>(&pa[1][at]) = u2{lo.q1, hi.q1};
      *reinterpret_cast<u2 *>(&pa[2][at]) = u2{lo.q2, hi.q2};
    }
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const Bf3x2 lo = split3x2(rb[h][0], rb[h][1]), hi = split3x2(rb[h][2], rb[h][3]);
      const int at = (ld_row + 32 * h) * RW + 4 * ld_c;
      *reinterpret_cast<u2 *>(&pb[0][at]) = u2{lo.q0, hi.q0};
      *reinterpret_cast<u2 *>(&pb[1][at]) = u2{lo.q1, hi.q1};
      *reinterpret_cast<u2 *>(&pb[2][at]) = u2{lo.q2, hi.q2};
    }
  };

  v16f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v16f{};

  const int nk = (k + BK - 1) / BK;
  const int fr = lane & 31, half = lane >> 5;
  load(0);
  for (int kt = 0; kt < nk; ++kt) {
    split_store();
    lds_barrier();  // the step's planes are complete
    if (kt + 1 < nk) load(kt + 1);  // the next step's rows load during the MFMAs
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      bf8 a[WM][3], b[WN][3];
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        const int at = (wm * 32 * WM + i * 32 + fr) * RW + 16 * s + 8 * half;
#pragma unroll
        for (int p = 0; p < 3; ++p) a[i][p] = *reinterpret_cast<const bf8 *>(&pa[p][at]);
      }
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int at = (wn * 32 * WN + j * 32 + fr) * RW + 16 * s + 8 * half;
#pragma unroll
        for (int p = 0; p < 3; ++p) b[j][p] = *reinterpret_cast<const bf8 *>(&pb[p][at]);
      }
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          v16f c = acc[i][j];
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][2], b[j][0], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][1], b[j][1], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][2], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][1], b[j][0], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][1], c, 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][0], c, 0, 0, 0);
        }
    }
    lds_barrier();  // every wave is done with the planes
  }

#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int col = n0 + wn * 32 * WN + j * 32 + (lane & 31);
    if (col >= n) continue;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row =
            m0 + wm * 32 * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < m) dst[(size_t)row * dstr + col] = ep.apply(acc[i][j][r], row, col, dstr);
      }
  }
}

// Any shape, any alignment: one thread per output.
__global__ __launch_bounds__(kThreads) void gemm_f32_generic_kernel(
    float *__restrict__ dst, int dstr, const float *__restrict__ mat, int mstr,
    const float *__restrict__ src, int sstr, int m, int n, int k, F32Epilogue ep) {
  const int col = blockIdx.x * 64 + (threadIdx.x & 63);
  const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (row >= m || col >= n) return;
  const float *a = src + (size_t)row * sstr;
  const float *b = mat + (size_t)col * mstr;
  float acc = 0.0f;
  for (int l = 0; l < k; ++l) acc = __builtin_fmaf(a[l], b[l], acc);
  dst[(size_t)row * dstr + col] = ep.apply(acc, row, col, dstr);
}

// The fp64 twin of the fp32 GEMM for the verification modes: each output is
// the fp64 sum, rounded once by the epilogue.  A workgroup computes a 32 x 64
// tile, each thread 2 x 4 outputs, over K in LDS chunks of 32.
constexpr int kF64M = 32, kF64N = 64, kF64K = 32;

__global__ __launch_bounds__(kThreads) void gemm_f64_kernel(
    float *__restrict__ dst, int dstr, const float *__restrict__ mat, int mstr,
    const float *__restrict__ src, int sstr, int m, int n, int k, F32Epilogue ep) {
  __shared__ float as[kF64M][kF64K + 1];
  __shared__ float bs[kF64N][kF64K + 1];
  const int tid = threadIdx.x;
  const int m0 = blockIdx.y * kF64M, n0 = blockIdx.x * kF64N;
  const int tm = tid / 16, tn = tid % 16;  // outputs (m0 + 2 tm + i, n0 + tn + 16 j)
  double acc[2][4] = {};
  for (int k0 = 0; k0 < k; k0 += kF64K) {
    for (int i = tid; i < kF64M * kF64K; i += kThreads) {
      const int r = i / kF64K, c = i % kF64K;
      as[r][c] = (m0 + r < m && k0 + c < k) ? src[(size_t)(m0 + r) * sstr + k0 + c] : 0.0f;
    }
    for (int i = tid; i < kF64N * kF64K; i += kThreads) {
      const int r = i / kF64K, c = i % kF64K;
      bs[r][c] = (n0 + r < n && k0 + c < k) ? mat[(size_t)(n0 + r) * mstr + k0 + c] : 0.0f;
    }
    __syncthreads();
#pragma unroll 4
    for (int c = 0; c < kF64K; ++c) {
      const double x0 = as[2 * tm][c], x1 = as[2 * tm + 1][c];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double w = bs[tn + 16 * j][c];
        acc[0][j] = fma(x0, w, acc[0][j]);
        acc[1][j] = fma(x1, w, acc[1][j]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = m0 + 2 * tm + i;
    if (row >= m) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + tn + 16 * j;
      if (col < n) dst[(size_t)row * dstr + col] = ep.apply_f64(acc[i][j], row, col, dstr);
    }
  }
}

// The fp32 GEMM's kernel: the split-bf16 one by default, the fp32-MFMA one
// with GEMMA_HIP_GEMM_F32=mfma (read at every launch, so that one process
// can time or check both).
bool gemm_f32_split() {
  const char *e = getenv("GEMMA_HIP_GEMM_F32");
  return e == nullptr || strcmp(e, "mfma") != 0;
}

}  // namespace

// Block tile: 128x128 when that gives every CU at least two workgroups,
// else 64x64 (k/v, o and down at the gemma-3-4b prefill shapes leave most of
// the GPU idle at 128x128).  GEMMA_HIP_GEMM_F32_TILE=128 or 64 forces one.
hipError_t launch_gemm_f32(float *dst, int dstr, const float *mat, int mstr,
                           const float *src, int sstr, int m, int n, int k,
                           const F32Epilogue &ep, const DeviceInfo &dev, hipStream_t stream,
                           bool f64) {
  if (f64) {
    const dim3 grid((n + kF64N - 1) / kF64N, (m + kF64M - 1) / kF64M);
    gemm_f64_kernel<<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr, src, sstr, m, n, k, ep);
    return hipGetLastError();
  }
  const bool fast = k % 4 == 0 && mstr % 4 == 0 && sstr % 4 == 0 &&
                    (uintptr_t)mat % 16 == 0 && (uintptr_t)src % 16 == 0;
  if (fast) {
    static const int forced = [] {
      const char *e = getenv("GEMMA_HIP_GEMM_F32_TILE");
      return e != nullptr ? atoi(e) : 0;
    }();
    const long tiles128 = (long)((m + 127) / 128) * ((n + 127) / 128);
    const bool big = forced == 128 || (forced != 64 && tiles128 >= 2L * dev.cus);
    const bool split = gemm_f32_split();
    if (big) {
      const dim3 grid((n + 127) / 128, (m + 127) / 128);
      if (split)
        gemm_bf3_kernel<2, 2><<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr, src, sstr, m,
                                                            n, k, ep);
      else
        gemm_f32_kernel<2, 2><<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr, src, sstr, m,
                                                            n, k, ep);
    } else {
      const dim3 grid((n + 63) / 64, (m + 63) / 64);
      if (split)
        gemm_bf3_kernel<1, 1><<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr, src, sstr, m,
                                                            n, k, ep);
      else
        gemm_f32_kernel<1, 1><<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr, src, sstr, m,
                                                            n, k, ep);
    }
  } else {
    const dim3 grid((n + 63) / 64, (m + 3) / 4);
    gemm_f32_generic_kernel<<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr,
                                                           src, sstr, m, n, k, ep);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_f32(float *dst, int dstr, const float *mat, int mstr,
                           const float *src, int sstr, int m, int n, int k,
                           const float *bias, bool clamp,
                           const DeviceInfo &dev, hipStream_t stream) {
  F32Epilogue ep{};
  ep.bias = bias;
  ep.clamp = clamp;
  return launch_gemm_f32(dst, dstr, mat, mstr, src, sstr, m, n, k, ep, dev, stream, false);
}

}  // namespace gh
