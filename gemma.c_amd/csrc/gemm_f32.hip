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
#include <algorithm>
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
// registers; one buffer (60 KB at 128x128: two workgroups per CU), two
// barriers per step.  Measured on the 4b prefill shapes and dropped: two
// buffers with one barrier per step (16- or 32-float steps) ran 3-10%
// slower at the same tiles.
//
// B comes as segments (F32Segs: q, k, v or gate, up side by side in the
// output); each thread resolves the rows it loads to their segment once.
// Split-K (SK, splits > 1): workgroup (x, y, z) computes K steps
// [z nk / splits, (z + 1) nk / splits) of tile (x, y), stores its fp32
// partial tile to the workspace, and counts itself in on the tile's counter;
// the workgroup that arrives last sums the splits' partials in split order
// (its own from registers), so the result does not depend on the order of
// arrival, runs the epilogue and resets the counter.
struct F32Split {
  int splits;
  int *ws;   // [tiles][splits][kThreads * WM * WN * 16] fp32 bits
  int *cnt;  // [tiles], zero between launches
};

template <int WM, int WN, bool SK>
__global__ __launch_bounds__(kThreads, 2) void gemm_bf3_kernel(
    float *__restrict__ dst, int dstr, F32Segs b, int mstr, const float *__restrict__ src,
    int sstr, int m, int k, F32Epilogue ep, F32Split sk) {
  constexpr int kBM = 64 * WM, kBN = 64 * WN;
  constexpr int BK = 32;              // floats of K per step
  constexpr int RW = BK + 8;          // plane row (bf16): 8 consecutive rows in distinct banks
  constexpr int CPR = BK / 4;         // float4 chunks per row and step
  constexpr int RPP = kThreads / CPR; // rows per load pass
  constexpr int HA = kBM / RPP, HB = kBN / RPP;
  static_assert(kBM % RPP == 0 && kBN % RPP == 0, "tile");
  __shared__ __attribute__((aligned(16))) uint16_t pa[3][kBM * RW];
  __shared__ __attribute__((aligned(16))) uint16_t pb[3][kBN * RW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int n = b.end[b.nseg - 1];
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;
  const int ld_row = tid / CPR, ld_c = tid % CPR;  // chunk ld_c of rows ld_row + RPP h

  // the B rows this thread loads (null past the last column)
  const float *brow[HB];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    const int gn = n0 + ld_row + RPP * h;
    const int t = (b.nseg > 1 && gn >= b.end[0]) + (b.nseg > 2 && gn >= b.end[1]);
    const int first = t == 0 ? 0 : t == 1 ? b.end[0] : b.end[1];
    const float *w = t == 0 ? b.w[0] : t == 1 ? b.w[1] : b.w[2];
    brow[h] = gn < n ? w + (size_t)(gn - first) * mstr : nullptr;
  }

  v4f ra[HA], rb[HB];
  auto load = [&](int kt) {
    const int kb = kt * BK + 4 * ld_c;
#pragma unroll
    for (int h = 0; h < HA; ++h) {
      const int gm = m0 + ld_row + RPP * h;
      ra[h] = (gm < m && kb < k)
                  ? *reinterpret_cast<const v4f *>(src + (size_t)gm * sstr + kb)
                  : v4f{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int h = 0; h < HB; ++h)
      rb[h] = (brow[h] != nullptr && kb < k) ? *reinterpret_cast<const v4f *>(brow[h] + kb)
                                             : v4f{0.f, 0.f, 0.f, 0.f};
  };
  auto split_store = [&]() {
#pragma unroll
    for (int h = 0; h < HA; ++h) {
      const Bf3x2 lo = split3x2(ra[h][0], ra[h][1]), hi = split3x2(ra[h][2], ra[h][3]);
      const int at = (ld_row + RPP * h) * RW + 4 * ld_c;
      *reinterpret_cast<u2 *>(&pa[0][at]) = u2{lo.q0, hi.q0};
      *reinterpret_cast<u2 *>(&pa[1][at]) = u2{lo.q1, hi.q1};
      *reinterpret_cast<u2 *>(&pa[2][at]) = u2{lo.q2, hi.q2};
    }
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const Bf3x2 lo = split3x2(rb[h][0], rb[h][1]), hi = split3x2(rb[h][2], rb[h][3]);
      const int at = (ld_row + RPP * h) * RW + 4 * ld_c;
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

  const int fr = lane & 31, half = lane >> 5;
  auto mfmas = [&]() {
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      bf8 a[WM][3], bb[WN][3];
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
        for (int p = 0; p < 3; ++p) bb[j][p] = *reinterpret_cast<const bf8 *>(&pb[p][at]);
      }
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          v16f c = acc[i][j];
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][2], bb[j][0], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][1], bb[j][1], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], bb[j][2], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][1], bb[j][0], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], bb[j][1], c, 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], bb[j][0], c, 0, 0, 0);
        }
    }
  };

  const int nk = (k + BK - 1) / BK;
  int kt0 = 0, kt1 = nk;
  if constexpr (SK) {
    kt0 = (int)((long)blockIdx.z * nk / sk.splits);
    kt1 = (int)((long)(blockIdx.z + 1) * nk / sk.splits);
  }
  load(kt0);
  for (int kt = kt0; kt < kt1; ++kt) {
    split_store();
    lds_barrier();  // the step's planes are complete
    if (kt + 1 < kt1) load(kt + 1);  // the next step's rows load during the MFMAs
    mfmas();
    lds_barrier();  // every wave is done with the planes
  }

  if constexpr (SK) {
    // Partials go out and come back in with device-coherent (agent-scope)
    // accesses, which write through and read past this XCD's L2.
    constexpr int kTileInts = kThreads * WM * WN * 16;
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int z = blockIdx.z;
    int *part = sk.ws + (size_t)tile * sk.splits * kTileInts;
    int *mine = part + (size_t)z * kTileInts;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          __hip_atomic_store(mine + ((i * WN + j) * 16 + r) * kThreads + tid,
                             __float_as_int(acc[i][j][r]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    __shared__ int last;
    wait_vmcnt<0>();  // this thread's partial has reached the coherence point
    __syncthreads();
    if (tid == 0) last = atomicAdd(sk.cnt + tile, 1) == sk.splits - 1;
    __syncthreads();
    if (!last) return;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int at = ((i * WN + j) * 16 + r) * kThreads + tid;
          float t = 0.f;
          for (int o = 0; o < sk.splits; ++o)
            t += o == z ? acc[i][j][r]
                        : __int_as_float(__hip_atomic_load(part + (size_t)o * kTileInts + at,
                                                           __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT));
          acc[i][j][r] = t;
        }
    if (tid == 0) sk.cnt[tile] = 0;
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

// One launch of the split kernel: tiles of (64 WM) x (64 WN), `splits`
// workgroups per tile along z (1: no split-K).
template <int WM, int WN>
hipError_t launch_bf3(float *dst, int dstr, const F32Segs &b, int mstr, const float *src,
                      int sstr, int m, int k, const F32Epilogue &ep, int splits,
                      hipStream_t stream) {
  const int n = b.end[b.nseg - 1];
  const dim3 grid((n + 64 * WN - 1) / (64 * WN), (m + 64 * WM - 1) / (64 * WM), splits);
  F32Split sk{splits, nullptr, nullptr};
  if (splits > 1) {
    const int tiles = (int)(grid.x * grid.y);
    const hipError_t e = split_workspace(
        stream, (size_t)tiles * splits * kThreads * WM * WN * 16, tiles, &sk.ws, &sk.cnt);
    if (e != hipSuccess) return e;
    gemm_bf3_kernel<WM, WN, true><<<grid, kThreads, 0, stream>>>(dst, dstr, b, mstr, src, sstr,
                                                                m, k, ep, sk);
  } else {
    gemm_bf3_kernel<WM, WN, false><<<grid, kThreads, 0, stream>>>(dst, dstr, b, mstr, src, sstr,
                                                                 m, k, ep, sk);
  }
  return hipGetLastError();
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

// Block tile of the fp32-MFMA kernel: 128x128 when that gives every CU at
// least two workgroups, else 64x64 (k/v, o and down at the gemma-3-4b
// prefill shapes leave most of the GPU idle at 128x128).
// GEMMA_HIP_GEMM_F32_TILE=128, 128x64 or 64 (read at every launch) forces a
// tile for either kernel.
enum Tile { kTile64, kTile128x64, kTile128 };
bool forced_tile(Tile *t) {
  const char *e = getenv("GEMMA_HIP_GEMM_F32_TILE");
  if (e == nullptr) return false;
  if (strcmp(e, "128") == 0) *t = kTile128;
  else if (strcmp(e, "128x64") == 0) *t = kTile128x64;
  else if (strcmp(e, "64") == 0) *t = kTile64;
  else return false;
  return true;
}

Tile f32_tile(int m, int n, const DeviceInfo &dev) {
  Tile t;
  if (forced_tile(&t)) return t;
  const long tiles128 = (long)((m + 127) / 128) * ((n + 127) / 128);
  return tiles128 >= 2L * dev.cus ? kTile128 : kTile64;
}

long tile_count(int m, int n, Tile t) {
  const int bm = t == kTile64 ? 64 : 128, bn = t == kTile128 ? 128 : 64;
  return (long)((m + bm - 1) / bm) * ((n + bn - 1) / bn);
}

// Tile and split-K ways of the split kernel (two 128x128, three 128x64 or
// four 64x64 workgroups per CU), from a sweep of the gemma-3 prefill and
// SigLIP shapes (M = 512, 2048, 4096; T = the count of 128x128 tiles):
//   T >= 1.5 per CU:           128x128, no split
//   T >= 1 per CU:             128x128 in 3 splits when K >= 3072 floats
//                              (4b down 743 -> 604 us, SigLIP fc2 315 -> 285);
//                              else 128x128 in 2 when those fill two per CU
//                              to within 10% (4b q 166 -> 140), else 128x64
//                              in 2 (4b o 147)
//   128x64 tiles >= 1 per CU:  128x64 in 2 (4b k/v 89 -> 83)
//   fewer:                     64x64, splits for ~1.5 workgroups per CU
//                              (1b down at M=512: 3 splits, 86 us; 6: 92)
// Each split keeps at least 8 K steps (256 floats); at most 16 splits.
// GEMMA_HIP_GEMM_F32_TILE forces the tile (the split then follows the last
// rule for that tile's count), GEMMA_HIP_GEMM_F32_SPLIT=s the splits
// (clamped to 1..min(16, K steps)); both are read at every launch.
struct Bf3Plan {
  Tile tile;
  int splits;
};
Bf3Plan bf3_plan(int m, int n, int k, const DeviceInfo &dev) {
  const int nk = (k + 31) / 32;
  Bf3Plan p{kTile64, 1};
  const long t128 = tile_count(m, n, kTile128);
  if (forced_tile(&p.tile)) {
    const long t = tile_count(m, n, p.tile);
    p.splits = t >= dev.cus ? 1 : (int)((3L * dev.cus + 2 * t - 1) / (2 * t));
  } else if (2 * t128 >= 3L * dev.cus) {
    p = {kTile128, 1};
  } else if (t128 >= dev.cus) {
    if (nk >= 96)
      p = {kTile128, 3};
    else if (10 * t128 <= 11L * dev.cus)
      p = {kTile128, 2};
    else
      p = {kTile128x64, 2};
  } else if (tile_count(m, n, kTile128x64) >= dev.cus) {
    p = {kTile128x64, 2};
  } else {
    const long t = tile_count(m, n, kTile64);
    p = {kTile64, (int)((3L * dev.cus + 2 * t - 1) / (2 * t))};
  }
  p.splits = std::min(p.splits, std::max(1, nk / 8));
  const char *e = getenv("GEMMA_HIP_GEMM_F32_SPLIT");
  if (e != nullptr) p.splits = atoi(e);
  p.splits = std::max(1, std::min({p.splits, nk, 16}));
  return p;
}

hipError_t launch_bf3_auto(float *dst, int dstr, const F32Segs &b, int mstr, const float *src,
                           int sstr, int m, int k, const F32Epilogue &ep, const DeviceInfo &dev,
                           hipStream_t stream) {
  Bf3Plan p = bf3_plan(m, b.end[b.nseg - 1], k, dev);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (p.splits > 1 &&
      (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone))
    p.splits = 1;  // the split-K workspace may have to be allocated: not under capture
  if (p.tile == kTile128)
    return launch_bf3<2, 2>(dst, dstr, b, mstr, src, sstr, m, k, ep, p.splits, stream);
  if (p.tile == kTile128x64)
    return launch_bf3<2, 1>(dst, dstr, b, mstr, src, sstr, m, k, ep, p.splits, stream);
  return launch_bf3<1, 1>(dst, dstr, b, mstr, src, sstr, m, k, ep, p.splits, stream);
}

// float4 loads of both operands: K and the row strides multiples of 4
// floats, the bases 16-byte aligned.
bool f32_vec4(int k, int mstr, int sstr, const float *mat, const float *src) {
  return k % 4 == 0 && mstr % 4 == 0 && sstr % 4 == 0 && (uintptr_t)mat % 16 == 0 &&
         (uintptr_t)src % 16 == 0;
}

}  // namespace

hipError_t launch_gemm_f32(float *dst, int dstr, const float *mat, int mstr,
                           const float *src, int sstr, int m, int n, int k,
                           const F32Epilogue &ep, const DeviceInfo &dev, hipStream_t stream,
                           bool f64) {
  if (f64) {
    const dim3 grid((n + kF64N - 1) / kF64N, (m + kF64M - 1) / kF64M);
    gemm_f64_kernel<<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr, src, sstr, m, n, k, ep);
    return hipGetLastError();
  }
  if (f32_vec4(k, mstr, sstr, mat, src)) {
    if (gemm_f32_split()) {
      const F32Segs b{{mat, nullptr, nullptr}, {n, n, n}, 1};
      return launch_bf3_auto(dst, dstr, b, mstr, src, sstr, m, k, ep, dev, stream);
    }
    const Tile tile = f32_tile(m, n, dev);
    if (tile == kTile128) {
      const dim3 grid((n + 127) / 128, (m + 127) / 128);
      gemm_f32_kernel<2, 2><<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr, src, sstr, m,
                                                          n, k, ep);
    } else if (tile == kTile128x64) {
      const dim3 grid((n + 63) / 64, (m + 127) / 128);
      gemm_f32_kernel<2, 1><<<grid, kThreads, 0, stream>>>(dst, dstr, mat, mstr, src, sstr, m,
                                                          n, k, ep);
    } else {
      const dim3 grid((n + 63) / 64, (m + 63) / 64);
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

hipError_t launch_gemm_f32_segs(float *dst, int dstr, const F32Segs &b, int mstr,
                                const float *src, int sstr, int m, int k,
                                const F32Epilogue &ep, const DeviceInfo &dev, hipStream_t stream,
                                bool f64) {
  bool vec4 = true;
  for (int t = 0; t < b.nseg; ++t) vec4 = vec4 && f32_vec4(k, mstr, sstr, b.w[t], src);
  if (!f64 && vec4 && gemm_f32_split())
    return launch_bf3_auto(dst, dstr, b, mstr, src, sstr, m, k, ep, dev, stream);
  // one launch per segment, the epilogue's column-indexed inputs shifted
  // to the segment's first column
  for (int t = 0; t < b.nseg; ++t) {
    const int first = t ? b.end[t - 1] : 0;
    F32Epilogue et = ep;
    if (et.bias != nullptr) et.bias += first;
    if (et.pos_q != nullptr) et.pos_q += first;
    if (et.pos_f != nullptr) et.pos_f += first;
    const hipError_t e = launch_gemm_f32(dst + first, dstr, b.w[t], mstr, src, sstr, m,
                                         b.end[t] - first, k, et, dev, stream, f64);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
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
