// gemm_i8.hip -- prefill / SigLIP int8 GEMM on CDNA4 int8 MFMA
// (gemma.c:3937-4054 gemm_int8 and its tile/flush helpers 3847-3935).
//
//   dst[i][j] = (float)sum_l src[i][l]*mat[j][l] * (ssc[i]*matsc[j])
//
// Both operands are K-contiguous ("NT"), the layout MFMA wants: a lane feeds
// 16 consecutive int8 of one row to v_mfma_i32_32x32x32_i8.  A workgroup is
// 256 threads = 4 waves in a 2x2 grid; each wave owns WM x WN tiles of 32x32
// with int32 accumulators, so the sum is exact whatever order the hardware
// adds in.  Operand layout: a lane supplies row (lane % 32) of its 32-row
// tile and the 16-byte K chunk (lane / 32) of each 32-byte K sub-step, for A
// and B alike; the A and B k-index maps coincide, so the exact dot product
// does not depend on which k the hardware pairs inside one instruction.
// Output layout (32x32 MFMA): accumulator r of lane l holds row
// 8*(r/4) + 4*(l/32) + r%4, column l%32.
//
// Kernels:
//  - gemm_i8_dma_kernel (default): operands go global -> LDS by
//    buffer_load ... lds into an S-stage ring (no VGPRs held, zero fill by
//    out-of-range offsets), XOR-swizzled so fragment reads are bank-conflict
//    free; one barrier per K stage.  The epilogue (store_tile) fuses the
//    reference's dequant flush (gemma.c:3854-3865) with scales loaded at
//    kernel start and buffer stores whose out-of-range cells are dropped.
//  - gemm_i8_kernel: register-staged loads into a padded LDS double buffer;
//    used when an operand is too large for 32-bit buffer offsets.
//  - gemm_i8_generic_kernel: one thread per output, any shape/alignment.
// Tile choice and the measurements behind it are in launch_gemm_i8.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "gh_arith.h"
#include "gh_kernels.h"

// Caller-free workspace of gemma_hip_matmul_noalloc: the int32 partial tiles
// and tile counters of split-K launches, one copy per GPU that loads the
// library, held until the process ends.  Host code never passes `scratch`
// itself to a kernel (in host code the name is a host-side stand-in, not a
// device address): it uses the address hipGetSymbolAddress returned for the
// device, kept in g_scratch_dev.
static __device__ __align__(256) int scratch[gh::kGemmScratchBytes / sizeof(int)];

namespace gh {
namespace {

constexpr int kMaxDevices = 64;
int *g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;

constexpr int kThreads = 256;
constexpr int kBK = 64;                   // bytes of K per step
constexpr int kRowChunks = kBK / 16 + 1;  // 16-byte chunks per LDS row (+1 pad)
constexpr int kXcds = 8;                  // MI355X: 8 XCDs, each with its own L2
constexpr int kGroupM = 8;                // M tiles per group of the tile order
constexpr uint32_t kOob = 0x80000000u;    // buffer offset: reads zero, drops stores

// Block -> tile.  The dispatcher hands workgroup b to XCD b % 8, so first
// give each XCD a contiguous range of tile ids, then walk tiles in groups of
// kGroupM row-tiles so neighbouring workgroups of one XCD share A rows and B
// columns in that XCD's L2.
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n,
                                        int *tm, int *tn) {
  const int total = tiles_m * tiles_n;
  const int per = total / kXcds, extra = total % kXcds;
  const int xcd = b % kXcds, idx = b / kXcds;
  const int t = xcd * per + (xcd < extra ? xcd : extra) + idx;
  const int per_group = kGroupM * tiles_n;
  const int group = t / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = t - group * per_group;
  *tm = first_m + in_group % gsize;
  *tn = in_group / gsize;
}

// Requirement (checked by the launcher): k % 16 == 0 and every row 16-byte
// aligned; rows/columns beyond m/n and K beyond k load as zeros.
// WM x WN: each wave's sub-tile in 32x32 MFMA tiles; waves form a 2x2 grid,
// so the block tile is (64*WM) x (64*WN).
template <int WM, int WN, bool HEADS>
__global__ __launch_bounds__(kThreads) void gemm_i8_kernel(
    float *__restrict__ dst, int dstr, int hdim, const int8_t *__restrict__ mat,
    int mstr, const float *__restrict__ matsc, const int8_t *__restrict__ src,
    int sstr, const float *__restrict__ ssc, int m, int n, int k) {
  constexpr int kBM = 64 * WM;
  constexpr int kBN = 64 * WN;
  __shared__ v4i lds_a[2][kBM][kRowChunks];
  __shared__ v4i lds_b[2][kBN][kRowChunks];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = wave >> 1;  // wave's row half of the block tile
  const int wn = wave & 1;   // wave's column half
  int tm, tn;
  tile_of(blockIdx.x, (m + kBM - 1) / kBM, (n + kBN - 1) / kBN, &tm, &tn);
  const int m0 = tm * kBM;
  const int n0 = tn * kBN;

  // global -> register mapping: thread loads chunk (tid % 4) of rows
  // tid/4 + 64*h of the A and the B tile
  const int ld_row = tid >> 2;
  const int ld_chunk = tid & 3;

  v4i ra[WM], rb[WN];
  auto load_tiles = [&](int kt) {
    const int kb = kt * kBK + ld_chunk * 16;
#pragma unroll
    for (int h = 0; h < WM; ++h) {
      const int gm = m0 + ld_row + 64 * h;
      ra[h] = (gm < m && kb < k)
                  ? *reinterpret_cast<const v4i *>(src + (size_t)gm * sstr + kb)
                  : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int h = 0; h < WN; ++h) {
      const int gn = n0 + ld_row + 64 * h;
      rb[h] = (gn < n && kb < k)
                  ? *reinterpret_cast<const v4i *>(mat + (size_t)gn * mstr + kb)
                  : v4i{0, 0, 0, 0};
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int h = 0; h < WM; ++h) lds_a[buf][ld_row + 64 * h][ld_chunk] = ra[h];
#pragma unroll
    for (int h = 0; h < WN; ++h) lds_b[buf][ld_row + 64 * h][ld_chunk] = rb[h];
  };

  v16i acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v16i{};

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
      v4i a[WM], b[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i)
        a[i] = lds_a[cur][wm * 32 * WM + i * 32 + frag_row][ks * 2 + frag_chunk];
#pragma unroll
      for (int j = 0; j < WN; ++j)
        b[j] = lds_b[cur][wn * 32 * WN + j * 32 + frag_row][ks * 2 + frag_chunk];
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j],
                                                            acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // epilogue: rescale and store (gemma.c:3854-3865)
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int col = n0 + wn * 32 * WN + j * 32 + (lane & 31);
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
    for (int i = 0; i < WM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 32 * WM + i * 32 + 8 * (r >> 2) +
                        4 * (lane >> 5) + (r & 3);
        if (row < m)
          out_col[(size_t)row * row_stride] = rescale(acc[i][j][r], ssc[row], wsc);
      }
    }
  }
}

// ---- epilogue shared by the DMA kernels -----------------------------------
//
// Scales are loaded at kernel start (their latency, including address
// translation, hides under the K loop).  Whether the plain IEEE rescale is
// exact for every output of the wave is decided once from the scales'
// extremes; row-major outputs then go out as buffer stores whose row offset
// is a uniform soffset and whose out-of-range rows/columns the hardware
// drops, so the common path is cvt + 2 multiplies + 1 store per output.
template <int WM, int WN>
struct TileScales {
  float act[WM][16];
  float w[WN];
};

template <int WM, int WN>
__device__ __forceinline__ void load_tile_scales(TileScales<WM, WN> &sc,
                                                 const float *__restrict__ ssc,
                                                 const float *__restrict__ matsc,
                                                 int m, int n, int m0, int n0,
                                                 int wm, int wn, int lane) {
#pragma unroll
  for (int j = 0; j < WN; ++j)
    sc.w[j] = matsc[min(n0 + wn * 32 * WN + j * 32 + (lane & 31), n - 1)];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      sc.act[i][r] = ssc[min(m0 + wm * 32 * WM + i * 32 + 8 * (r >> 2) +
                                 4 * (lane >> 5) + (r & 3), m - 1)];
}

template <int WM, int WN, bool HEADS>
__device__ __forceinline__ void store_tile(const v16i (&acc)[WM][WN],
                                           const TileScales<WM, WN> &sc,
                                           float *__restrict__ dst, int dstr,
                                           int hdim, int m, int n, int m0,
                                           int n0, int wm, int wn, int lane) {
  float amin = __builtin_inff(), wmin = __builtin_inff();
  bool asub = false, wsub = false;
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) scale_extremes(sc.act[i][r], &amin, &asub);
#pragma unroll
  for (int j = 0; j < WN; ++j) scale_extremes(sc.w[j], &wmin, &wsub);
  const bool plain_lane = rescale_all_plain(amin, asub, wmin, wsub);
  const bool all_plain = __builtin_amdgcn_readfirstlane(__any(!plain_lane) ? 0 : 1) != 0;

  if (!HEADS && all_plain) {
    // bytes of dst covered by valid cells: any offset at or past it is dropped
    const uint32_t extent = ((uint32_t)(m - 1) * (uint32_t)dstr + (uint32_t)n) * 4u;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        dst, (short)0, (int)extent, 0x00020000);
    const int row_lane = 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int col = n0 + wn * 32 * WN + j * 32 + (lane & 31);
      const uint32_t voff = col < n ? ((uint32_t)row_lane * dstr + col) * 4u : kOob;
#pragma unroll
      for (int i = 0; i < WM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row_base = m0 + wm * 32 * WM + i * 32 + 8 * (r >> 2) + (r & 3);
          const float y = (float)acc[i][j][r] * (sc.act[i][r] * sc.w[j]);
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), rs, voff,
                                                (uint32_t)row_base * dstr * 4u, 0);
        }
      }
    }
    return;
  }
  // head-major layout, or scales in FTZ/DAZ territory: guarded stores
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int col = n0 + wn * 32 * WN + j * 32 + (lane & 31);
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
    for (int i = 0; i < WM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 32 * WM + i * 32 + 8 * (r >> 2) +
                        4 * (lane >> 5) + (r & 3);
        const float y = all_plain ? (float)acc[i][j][r] * (sc.act[i][r] * sc.w[j])
                                  : rescale(acc[i][j][r], sc.act[i][r], sc.w[j]);
        if (row < m && col < n) out_col[(size_t)row * row_stride] = y;
      }
    }
  }
}

// ---- LDS-DMA pipelined kernel ------------------------------------------
//
// The register-staged kernel above waits one global round trip per 64-byte
// K step.  Here K steps are fetched S-1 steps ahead straight into an S-stage
// LDS ring with buffer_load_dwordx4 ... lds (no VGPRs held), so the MFMAs of
// step kt overlap the loads of steps kt+1 .. kt+S-1.
//
// LDS stage layout: 16-byte slots, A rows then B rows, 4 slots (64 bytes of
// K) per row; chunk c of row r sits in slot 4r + (c ^ ((r >> 2) & 3)).  The
// XOR swizzle makes the MFMA fragment reads (16 lanes = 16 consecutive rows,
// one chunk) hit 16 distinct 16-byte bank groups.  A DMA instruction writes
// 64 consecutive slots (lane i -> slot base + i), so each lane fetches the
// global chunk that the swizzle assigns to its slot.
//
// Zero fill: a lane whose row is past m (or n) or whose chunk is past k gets
// a buffer offset beyond the descriptor's range, for which the hardware
// returns zeros.
//
// Synchronisation per step kt: wait until this wave's loads of step kt are
// done (vmcnt = loads issued after them), s_barrier (every wave's loads of
// kt have landed, and every wave has finished reading step kt-1), issue step
// kt+S-1 into the slot step kt-1 used, then compute step kt.


template <int kPerWave, int kMaxAhead>
__device__ __forceinline__ void wait_ahead(int ahead) {
  // ahead in [0, kMaxAhead]: loads still allowed in flight = ahead*kPerWave
  if constexpr (kMaxAhead >= 4) { if (ahead >= 4) { wait_vmcnt<4 * kPerWave>(); return; } }
  if constexpr (kMaxAhead >= 3) { if (ahead == 3) { wait_vmcnt<3 * kPerWave>(); return; } }
  if constexpr (kMaxAhead >= 2) { if (ahead == 2) { wait_vmcnt<2 * kPerWave>(); return; } }
  if constexpr (kMaxAhead >= 1) { if (ahead == 1) { wait_vmcnt<kPerWave>(); return; } }
  wait_vmcnt<0>();
}

__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Split-K (SK): workgroup b computes the K stages [s nk / splits, (s + 1) nk /
// splits) of tile b % tiles, s = b / tiles.  Each writes its int32 partial
// tile to the workspace, waits for the writes to complete, and (after a
// barrier) counts itself in with one atomic add on the tile's counter; the
// workgroup that arrives last adds the other partials to its own, runs the
// epilogue and resets the counter for the next launch on the stream.
// Integer sums are exact, so the result is bit-identical to the unsplit
// kernel.  No workgroup ever waits for another.
struct SplitK {
  int splits;
  int *ws;   // [tiles][splits][kThreads * WM * WN * 16] int32
  int *cnt;  // [tiles], zero between launches
};

template <int WM, int WN, int S, int BKB, bool HEADS, bool SK>
__global__ __launch_bounds__(kThreads) void gemm_i8_dma_kernel(
    float *__restrict__ dst, int dstr, int hdim, GemmSegs bs, int mstr,
    const int8_t *__restrict__ src, int sstr, const float *__restrict__ ssc, int m, int k,
    SplitK sk) {
  constexpr int kBM = 64 * WM;
  constexpr int kBN = 64 * WN;
  constexpr int kC = BKB / 16;                 // 16-byte chunks per row and stage
  constexpr int kSlots = (kBM + kBN) * kC;
  constexpr int kPerWave = kSlots / 64 / 4;
  constexpr int kSub = BKB / 32;               // MFMA K sub-steps per stage
  static_assert(S >= 2 && S <= 6, "stages");
  static_assert(BKB == 64 || BKB == 128, "stage depth");
  __shared__ v4i lds[S][kSlots];

  // chunk c of row r lives in slot r*kC + (c ^ swz(r)): 16 consecutive rows
  // reading one chunk land in 16 distinct 16-byte bank groups
  auto swz = [](int r) { return kC == 4 ? ((r >> 2) & 3) : ((r >> 1) & 7); };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int n = bs.end[bs.nseg - 1];
  const int tiles_m = (m + kBM - 1) / kBM, tiles_n = (n + kBN - 1) / kBN;
  const int tile = SK ? (int)(blockIdx.x % (unsigned)(tiles_m * tiles_n)) : (int)blockIdx.x;
  const int sidx = SK ? (int)(blockIdx.x / (unsigned)(tiles_m * tiles_n)) : 0;
  int tm, tn;
  tile_of(tile, tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * kBM;
  const int n0 = tn * kBN;
  // the B matrix of this tile's columns (inner segment ends are multiples of
  // kBN, so a tile lies in one segment); its rows are columns c0 .. of dst
  int sj = 0;
#pragma unroll
  for (int t = 0; t < kMaxGemmSegs - 1; ++t)
    if (t + 1 < bs.nseg && n0 >= bs.end[t]) sj = t + 1;
  const int c0 = sj == 0 ? 0 : bs.end[sj - 1];
  const int8_t *mat = bs.w[sj];
  const int nb = bs.end[sj] - c0;
  TileScales<WM, WN> scales;
  load_tile_scales<WM, WN>(scales, ssc, bs.s[sj] - c0, m, n, m0, n0, wm, wn, lane);

  const __amdgpu_buffer_rsrc_t rs_a = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(src), (short)0, (int)((uint32_t)(m - 1) * sstr + k), 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_b = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(mat), (short)0, (int)((uint32_t)(nb - 1) * mstr + k), 0x00020000);

  // this lane's slot of each of its kPerWave DMA instructions
  uint32_t row_off[kPerWave];
  int chunk16[kPerWave];
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const int instr = wave * kPerWave + i;
    const bool is_a = instr * 64 < kBM * kC;  // wave-uniform
    const int slot = instr * 64 + lane - (is_a ? 0 : kBM * kC);
    const int row = slot / kC;
    const int chunk = (slot % kC) ^ swz(row);
    const int grow = (is_a ? m0 : n0 - c0) + row;
    const bool in = grow < (is_a ? m : nb);
    row_off[i] = in ? (uint32_t)grow * (uint32_t)(is_a ? sstr : mstr) + chunk * 16 : kOob;
    chunk16[i] = chunk * 16;
  }
  auto issue = [&](int kt, int buf) {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const int instr = wave * kPerWave + i;
      const bool is_a = instr * 64 < kBM * kC;
      const int kb = kt * BKB;
      const uint32_t voff =
          (row_off[i] == kOob || kb + chunk16[i] >= k) ? kOob : row_off[i] + kb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          is_a ? rs_a : rs_b,
          (__attribute__((address_space(3))) void *)&lds[buf][instr * 64], 16, voff, 0, 0, 0);
    }
  };

  v16i acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v16i{};

  const int nk_all = (k + BKB - 1) / BKB;
  const int kbeg = SK ? (int)((long)sidx * nk_all / sk.splits) : 0;
  const int nk = (SK ? (int)((long)(sidx + 1) * nk_all / sk.splits) : nk_all) - kbeg;
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < nk) issue(kbeg + st, st);

  const int frag_row = lane & 31;
  const int frag_chunk = lane >> 5;
  auto load_frags = [&](const v4i *stage, int ks, v4i (&a)[WM], v4i (&b)[WN]) {
    const int c = ks * 2 + frag_chunk;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int r = wm * 32 * WM + i * 32 + frag_row;
      a[i] = stage[r * kC + (c ^ swz(r))];
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int r = wn * 32 * WN + j * 32 + frag_row;
      b[j] = stage[kBM * kC + r * kC + (c ^ swz(r))];
    }
  };
  for (int kt = 0; kt < nk; ++kt) {
    const int ahead = min(S - 2, nk - 1 - kt);
    wait_ahead<kPerWave, S - 2>(ahead);
    block_barrier();
    if (kt + S - 1 < nk) issue(kbeg + kt + S - 1, (kt + S - 1) % S);
    const v4i *stage = lds[kt % S];
    // interleave the fragment reads with the MFMAs (the compiler's default
    // order issues the reads of sub-step ks+1 after the MFMAs of ks and
    // waits on them): 128x128 tiles measured +7% at gemma-3-4b down, +5% at
    // o, -2% at gate/up
    __builtin_amdgcn_iglp_opt(0);
    // fragments of sub-step ks+1 are read while the MFMAs of ks run
    v4i a[2][WM], b[2][WN];
    load_frags(stage, 0, a[0], b[0]);
#pragma unroll
    for (int ks = 0; ks < kSub; ++ks) {
      if (ks + 1 < kSub) load_frags(stage, ks + 1, a[(ks + 1) & 1], b[(ks + 1) & 1]);
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[ks & 1][i], b[ks & 1][j],
                                                            acc[i][j], 0, 0, 0);
    }
  }

  if constexpr (SK) {
    if (sk.splits > 1) {
      // Partials go out and come back in with device-coherent (agent-scope)
      // accesses, which write through and read past this XCD's L2; no cache
      // maintenance is needed, which matters: invalidating the L2 here would
      // also evict the operands of every other workgroup on the XCD.
      constexpr int kTileInts = kThreads * WM * WN * 16;
      int *mine = sk.ws + ((size_t)tile * sk.splits + sidx) * kTileInts;
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            __hip_atomic_store(mine + ((i * WN + j) * 16 + r) * kThreads + tid, acc[i][j][r],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __shared__ int last;
      wait_vmcnt<0>();  // this thread's partial has reached the coherence point
      __syncthreads();
      if (tid == 0) last = atomicAdd(sk.cnt + tile, 1) == sk.splits - 1;
      __syncthreads();
      if (!last) return;
      for (int o = 0; o < sk.splits; ++o) {
        if (o == sidx) continue;
        const int *other = sk.ws + ((size_t)tile * sk.splits + o) * kTileInts;
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              acc[i][j][r] += __hip_atomic_load(other + ((i * WN + j) * 16 + r) * kThreads + tid,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (tid == 0) sk.cnt[tile] = 0;
    }
  }
  // epilogue: rescale and store (gemma.c:3854-3865)
  store_tile<WM, WN, HEADS>(acc, scales, dst, dstr, hdim, m, n, m0, n0, wm, wn, lane);
}

// ---- ping-pong kernel (8 waves, one workgroup per CU) ----------------------
//
// Eight waves in two groups of four (waves 0-3 and 4-7; each SIMD runs one
// wave of each group).  Period p of the K loop is
//
//     group 0: [memory p] [compute p]       group 1: [compute p-1] [memory p]
//
// followed by one s_barrier, so on every SIMD one wave issues MFMAs while the
// other issues its LDS fragment reads and global->LDS DMA, and the two swap
// halfway through the period without a barrier in between (group 1 runs half
// a period behind in program order; its compute has the higher s_setprio so
// its MFMAs go first).  "memory p" issues the DMA of period p+D into the LDS
// ring, reads this group's fragments of period p and waits for them; each
// wave then waits until its own DMA of period p+1 has landed, and the barrier
// makes every wave's DMA of period p+1 visible (and frees the slots period p
// used) before anyone reads them.
//
// Two layouts of the eight waves:
//  - rows  (KALT = false): the groups split the tile's rows and consume the
//    same K stage each period (256x320 tiles: 2x2 waves of 64x160 per group);
//  - K-alternating (KALT = true): each group covers the whole tile with its
//    own 2x2 (or 4x1) waves and takes every other K stage (intra-workgroup
//    split-K); at the end the groups add their int32 sums through LDS, each
//    finishing half of the tile.  This doubles the MFMA work per period for
//    the 128-row tiles that give the one-tile-per-CU shapes exactly one round.
// Stages are 64 bytes of K for all BM+BN rows, XOR-swizzled as in the DMA
// kernel above; the tile's row and column scales come in by DMA with the
// first stages, so no registers carry them through the loop.  MF selects
// v_mfma_i32_32x32x32_i8 (32x32 tiles) or v_mfma_i32_16x16x64_i8 (16x16,
// for tile widths like 144 and 160 that are not multiples of 64).  Integer
// sums are exact, so every layout gives the same bits as the other kernels.

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// one 64-lane global->LDS DMA: lane i's 16 (or 4) bytes land at lds + 16 i
// (4 i); m0 carries the LDS address.  Issued from asm so that the compiler's
// own wait counting does not put a vmcnt(0) between the ring's DMA and the
// fragment reads of other slots (it cannot tell the slots apart); the
// kernel's explicit waits order them.
__device__ __forceinline__ void dma_b128(v4i rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(lds), "v"(voff), "s"(rsrc) : "memory", "m0");
}
__device__ __forceinline__ void dma_b32(v4i rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               ::"s"(lds), "v"(voff), "s"(rsrc) : "memory", "m0");
}
__device__ __forceinline__ v4i raw_rsrc(const void *base, uint32_t bytes) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  return v4i{(int)(uint32_t)b, (int)(uint32_t)((b >> 32) & 0xffffu), (int)bytes, 0x00020000};
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
__device__ __forceinline__ void pp_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
// at most a*P of this wave's DMA instructions outstanding, a in [0, A]
template <int P, int A>
__device__ __forceinline__ void wait_periods(int a) {
  if constexpr (A >= 2) { if (a >= 2) { wait_vmcnt<2 * P>(); return; } }
  if constexpr (A >= 1) { if (a == 1) { wait_vmcnt<P>(); return; } }
  wait_vmcnt<0>();
}

template <int MF> struct PpMfma;
template <> struct PpMfma<32> {
  typedef v16i Acc;
  static constexpr int NA = 16, NSUB = 2;  // accumulators per lane, MFMAs per stage
  static __device__ __forceinline__ Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  // 16-byte K chunk a lane supplies in sub-step sub
  static __device__ __forceinline__ int chunk(int sub, int lane) { return 2 * sub + (lane >> 5); }
  // accumulator r of lane l: row rsub(r) + rlane(l), column l % 32
  static __device__ __forceinline__ int rlane(int lane) { return 4 * (lane >> 5); }
  static constexpr int rsub(int r) { return 8 * (r >> 2) + (r & 3); }
};
template <> struct PpMfma<16> {
  typedef v4i Acc;
  static constexpr int NA = 4, NSUB = 1;
  static __device__ __forceinline__ Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int chunk(int, int lane) { return lane >> 4; }
  static __device__ __forceinline__ int rlane(int lane) { return 4 * (lane >> 4); }
  static constexpr int rsub(int r) { return r; }
};

template <int MF, int GWM, int GWN, int TM, int TN, bool KALT>
struct PpGeo {
  static constexpr int BM = (KALT ? 1 : 2) * GWM * TM * MF;
  static constexpr int BN = GWN * TN * MF;
};

// KS: 64-byte stages per group and period; D: periods of DMA lookahead
template <int MF, int GWM, int GWN, int TM, int TN, bool KALT, int KS, int D, bool HEADS>
__global__ __launch_bounds__(512, 1) void gemm_i8_pp_kernel(
    float *__restrict__ dst, int dstr, int hdim, GemmSegs bs, int mstr,
    const int8_t *__restrict__ src, int sstr, const float *__restrict__ ssc, int m, int k) {
  static_assert(GWM * GWN == 4, "four waves per group");
  typedef PpMfma<MF> M;
  typedef typename M::Acc Acc;
  constexpr int BM = PpGeo<MF, GWM, GWN, TM, TN, KALT>::BM;
  constexpr int BN = PpGeo<MF, GWM, GWN, TM, TN, KALT>::BN;
  constexpr int C = KALT ? 2 * KS : KS;   // stages per period
  constexpr int S = C * (D + 1);          // ring depth
  constexpr int kSlots = (BM + BN) * 4;   // 16-byte slots per stage
  constexpr int kInstr = kSlots / 64;     // DMA instructions per stage
  constexpr int kPer = (kInstr + 7) / 8;  // ... per wave (the last ones may be padding)
  constexpr int kScI = (BM + BN + 511) / 512;
  static_assert(C * kPer * (D - 1) <= 63, "vmcnt range");
  static_assert(S * kSlots * 16 + 1024 + kScI * 2048 <= 160 * 1024, "LDS");
  __shared__ v4i lds[S][kSlots];
  __shared__ v4i lpad[64];  // target of the padding DMAs (zeros, never read)
  __shared__ float lsc[kScI * 512];  // [0, BM) row scales, [BM, BM+BN) column scales

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, w4 = wave & 3;
  const int row_w = ((KALT ? 0 : grp * GWM) + w4 / GWN) * TM * MF;
  const int col_w = (w4 % GWN) * TN * MF;
  const int n = bs.end[bs.nseg - 1];
  int tm, tn;
  tile_of(blockIdx.x, (m + BM - 1) / BM, (n + BN - 1) / BN, &tm, &tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  // inner segment ends are multiples of BN: the tile's columns are in one segment
  int sj = 0;
#pragma unroll
  for (int t = 0; t < kMaxGemmSegs - 1; ++t)
    if (t + 1 < bs.nseg && n0 >= bs.end[t]) sj = t + 1;
  const int c0 = sj == 0 ? 0 : bs.end[sj - 1];
  const int nb = bs.end[sj] - c0;

  const v4i rs_a = raw_rsrc(src, (uint32_t)(m - 1) * sstr + k);
  const v4i rs_b = raw_rsrc(bs.w[sj], (uint32_t)(nb - 1) * mstr + k);
  const uint32_t ring = lds_addr(&lds[0][0]);
  const uint32_t pad = lds_addr(&lpad[0]);
  {
    const v4i rs_as = raw_rsrc(ssc, (uint32_t)m * 4);
    const v4i rs_bs = raw_rsrc(bs.s[sj], (uint32_t)nb * 4);
    const uint32_t sc = lds_addr(&lsc[0]);
#pragma unroll
    for (int u = 0; u < kScI; ++u) {
      const int base = u * 512 + wave * 64;  // wave-uniform; BM is a multiple of 64
      const int s = base + lane;
      if (base < BM) {
        dma_b32(rs_as, m0 + s < m ? (uint32_t)(m0 + s) * 4 : kOob, sc + base * 4);
      } else {
        const int col = n0 - c0 + s - BM;
        dma_b32(rs_bs, s - BM < BN && col < nb ? (uint32_t)col * 4 : kOob, sc + base * 4);
      }
    }
  }
  // this lane's slot in each of its DMA instructions
  uint32_t row_off[kPer];
  int chunk16[kPer];
  bool is_a[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int instr = i * 8 + wave;
    is_a[i] = instr * 64 < BM * 4;
    const int slot = instr * 64 + lane - (is_a[i] ? 0 : BM * 4);
    const int row = slot >> 2;
    const int chunk = (slot & 3) ^ ((row >> 2) & 3);
    const int grow = (is_a[i] ? m0 : n0 - c0) + row;
    const bool in = instr < kInstr && grow < (is_a[i] ? m : nb);
    row_off[i] = in ? (uint32_t)grow * (uint32_t)(is_a[i] ? sstr : mstr) + chunk * 16 : kOob;
    chunk16[i] = chunk * 16;
  }
  auto issue = [&](int kt) {
    const int buf = kt % S;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int instr = i * 8 + wave;
      const int kb = kt * 64;
      const uint32_t voff = (row_off[i] == kOob || kb + chunk16[i] >= k) ? kOob : row_off[i] + kb;
      dma_b128(is_a[i] ? rs_a : rs_b, voff,
               instr < kInstr ? ring + (uint32_t)((buf * kSlots + instr * 64) * 16) : pad);
    }
  };

  Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = Acc{};
  v4i fa[KS][M::NSUB][TM], fb[KS][M::NSUB][TN];
  auto read_frags = [&](int kt0) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const v4i *st = lds[(kt0 + s) % S];
#pragma unroll
      for (int sub = 0; sub < M::NSUB; ++sub) {
        const int c = M::chunk(sub, lane);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int r = row_w + i * MF + (lane % MF);
          fa[s][sub][i] = st[r * 4 + (c ^ ((r >> 2) & 3))];
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int r = col_w + j * MF + (lane % MF);
          fb[s][sub][j] = st[BM * 4 + r * 4 + (c ^ ((r >> 2) & 3))];
        }
      }
    }
  };
  auto compute = [&]() {
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int sub = 0; sub < M::NSUB; ++sub)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = M::mma(fa[s][sub][i], fb[s][sub][j], acc[i][j]);
  };

  const int nk = (k + 63) / 64;
  const int np = (nk + C - 1) / C;  // stages past nk read as zeros
  for (int p = 0; p < D && p < np; ++p)
#pragma unroll
    for (int c = 0; c < C; ++c) issue(p * C + c);
  wait_periods<C * kPer, D - 1>(min(D - 1, np - 1));  // period 0 (and the scales)
  pp_barrier();
  const int own = KALT ? grp * KS : 0;
  for (int p = 0; p < np; ++p) {
    if (grp == 1 && p > 0) {
      __builtin_amdgcn_s_setprio(2);
      compute();
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (p + D < np) {
#pragma unroll
      for (int c = 0; c < C; ++c) issue((p + D) * C + c);
    }
    read_frags(p * C + own);
    wait_lgkm0();
    __builtin_amdgcn_sched_barrier(0);
    if (grp == 0) {
      __builtin_amdgcn_s_setprio(1);
      compute();
      __builtin_amdgcn_s_setprio(0);
    }
    wait_periods<C * kPer, D - 1>(max(0, min(D - 1, np - 2 - p)));  // period p+1 landed
    pp_barrier();
  }
  if (grp == 1) compute();

  // The accumulator tiles [I0, I0+NI) x [J0, J0+NJ) this wave finishes:
  // all of them, or with KALT the half its group keeps after the exchange.
  constexpr bool kSplitI = TM % 2 == 0;
  static_assert(!KALT || kSplitI || TN % 2 == 0, "KALT halves the wave tile");
  constexpr int HI = KALT && kSplitI ? TM / 2 : TM;
  constexpr int HJ = KALT && !kSplitI ? TN / 2 : TN;
  static_assert(!KALT || 8 * HI * HJ * M::NA * 64 * 4 <= S * kSlots * 16, "exchange area");
  if constexpr (KALT) {
    // every ring read and DMA is complete (last wait was vmcnt(0), the reads
    // were waited before the last barrier): the ring is reused for the exchange
    int *xa = reinterpret_cast<int *>(&lds[0][0]);
    int *mine = xa + (wave * HI * HJ * M::NA) * 64;
    const int *theirs = xa + ((wave ^ 4) * HI * HJ * M::NA) * 64;
    auto put = [&](auto G) {
      constexpr int g = decltype(G)::value;
      constexpr int gi = kSplitI && g == 0 ? HI : 0, gj = !kSplitI && g == 0 ? HJ : 0;
#pragma unroll
      for (int i = 0; i < HI; ++i)
#pragma unroll
        for (int j = 0; j < HJ; ++j)
#pragma unroll
          for (int r = 0; r < M::NA; ++r)
            mine[((i * HJ + j) * M::NA + r) * 64 + lane] = acc[gi + i][gj + j][r];
    };
    auto take = [&](auto G) {
      constexpr int g = decltype(G)::value;
      constexpr int ki = kSplitI && g == 1 ? HI : 0, kj = !kSplitI && g == 1 ? HJ : 0;
#pragma unroll
      for (int i = 0; i < HI; ++i)
#pragma unroll
        for (int j = 0; j < HJ; ++j)
#pragma unroll
          for (int r = 0; r < M::NA; ++r)
            acc[ki + i][kj + j][r] += theirs[((i * HJ + j) * M::NA + r) * 64 + lane];
    };
    if (grp == 0) put(std::integral_constant<int, 0>{}); else put(std::integral_constant<int, 1>{});
    __syncthreads();
    if (grp == 0) take(std::integral_constant<int, 0>{}); else take(std::integral_constant<int, 1>{});
  }

  // epilogue (gemma.c:3854-3865): y = (float)acc * (act_scale * w_scale)
  auto finish = [&](auto I0c, auto J0c) {
    constexpr int I0 = decltype(I0c)::value, J0 = decltype(J0c)::value;
    float amin = __builtin_inff(), wmin = __builtin_inff();
    bool asub = false, wsub = false;
#pragma unroll
    for (int i = 0; i < HI; ++i)
#pragma unroll
      for (int r = 0; r < M::NA; ++r)
        scale_extremes(lsc[row_w + (I0 + i) * MF + M::rsub(r) + M::rlane(lane)], &amin, &asub);
#pragma unroll
    for (int j = 0; j < HJ; ++j)
      scale_extremes(lsc[BM + col_w + (J0 + j) * MF + (lane % MF)], &wmin, &wsub);
    const bool plain_lane = rescale_all_plain(amin, asub, wmin, wsub);
    const bool all_plain = __builtin_amdgcn_readfirstlane(__any(!plain_lane) ? 0 : 1) != 0;
    if (!HEADS && all_plain) {
      // out-of-range rows and columns fall past the descriptor and are dropped
      const uint32_t extent = ((uint32_t)(m - 1) * (uint32_t)dstr + (uint32_t)n) * 4u;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          dst, (short)0, (int)extent, 0x00020000);
#pragma unroll
      for (int j = 0; j < HJ; ++j) {
        const int cl = col_w + (J0 + j) * MF + (lane % MF);
        const float wsc = lsc[BM + cl];
        const uint32_t voff =
            n0 + cl < n ? ((uint32_t)M::rlane(lane) * dstr + n0 + cl) * 4u : kOob;
#pragma unroll
        for (int i = 0; i < HI; ++i)
#pragma unroll
          for (int r = 0; r < M::NA; ++r) {
            const int rl = row_w + (I0 + i) * MF + M::rsub(r);
            const float y = (float)acc[I0 + i][J0 + j][r] * (lsc[rl + M::rlane(lane)] * wsc);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), rs, voff,
                                                  (uint32_t)(m0 + rl) * dstr * 4u, 0);
          }
      }
      return;
    }
    // head-major layout, or scales in FTZ/DAZ territory: guarded stores
#pragma unroll
    for (int j = 0; j < HJ; ++j) {
      const int cl = col_w + (J0 + j) * MF + (lane % MF);
      const int col = n0 + cl;
      const float wsc = lsc[BM + cl];
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
      for (int i = 0; i < HI; ++i)
#pragma unroll
        for (int r = 0; r < M::NA; ++r) {
          const int rl = row_w + (I0 + i) * MF + M::rsub(r) + M::rlane(lane);
          const int32_t a = acc[I0 + i][J0 + j][r];
          const float y = all_plain ? (float)a * (lsc[rl] * wsc) : rescale(a, lsc[rl], wsc);
          if (m0 + rl < m && col < n) out_col[(size_t)(m0 + rl) * row_stride] = y;
        }
    }
  };
  constexpr int kKeepI = KALT && kSplitI ? HI : 0, kKeepJ = KALT && !kSplitI ? HJ : 0;
  if (KALT && grp == 1)
    finish(std::integral_constant<int, kKeepI>{}, std::integral_constant<int, kKeepJ>{});
  else
    finish(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
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

// Tile shape: GEMMA_HIP_GEMM_TILE=WMxWN (register-staged kernel), WMxWNxS
// (LDS-DMA kernel, S stages of 64-byte K) or WMxWNxSx128 (128-byte K stages)
// overrides the choice below (a launch-shape knob like the reference's
// GEMM_MC/GEMM_NC, gemma.c:458-493).
int env_tile() {
  static const int t = [] {
    const char *e = getenv("GEMMA_HIP_GEMM_TILE");
    if (e == nullptr) return 0;
    int a = 0, b = 0, c = 0, d = 0;
    const int got = sscanf(e, "%dx%dx%dx%d", &a, &b, &c, &d);
    if (got == 4) return a * 1000 + b * 100 + c * 10 + (d == 128 ? 1 : 0);
    if (got == 3) return a * 100 + b * 10 + c;
    if (got == 2) return a * 10 + b;
    return 0;
  }();
  return t;
}

// 2221 (128x128, two 128-byte stages) with a tile per CU, else 214 (128x64)
// with a tile per CU, else 114 (64x64)
int narrow_tile(int m, int n, const DeviceInfo &dev) {
  const long tiles128 = (long)((m + 127) / 128) * ((n + 127) / 128);
  const long tiles128x64 = (long)((m + 127) / 128) * ((n + 63) / 64);
  return tiles128 >= dev.cus ? 2221 : tiles128x64 >= dev.cus ? 214 : 114;
}


GemmSegs one_seg(const int8_t *mat, const float *matsc, int n) {
  GemmSegs bs{};
  bs.w[0] = mat;
  bs.s[0] = matsc;
  bs.end[0] = n;
  bs.nseg = 1;
  return bs;
}

// ---- ping-pong kernel: configurations and their choice ---------------------
//
// Measured on MI355X (random int8 operands, one launch at a time):
//   256x320 rows layout (2x2 waves of 64x160 per group, 32x32 MFMA): gemma-3-4b
//     gate/up 2048x10240x2560 60.5 us (DMA kernel 70.5), SigLIP fc1
//     4096x4304x1152 33.2 us (36.7);
//   128x160 K-alternating (2x2 waves of 64x80, 16x16 MFMA): 4b o 19.7 us
//     (20.4), 4b down 2048x2560x10240 70.3 us (71.5);
//   128x144 K-alternating (4x1 waves of 32x144): SigLIP q/k/v/o 14.4 us (14.9),
//     fc2 37.7 us (40.0);
//   128x128 K-alternating (2x2 waves of 64x64, 32x32 MFMA): 4b q 19.0 us (21.6);
//   128x64 K-alternating, two stages per group step: 4b k/v 13.9 us (18.0).
//   gemma-3-4b gate/up as one launch (2048x20480x2560, two rounds of 256x320):
//     111.6 us (132.5).
// A launch is worth it when the tiles fill at least 3/4 of the CUs in one
// round (two for 256x320); the cost model below (per round: a fixed 5.5 us
// of launch, prologue and drain, the tile's stores, and the K loop at the
// configuration's measured rate per CU) picks among the configurations whose
// tile width divides the segment ends.
struct PpConfig {
  int bm, bn;
  double tops_per_cu;  // K-loop rate per CU, TOPS
};
constexpr PpConfig kPpConfigs[] = {
    {0, 0, 0.0}, {256, 320, 8.45}, {128, 160, 6.6}, {128, 144, 5.0}, {128, 128, 6.0}, {128, 64, 4.0},
};
constexpr int kPpCount = 5;

// GEMMA_HIP_GEMM_PP=0 turns the ping-pong kernel off, 1..5 forces a
// configuration of kPpConfigs (a launch-shape knob like GEMMA_HIP_GEMM_TILE)
int env_pp() {
  const char *e = getenv("GEMMA_HIP_GEMM_PP");
  return e == nullptr ? -1 : atoi(e);
}

int choose_pp(int m, int n, int k, const GemmSegs &bs, const DeviceInfo &dev) {
  const int forced = env_pp();
  if (forced == 0) return 0;
  // a forced split-K (GEMMA_HIP_GEMM_SPLIT) asks for the split DMA kernel
  const char *split = getenv("GEMMA_HIP_GEMM_SPLIT");
  if (split != nullptr && atoi(split) > 0) return 0;
  int best = 0;
  double best_cost = 0.0;
  for (int id = 1; id <= kPpCount; ++id) {
    const PpConfig &c = kPpConfigs[id];
    bool aligned = true;
    for (int t = 0; t + 1 < bs.nseg; ++t) aligned = aligned && bs.end[t] % c.bn == 0;
    if (!aligned) continue;
    if (forced > 0) {
      if (id == forced) return id;
      continue;
    }
    const long tiles = (long)((m + c.bm - 1) / c.bm) * ((n + c.bn - 1) / c.bn);
    if (tiles * 4 < 3L * dev.cus) continue;
    const long rounds = (tiles + dev.cus - 1) / dev.cus;
    // one workgroup per CU pays its prologue and drain every round: past one
    // round (two for the 256x320 tiles) the DMA kernel, two workgroups per CU,
    // measured faster (gemma-3-4b q/k/v at 2048 tokens 29.0 us against 38.5
    // for 128x128 tiles in two rounds; gemma-3-1b gate/up at 512 tokens 16.4
    // against 21.1; SigLIP q/k/v 28.9 against 35.7)
    if (rounds > (id == 1 ? 2 : 1)) continue;
    const double area = (double)c.bm * c.bn;
    const double cost = rounds * (5.5 + 6e-5 * area + 2.0 * area * k / (c.tops_per_cu * 1e6));
    if (best == 0 || cost < best_cost) {
      best = id;
      best_cost = cost;
    }
  }
  return best;
}

template <int MF, int GWM, int GWN, int TM, int TN, bool KALT, int KS, int D>
void launch_pp_cfg(bool heads, hipStream_t stream, float *dst, int dstr, int hdim,
                   const GemmSegs &bs, int mstr, const int8_t *src, int sstr, const float *ssc,
                   int m, int k) {
  constexpr int BM = PpGeo<MF, GWM, GWN, TM, TN, KALT>::BM;
  constexpr int BN = PpGeo<MF, GWM, GWN, TM, TN, KALT>::BN;
  const int n = bs.end[bs.nseg - 1];
  const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  if (heads)
    gemm_i8_pp_kernel<MF, GWM, GWN, TM, TN, KALT, KS, D, true><<<tiles, 512, 0, stream>>>(
        dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k);
  else
    gemm_i8_pp_kernel<MF, GWM, GWN, TM, TN, KALT, KS, D, false><<<tiles, 512, 0, stream>>>(
        dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k);
}

void launch_pp(int id, bool heads, hipStream_t stream, float *dst, int dstr, int hdim,
               const GemmSegs &bs, int mstr, const int8_t *src, int sstr, const float *ssc, int m,
               int k) {
  switch (id) {
    case 1: launch_pp_cfg<32, 2, 2, 2, 5, false, 1, 2>(heads, stream, dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k); break;
    case 2: launch_pp_cfg<16, 2, 2, 4, 5, true, 1, 2>(heads, stream, dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k); break;
    case 3: launch_pp_cfg<16, 4, 1, 2, 9, true, 1, 2>(heads, stream, dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k); break;
    case 4: launch_pp_cfg<32, 2, 2, 2, 2, true, 1, 3>(heads, stream, dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k); break;
    default: launch_pp_cfg<16, 2, 2, 4, 2, true, 2, 2>(heads, stream, dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k); break;
  }
}

template <int WM, int WN, int S, int BKB = 64>
void launch_dma_segs(bool heads, hipStream_t stream, float *dst, int dstr, int hdim,
                     const GemmSegs &bs, int mstr, const int8_t *src, int sstr,
                     const float *ssc, int m, int k) {
  const int n = bs.end[bs.nseg - 1];
  const int tiles = ((m + 64 * WM - 1) / (64 * WM)) * ((n + 64 * WN - 1) / (64 * WN));
  const SplitK none{1, nullptr, nullptr};
  if (heads)
    gemm_i8_dma_kernel<WM, WN, S, BKB, true, false><<<tiles, kThreads, 0, stream>>>(
        dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k, none);
  else
    gemm_i8_dma_kernel<WM, WN, S, BKB, false, false><<<tiles, kThreads, 0, stream>>>(
        dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k, none);
}

// Split-K workspace and tile counters, one set per (device, stream): launches
// on one stream run in order, so they can share it.  Grown (never shrunk) on
// demand; the counters start at zero and every launch leaves them at zero.
struct SplitWs {
  int *ws = nullptr, *cnt = nullptr;
  size_t ws_ints = 0;
  int ncnt = 0;
};
std::mutex g_split_mu;
std::map<std::pair<int, hipStream_t>, SplitWs> g_split;

hipError_t split_ws(hipStream_t stream, size_t ws_ints, int ncnt, SplitK *sk) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_split_mu);
  SplitWs &w = g_split[{dev, stream}];
  if (w.ws_ints < ws_ints || w.ncnt < ncnt) {
    // launches already queued on the stream may still use the old buffers
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
    if (w.ws_ints < ws_ints) {
      if (w.ws != nullptr && (e = hipFree(w.ws)) != hipSuccess) return e;
      w.ws = nullptr;
      w.ws_ints = 0;
      if ((e = hipMalloc(&w.ws, ws_ints * sizeof(int))) != hipSuccess) return e;
      w.ws_ints = ws_ints;
    }
    if (w.ncnt < ncnt) {
      if (w.cnt != nullptr && (e = hipFree(w.cnt)) != hipSuccess) return e;
      w.cnt = nullptr;
      w.ncnt = 0;
      if ((e = hipMalloc(&w.cnt, ncnt * sizeof(int))) != hipSuccess) return e;
      if ((e = hipMemsetAsync(w.cnt, 0, ncnt * sizeof(int), stream)) != hipSuccess) return e;
      w.ncnt = ncnt;
    }
  }
  sk->ws = w.ws;
  sk->cnt = w.cnt;
  return hipSuccess;
}

}  // namespace

hipError_t split_workspace(hipStream_t stream, size_t ws_ints, int ncnt, int **ws, int **cnt) {
  SplitK sk{};
  const hipError_t e = split_ws(stream, ws_ints, ncnt, &sk);
  *ws = sk.ws;
  *cnt = sk.cnt;
  return e;
}

hipError_t gemm_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[device] != nullptr) return hipSuccess;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  g_scratch_dev[device] = static_cast<int *>(p);
  return hipSuccess;
}

GemmWs gemm_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (device < 0 || device >= kMaxDevices) return GemmWs{nullptr, 0};
  return GemmWs{g_scratch_dev[device], g_scratch_dev[device] ? kGemmScratchBytes : 0};
}

void release_gemm_workspaces() {
  std::lock_guard<std::mutex> lock(g_split_mu);
  for (auto &kv : g_split) {  // hipFree waits for the device's queued work
    if (kv.second.ws != nullptr) (void)hipFree(kv.second.ws);
    if (kv.second.cnt != nullptr) (void)hipFree(kv.second.cnt);
  }
  g_split.clear();
}

namespace {

// GEMMA_HIP_GEMM_SPLIT=s forces s-way split-K on the 128x128 kernel (a
// launch-shape knob like GEMMA_HIP_GEMM_TILE; read at every launch, so a
// process can change it); 0 or unset = the cost model.
int env_split() {
  const char *e = getenv("GEMMA_HIP_GEMM_SPLIT");
  return e == nullptr ? 0 : atoi(e);
}

// Counters of a caller-free workspace are cleared by a kernel (not
// hipMemsetAsync) on every call, so the call may be captured into a graph.
__global__ __launch_bounds__(kThreads) void gemm_zero_kernel(int *p, int n) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < n) p[i] = 0;
}

// A split-K launch: square tiles of 64 * wm (wm = 1: 64x64 tiles, four
// 64-byte K stages; wm = 2: 128x128, two 128-byte stages) in `splits` pieces
// (1 = no split).
struct SplitPlan {
  int wm = 2, splits = 1;
};

int split_tiles(int m, int n, int wm) {
  const int t = 64 * wm;
  return ((m + t - 1) / t) * ((n + t - 1) / t);
}

// int32 partial-tile elements of a split launch: kThreads * wm * wm * 16 per
// tile and piece
size_t split_part_ints(int tiles, int splits, int wm) {
  return (size_t)tiles * splits * kThreads * wm * wm * 16;
}

// Bytes of workspace a split-K launch needs: the partial tiles, then the
// tile counters on a 256-byte boundary.
size_t split_bytes(int tiles, int splits, int wm) {
  return split_part_ints(tiles, splits, wm) * sizeof(int) +
         (((size_t)tiles * sizeof(int) + 255) & ~(size_t)255);
}

// W x W blocks of 32x32 tiles per wave (64W x 64W workgroup tiles), S stages
// of BKB bytes, split-K over `splits` workgroups per tile (splits >= 2, at
// most the number of K stages).
template <int W, int S, int BKB>
hipError_t launch_dma_split(bool heads, hipStream_t stream, float *dst, int dstr, int hdim,
                            const GemmSegs &bs, int mstr, const int8_t *src, int sstr,
                            const float *ssc, int m, int k, int splits, const GemmWs *fixed) {
  const int n = bs.end[bs.nseg - 1];
  const int tiles = split_tiles(m, n, W);
  const size_t part = split_part_ints(tiles, splits, W);
  SplitK sk{splits, nullptr, nullptr};
  if (fixed != nullptr) {
    if (split_bytes(tiles, splits, W) > fixed->bytes) return hipErrorOutOfMemory;
    sk.ws = fixed->base;
    sk.cnt = fixed->base + ((part * sizeof(int) + 255) & ~(size_t)255) / sizeof(int);
    gemm_zero_kernel<<<(tiles + kThreads - 1) / kThreads, kThreads, 0, stream>>>(sk.cnt, tiles);
  } else {
    hipError_t e = split_ws(stream, part, tiles, &sk);
    if (e != hipSuccess) return e;
  }
  if (heads)
    gemm_i8_dma_kernel<W, W, S, BKB, true, true><<<tiles * splits, kThreads, 0, stream>>>(
        dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k, sk);
  else
    gemm_i8_dma_kernel<W, W, S, BKB, false, true><<<tiles * splits, kThreads, 0, stream>>>(
        dst, dstr, hdim, bs, mstr, src, sstr, ssc, m, k, sk);
  return hipGetLastError();
}

hipError_t launch_split(const SplitPlan &p, bool heads, hipStream_t stream, float *dst,
                        int dstr, int hdim, const GemmSegs &bs, int mstr, const int8_t *src,
                        int sstr, const float *ssc, int m, int k, const GemmWs *fixed) {
  return p.wm == 1 ? launch_dma_split<1, 4, 64>(heads, stream, dst, dstr, hdim, bs, mstr, src,
                                                sstr, ssc, m, k, p.splits, fixed)
                   : launch_dma_split<2, 2, 128>(heads, stream, dst, dstr, hdim, bs, mstr, src,
                                                 sstr, ssc, m, k, p.splits, fixed);
}

// The split-K plan (splits = 1: none).  Measured on MI355X, the partial
// tiles' round trip through memory costs about as much as 15 K stages, so a
// split pays only when the grid leaves CUs idle and K is long.  With fewer
// 64x64 tiles than CUs and K >= 2048, 64x64 tiles in about 1.5 workgroups per
// CU (at most 6 pieces of at least 8 stages): gemma-3-1b down at 512 tokens
// 23.3 -> 16.7 us (3 pieces; 128x128 tiles in 6 pieces: 23.3), at 256 tokens
// 20.5 -> 13.0, gemma-3-4b down at 256 tokens 26.9 -> 22.2.  Otherwise, with
// at most one 128x128 tile per two CUs and K >= 4096, 128x128 tiles in about
// two workgroups per CU (at most 8 pieces): gemma-3-1b down at 1024 tokens
// 28.6 -> 25.8 us, gemma-3-4b down at 512 tokens 40.7 -> 32.5.  Every
// gemma-3-4b and SigLIP shape at full length (>= 256 tiles of 128x128) lost
// 15-60% with forced splits.  GEMMA_HIP_GEMM_SPLIT forces 128x128 pieces.
SplitPlan choose_split(int m, int n, int k, const DeviceInfo &dev, hipStream_t stream,
                       bool fixed_ws) {
  SplitPlan p;
  const int nk128 = (k + 127) / 128, nk64 = (k + 63) / 64;
  const int forced = env_split();
  if (forced > 0) {
    p.splits = forced > nk128 ? nk128 : forced;
    return p;
  }
  const long tiles64 = split_tiles(m, n, 1), tiles128 = split_tiles(m, n, 2);
  if (tiles64 <= 0) return p;
  SplitPlan want;
  if (tiles64 < dev.cus && nk64 >= 32) {
    want.wm = 1;
    const long fill = (3L * dev.cus + 2 * tiles64 - 1) / (2 * tiles64);  // ~1.5 per CU
    want.splits = (int)std::min<long>({6, nk64 / 8, fill});
  } else if (tiles128 * 2 <= dev.cus && nk128 >= 32) {
    want.splits = (int)std::min<long>({8, 2L * dev.cus / tiles128, nk128 / 8});
  }
  if (want.splits < 2) return p;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (!fixed_ws &&
      (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone))
    return p;  // the workspace may have to be allocated: not under capture
  return want;
}

template <int WM, int WN, int S, int BKB = 64>
void launch_dma(bool heads, hipStream_t stream, float *dst, int dstr, int hdim,
                const int8_t *mat, int mstr, const float *matsc,
                const int8_t *src, int sstr, const float *ssc, int m, int n,
                int k) {
  GemmSegs bs{};
  bs.w[0] = mat;
  bs.s[0] = matsc;
  bs.end[0] = n;
  bs.nseg = 1;
  launch_dma_segs<WM, WN, S, BKB>(heads, stream, dst, dstr, hdim, bs, mstr, src, sstr, ssc, m,
                                  k);
}

template <int WM, int WN>
void launch_tiled(bool heads, hipStream_t stream, float *dst, int dstr, int hdim,
                  const int8_t *mat, int mstr, const float *matsc,
                  const int8_t *src, int sstr, const float *ssc, int m, int n,
                  int k) {
  const int tiles = ((m + 64 * WM - 1) / (64 * WM)) * ((n + 64 * WN - 1) / (64 * WN));
  if (heads)
    gemm_i8_kernel<WM, WN, true><<<tiles, kThreads, 0, stream>>>(
        dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k);
  else
    gemm_i8_kernel<WM, WN, false><<<tiles, kThreads, 0, stream>>>(
        dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k);
}

}  // namespace

size_t gemm_i8_scratch_bytes(int m, int n, int k, bool heads, const int8_t *mat, int mstr,
                             const int8_t *src, int sstr, int dstr, const DeviceInfo &dev) {
  const bool fast = k % 16 == 0 && mstr % 16 == 0 && sstr % 16 == 0 &&
                    (uintptr_t)mat % 16 == 0 && (uintptr_t)src % 16 == 0;
  const bool dma_ok = (uint64_t)(m - 1) * sstr + k < kOob &&
                      (uint64_t)(n - 1) * mstr + k < kOob &&
                      ((uint64_t)(m - 1) * dstr + n) * 4 < kOob;
  (void)heads;
  if (!fast || !dma_ok || env_tile() != 0) return 0;
  if (choose_pp(m, n, k, one_seg(mat, nullptr, n), dev) != 0) return 0;
  const SplitPlan sp = choose_split(m, n, k, dev, nullptr, true);
  return sp.splits > 1 ? split_bytes(split_tiles(m, n, sp.wm), sp.splits, sp.wm) : 0;
}

hipError_t launch_gemm_i8(float *dst, int dstr, int hdim, const int8_t *mat,
                          int mstr, const float *matsc, const int8_t *src,
                          int sstr, const float *ssc, int m, int n, int k,
                          const DeviceInfo &dev, hipStream_t stream, const GemmWs *fixed) {
  const bool fast = k % 16 == 0 && mstr % 16 == 0 && sstr % 16 == 0 &&
                    (uintptr_t)mat % 16 == 0 && (uintptr_t)src % 16 == 0;
  const bool heads = hdim > 0;
  // the DMA kernel addresses operands with 32-bit buffer offsets
  const bool dma_ok = (uint64_t)(m - 1) * sstr + k < kOob &&
                      (uint64_t)(n - 1) * mstr + k < kOob &&
                      ((uint64_t)(m - 1) * dstr + n) * 4 < kOob;
  if (fast) {
    int tile = env_tile();
    if (tile == 0 && dma_ok) {
      const GemmSegs one = one_seg(mat, matsc, n);
      const int pp = choose_pp(m, n, k, one, dev);
      if (pp != 0) {
        launch_pp(pp, heads, stream, dst, dstr, hdim, one, mstr, src, sstr, ssc, m, k);
        return hipGetLastError();
      }
      const SplitPlan sp = choose_split(m, n, k, dev, stream, fixed != nullptr);
      if (sp.splits > 1) {
        GemmSegs bs{};
        bs.w[0] = mat;
        bs.s[0] = matsc;
        bs.end[0] = n;
        bs.nseg = 1;
        const hipError_t e = launch_split(sp, heads, stream, dst, dstr, hdim, bs, mstr, src,
                                          sstr, ssc, m, k, fixed);
        return e != hipSuccess ? e : hipGetLastError();
      }
    }
    if (tile == 0) {
      // measured on MI355X at the 1b/4b prefill and SigLIP shapes: 128x128
      // tiles with two 128-byte K stages are fastest once there is a tile
      // per CU; below that, 128x64 tiles keep more CUs busy, and 64x64 tiles
      // where even those leave CUs idle (gemma-3-1b prefill o and q/k/v at
      // 512 tokens: 9.2 -> 7.6 us and 10.5 -> 9.1 us)
      tile = !dma_ok ? 22 : narrow_tile(m, n, dev);
    }
    if (tile >= 100 && !dma_ok) tile = 22;
    switch (tile) {
      case 224: launch_dma<2, 2, 4>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 223: launch_dma<2, 2, 3>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 226: launch_dma<2, 2, 6>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 424: launch_dma<4, 2, 4>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 244: launch_dma<2, 4, 4>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 2221: launch_dma<2, 2, 2, 128>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 2231: launch_dma<2, 2, 3, 128>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 4221: launch_dma<4, 2, 2, 128>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 114: launch_dma<1, 1, 4>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 214: launch_dma<2, 1, 4>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 11: launch_tiled<1, 1>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      case 21: launch_tiled<2, 1>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
      default: launch_tiled<2, 2>(heads, stream, dst, dstr, hdim, mat, mstr, matsc, src, sstr, ssc, m, n, k); break;
    }
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

hipError_t launch_gemm_i8_segs(float *dst, int dstr, const GemmSegs &b, const int8_t *src,
                               int sstr, const float *ssc, int m, int k, const DeviceInfo &dev,
                               hipStream_t stream) {
  if (b.nseg < 1 || b.nseg > kMaxGemmSegs || m <= 0 || k <= 0) return hipErrorInvalidValue;
  const int n = b.end[b.nseg - 1];
  bool fast = k % 16 == 0 && sstr % 16 == 0 && (uintptr_t)src % 16 == 0;
  bool dma_ok = (uint64_t)(m - 1) * sstr + k < kOob && ((uint64_t)(m - 1) * dstr + n) * 4 < kOob;
  for (int t = 0, start = 0; t < b.nseg; start = b.end[t], ++t) {
    const int rows = b.end[t] - start;
    if (rows <= 0) return hipErrorInvalidValue;
    fast = fast && (uintptr_t)b.w[t] % 16 == 0;
    dma_ok = dma_ok && (uint64_t)(rows - 1) * k + k < kOob;
  }
  if (fast && dma_ok && env_tile() == 0) {
    const int pp = choose_pp(m, n, k, b, dev);
    if (pp != 0) {
      launch_pp(pp, false, stream, dst, dstr, 0, b, k, src, sstr, ssc, m, k);
      return hipGetLastError();
    }
    // the tile choice of launch_gemm_i8 for the whole width
    const SplitPlan sp = choose_split(m, n, k, dev, stream, false);
    const int tile = sp.splits > 1 ? (sp.wm == 1 ? 114 : 2221) : narrow_tile(m, n, dev);
    const bool wide = tile == 2221;
    const int bn = wide ? 128 : 64;
    bool aligned = true;
    for (int t = 0; t + 1 < b.nseg; ++t) aligned = aligned && b.end[t] % bn == 0;
    if (aligned) {
      if (sp.splits > 1) {
        const hipError_t e =
            launch_split(sp, false, stream, dst, dstr, 0, b, k, src, sstr, ssc, m, k, nullptr);
        return e != hipSuccess ? e : hipGetLastError();
      }
      if (wide)
        launch_dma_segs<2, 2, 2, 128>(false, stream, dst, dstr, 0, b, k, src, sstr, ssc, m, k);
      else if (tile == 214)
        launch_dma_segs<2, 1, 4>(false, stream, dst, dstr, 0, b, k, src, sstr, ssc, m, k);
      else
        launch_dma_segs<1, 1, 4>(false, stream, dst, dstr, 0, b, k, src, sstr, ssc, m, k);
      return hipGetLastError();
    }
  }
  for (int t = 0, start = 0; t < b.nseg; start = b.end[t], ++t) {
    const hipError_t e = launch_gemm_i8(dst + start, dstr, 0, b.w[t], k, b.s[t], src, sstr, ssc,
                                        m, b.end[t] - start, k, dev, stream, nullptr);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace gh
