// gemv.hip -- decode GEMV (M = 1): int8 W8A8 (gemma.c:2754-2837 gemv_int8,
// gemv_int8_multi) and the fp32 fallback (gemma.c:2718-2752, 2839-2858
// gemv_fpx, gemv_fpx_multi).
//
// HBM-bound: every weight byte is read once, so the design is about keeping
// enough 128-bit loads in flight.  A 256-thread workgroup (4 waves) first
// stages the activation vector in LDS (quantizing it there when the caller
// hands over fp32), then each wave streams rows: L lanes share one row, each
// lane loading 16-byte chunks L chunks apart, so a wave covers 64/L rows per
// pass and every group of L lanes reads 16*L contiguous bytes.  int8 products
// use v_dot4 (4 multiply-adds per instruction) into an exact int32 sum; the
// L partial sums of a row are combined with cross-lane shuffles and lane 0
// of the group applies the rescale.  Workgroups loop over row blocks
// (grid <= 8 per CU) so the LDS staging is paid once per workgroup.
//
// Several weight matrices ("jobs": q/k/v or gate/up) are one flat row range,
// as in gemma.c:2803-2811, so a fused projection is one launch.
#include <cstdlib>
#include <type_traits>

#include "gh_arith.h"
#include "gh_kernels.h"

namespace gh {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ int job_of(const GemvJobs &jobs, int row,
                                      int *local) {
  int j = 0, start = 0;
#pragma unroll
  for (int t = 0; t < kMaxJobs - 1; ++t) {
    if (t + 1 < jobs.njobs && row >= jobs.end[t]) {
      j = t + 1;
      start = jobs.end[t];
    }
  }
  *local = row - start;
  return j;
}

__device__ __forceinline__ int32_t dot16(v4i w, v4i x, int32_t acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}

// The fused activation staging in two phases, for x that fits in
// registers (16-byte aligned, k % 4 == 0, k/4 <= kXRegs * NT): x_load issues
// the loads; x_quantize reduces amax, quantizes x into LDS as int8 and
// returns the scale (block 0 also stores xq_out / xs_out when given).
// Vector loads return in issue order, so a caller that issues its weight
// loads between the two phases does not delay the activation behind them.
constexpr int kXRegs = 4;

// Every load is issued (a chunk past k reloads chunk 0) and zeroed after it
// returns: a conditional load would make the compiler's wait counts wait
// for it, and for everything issued before it, at its first use.
template <int NT>
__device__ __forceinline__ void x_load(int k, const float *__restrict__ xf, v4f (&xr)[kXRegs]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < kXRegs; ++j) {
    const int c = tid + j * NT;
    xr[j] = reinterpret_cast<const v4f *>(xf)[c < k / 4 ? c : 0];
  }
#pragma unroll
  for (int j = 0; j < kXRegs; ++j)
    if (tid + j * NT >= k / 4) xr[j] = v4f{0.f, 0.f, 0.f, 0.f};
}

template <int NT>
__device__ __forceinline__ float x_quantize(int8_t *lds, int k, const v4f (&xr)[kXRegs],
                                            int8_t *__restrict__ xq_out,
                                            float *__restrict__ xs_out) {
  __shared__ float wave_amax[NT / 64];
  const int tid = threadIdx.x;
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < kXRegs; ++j)
    amax = fmaxf(amax, fmaxf(fmaxf(abs_daz(xr[j].x), abs_daz(xr[j].y)),
                             fmaxf(abs_daz(xr[j].z), abs_daz(xr[j].w))));
  amax = wave_max_dpp(amax);
  if ((tid & 63) == 0) wave_amax[tid >> 6] = amax;
  lds_barrier();
  amax = wave_amax[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) amax = fmaxf(amax, wave_amax[w]);
  const QuantParams qp = quant_params(amax);
#pragma unroll
  for (int j = 0; j < kXRegs; ++j) {
    const int c = tid + j * NT;
    if (c < k / 4)
      reinterpret_cast<uint32_t *>(lds)[c] =
          pack4(quant_one(xr[j].x, qp.inv), quant_one(xr[j].y, qp.inv),
                quant_one(xr[j].z, qp.inv), quant_one(xr[j].w, qp.inv));
  }
  lds_barrier();
  if (blockIdx.x == 0) {
    if (xq_out != nullptr)
      for (int c = tid; c < k; c += NT) xq_out[c] = lds[c];
    if (xs_out != nullptr && tid == 0) *xs_out = qp.scale;
  }
  return qp.scale;
}

// Stage the activation vector in LDS as int8.  FUSED: quantize x fp32 [k]
// (the quantize_act that precedes every decode GEMV); otherwise copy xq.
// Returns the activation scale.
template <bool FUSED, int NT = kThreads>
__device__ __forceinline__ float stage_x_i8(int8_t *lds, int k,
                                            const int8_t *__restrict__ xq,
                                            const float *__restrict__ xs,
                                            const float *__restrict__ xf,
                                            int8_t *__restrict__ xq_out,
                                            float *__restrict__ xs_out) {
  const int tid = threadIdx.x;
  if (!FUSED) {
    if (((uintptr_t)xq & 15) == 0 && (k & 15) == 0) {
      for (int c = tid; c < k / 16; c += NT)
        reinterpret_cast<v4i *>(lds)[c] =
            reinterpret_cast<const v4i *>(xq)[c];
    } else {
      for (int c = tid; c < k; c += NT) lds[c] = xq[c];
    }
    lds_barrier();
    return *xs;
  }
  const bool vec = ((uintptr_t)xf & 15) == 0 && (k & 3) == 0;
  if (vec && k / 4 <= kXRegs * NT) {
    v4f xr[kXRegs];
    x_load<NT>(k, xf, xr);
    return x_quantize<NT>(lds, k, xr, xq_out, xs_out);
  }
  // long or unaligned rows: two passes over x (the second from L2)
  __shared__ float wave_amax[NT / 64];
  float amax = 0.0f;
  if (vec) {
    for (int c = tid; c < k / 4; c += NT) {
      v4f v = reinterpret_cast<const v4f *>(xf)[c];
      amax = fmaxf(amax, fmaxf(fmaxf(abs_daz(v.x), abs_daz(v.y)),
                               fmaxf(abs_daz(v.z), abs_daz(v.w))));
    }
  } else {
    for (int c = tid; c < k; c += NT) amax = fmaxf(amax, abs_daz(xf[c]));
  }
  amax = wave_max_dpp(amax);
  if ((tid & 63) == 0) wave_amax[tid >> 6] = amax;
  lds_barrier();
  amax = wave_amax[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) amax = fmaxf(amax, wave_amax[w]);
  const QuantParams qp = quant_params(amax);
  if (vec) {
    for (int c = tid; c < k / 4; c += NT) {
      v4f v = reinterpret_cast<const v4f *>(xf)[c];
      reinterpret_cast<uint32_t *>(lds)[c] =
          pack4(quant_one(v.x, qp.inv), quant_one(v.y, qp.inv),
                quant_one(v.z, qp.inv), quant_one(v.w, qp.inv));
    }
  } else {
    for (int c = tid; c < k; c += NT)
      lds[c] = (int8_t)quant_one(xf[c], qp.inv);
  }
  lds_barrier();
  if (blockIdx.x == 0) {
    if (xq_out != nullptr)
      for (int c = tid; c < k; c += NT) xq_out[c] = lds[c];
    if (xs_out != nullptr && tid == 0) *xs_out = qp.scale;
  }
  return qp.scale;
}

// VEC: every job's rows start 16-byte aligned and k % 16 == 0.
template <int L, bool FUSED, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_i8_kernel(
    GemvJobs jobs, int total, int k, const int8_t *__restrict__ xq,
    const float *__restrict__ xs, const float *__restrict__ xf,
    int8_t *__restrict__ xq_out, float *__restrict__ xs_out) {
  extern __shared__ v4i lds_x4[];
  int8_t *lds_x = reinterpret_cast<int8_t *>(lds_x4);
  const float act_scale =
      stage_x_i8<FUSED>(lds_x, k, xq, xs, xf, xq_out, xs_out);

  constexpr int kRowsPerWave = 64 / L;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % L;
  const int rloc = lane / L;
  const int stride = gridDim.x * kWaves * kRowsPerWave;

  for (int base = (blockIdx.x * kWaves + wave) * kRowsPerWave; base < total;
       base += stride) {
    const int row = base + rloc;
    int32_t acc = 0;
    int j = 0, r = 0;
    if (row < total) {
      j = job_of(jobs, row, &r);
      const int8_t *w = static_cast<const int8_t *>(pick4(jobs.w, j));
      if (VEC) {
        const int kc = k >> 4;
        const v4i *w4 = reinterpret_cast<const v4i *>(w) + (size_t)r * kc;
#pragma unroll 4
        for (int c = sub; c < kc; c += L)
          acc = dot16(__builtin_nontemporal_load(w4 + c), lds_x4[c], acc);
      } else {
        const int8_t *wr = w + (size_t)r * k;
        for (int c = sub; c < k; c += L)
          acc += (int32_t)wr[c] * (int32_t)lds_x[c];
      }
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (sub == 0 && row < total)
      pick4(jobs.dst, j)[r] = rescale(acc, act_scale, pick4(jobs.sc, j)[r]);
  }
}

// Latency-oriented variant (VEC layout only): each lane owns at most CPL
// 16-byte chunks of its row, L = 64 / RPW lanes per row.  A lane issues the
// loads of its first row (weights, then its scale) before the activation is
// staged, so HBM latency overlaps the quantize prologue.  When the grid
// covers every row in one pass (the launch shapes this kernel is chosen
// for) that is all; otherwise each pass loads the next row before it
// reduces the current one (register double buffering).
// Weight loads are issued unconditionally (a row past the end reads the
// wave's own first row, or the last row, and is not used): the compiler's
// wait counts merge the paths of a conditional load by the path without it,
// which would make the prologue wait for the weights issued before it.
template <int L, int CPL, bool FUSED, int NT>
__global__ __launch_bounds__(NT) void gemv_i8_pipelined_kernel(
    GemvJobs jobs, int total, int k, const int8_t *__restrict__ xq,
    const float *__restrict__ xs, const float *__restrict__ xf,
    int8_t *__restrict__ xq_out, float *__restrict__ xs_out) {
  extern __shared__ v4i lds_x4[];
  hold_jobs(jobs);
  asm volatile("" ::"s"(k), "s"(xq), "s"(xs), "s"(xf), "s"(xq_out), "s"(xs_out));
  constexpr int kRowsPerWave = 64 / L;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane % L;
  const int rloc = lane / L;
  const int kc = k >> 4;
  constexpr int kBlockWaves = NT / 64;
  const int stride = gridDim.x * kBlockWaves * kRowsPerWave;
  const int base0 = (blockIdx.x * kBlockWaves + wave) * kRowsPerWave;  // wave-uniform
  const int own = base0 + rloc < total ? base0 + rloc : total - 1;

  struct Row {
    v4i w[CPL];
    float sc;
  };
  auto load_row = [&](int row, Row &buf) {
    int r;
    const int j = job_of(jobs, row < total ? row : own, &r);
    const gptr<const v4i> w4 =
        as_global(static_cast<const v4i *>(pick4(jobs.w, j))) + (size_t)r * kc;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;
      buf.w[i] = __builtin_nontemporal_load(w4 + (c < kc ? c : 0));
    }
    buf.sc = as_global(pick4(jobs.sc, j))[r];
  };

  Row cur;
  float act_scale;
  if (FUSED && ((uintptr_t)xf & 15) == 0 && (k & 3) == 0 && k / 4 <= kXRegs * NT) {
    // activation loads first, then the first weight row, then the quantize
    v4f xr[kXRegs];
    x_load<NT>(k, xf, xr);
    load_row(base0 + rloc, cur);
    act_scale = x_quantize<NT>(reinterpret_cast<int8_t *>(lds_x4), k, xr, xq_out, xs_out);
  } else {
    load_row(base0 + rloc, cur);
    act_scale = stage_x_i8<FUSED, NT>(reinterpret_cast<int8_t *>(lds_x4), k, xq, xs, xf, xq_out,
                                      xs_out);
  }

  auto process = [&](int base, const Row &w) {
    const int row = base + rloc;
    int32_t acc = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;
      if (c < kc) acc = dot16(w.w[i], lds_x4[c], acc);
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (sub == 0 && row < total) {
      int r;
      const int j = job_of(jobs, row, &r);
      as_global(pick4(jobs.dst, j))[r] = rescale(acc, act_scale, w.sc);
    }
  };
  if (total <= stride) {  // one pass: every row was loaded above
    if (base0 < total) process(base0, cur);
    return;
  }
  for (int base = base0; base < total; base += stride) {
    Row nxt;
    load_row(base + stride + rloc, nxt);
    process(base, cur);
    cur = nxt;
  }
}

// Streaming variant for long row ranges (VEC layout only).  Rows are taken
// in groups of R = 64 / L consecutive rows of one job, so the job, and with
// it every base pointer, is wave-uniform; groups are dealt to the waves of
// an all-resident grid round robin.  Each wave keeps D groups in flight in
// registers: it loads group i + D, then reduces group i.  Loads are raw
// buffer loads: a row past its job's end, a chunk past k and a group past
// the last are given an offset beyond the buffer, which returns zeros
// without touching memory, so every load is issued unconditionally and the
// waits stay exact.  Requires every job's m * k < 2^31.
constexpr uint32_t kOutOfRange = 0x80000000u;
// cache policy of the weight loads: nontemporal (each weight byte is read
// once per launch)
constexpr int kStreamPolicy = 2;

template <int L, int CPL, int D, bool FUSED, int NT>
__global__ __launch_bounds__(NT) void gemv_i8_stream_kernel(
    GemvJobs jobs, int ngroups, int k, const int8_t *__restrict__ xq,
    const float *__restrict__ xs, const float *__restrict__ xf,
    int8_t *__restrict__ xq_out, float *__restrict__ xs_out) {
  extern __shared__ v4i lds_x4[];
  hold_jobs(jobs);
  asm volatile("" ::"s"(ngroups), "s"(k), "s"(xq), "s"(xs), "s"(xf), "s"(xq_out), "s"(xs_out));
  constexpr int R = 64 / L;
  constexpr int kBlockWaves = NT / 64;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane % L;
  const int rloc = lane / L;
  const int kc = k >> 4;
  const int nwaves = gridDim.x * kBlockWaves;
  const int w0 = blockIdx.x * kBlockWaves + wave;

  // first group of each job (scalar)
  int gend[kMaxJobs];
  {
    int prev = 0, g = 0;
#pragma unroll
    for (int t = 0; t < kMaxJobs; ++t) {
      if (t < jobs.njobs) g += (jobs.end[t] - prev + R - 1) / R;
      gend[t] = g;
      prev = jobs.end[t];
    }
  }
  struct Where {
    int job, row, m;  // row within the job (per lane), rows of the job
  };
  auto where = [&](int g) {
    int j = 0, gs = 0, rs = 0;
#pragma unroll
    for (int t = 0; t < kMaxJobs - 1; ++t)
      if (t + 1 < jobs.njobs && g >= gend[t]) {
        j = t + 1;
        gs = gend[t];
        rs = jobs.end[t];
      }
    return Where{j, (g - gs) * R + rloc, pick4(jobs.end, j) - rs};
  };
  auto pick_s = [&](auto const (&a)[kMaxJobs], int j) {  // j is wave-uniform
    auto v = a[0];
#pragma unroll
    for (int t = 1; t < kMaxJobs; ++t)
      if (j == t) v = a[t];
    return v;
  };

  struct Slot {
    v4i w[CPL];
    int32_t sc;
  };
  auto load = [&](int g, Slot &s) {
    const Where at = where(g);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(pick_s(jobs.w, at.job)), (short)0, at.m * k, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(pick_s(jobs.sc, at.job)), (short)0, at.m * 4, 0x00020000);
    const bool ok = g < ngroups && at.row < at.m;
    const uint32_t row_off = ok ? (uint32_t)at.row * (uint32_t)k : kOutOfRange;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;
      s.w[i] = __builtin_amdgcn_raw_buffer_load_b128(
          rw, c < kc ? row_off + (uint32_t)c * 16u : kOutOfRange, 0, kStreamPolicy);
    }
    s.sc = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (uint32_t)at.row * 4u : kOutOfRange, 0,
                                                0);
  };

  Slot ring[D];
  float act_scale;
  if (FUSED && ((uintptr_t)xf & 15) == 0 && (k & 3) == 0 && k / 4 <= kXRegs * NT) {
    // activation loads first, then the first D groups, then the quantize
    v4f xr[kXRegs];
    x_load<NT>(k, xf, xr);
#pragma unroll
    for (int d = 0; d < D; ++d) load(w0 + d * nwaves, ring[d]);
    act_scale = x_quantize<NT>(reinterpret_cast<int8_t *>(lds_x4), k, xr, xq_out, xs_out);
  } else {
#pragma unroll
    for (int d = 0; d < D; ++d) load(w0 + d * nwaves, ring[d]);
    act_scale = stage_x_i8<FUSED, NT>(reinterpret_cast<int8_t *>(lds_x4), k, xq, xs, xf, xq_out,
                                      xs_out);
  }

  auto process = [&](int g, const Slot &s) {
    int32_t acc = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;  // chunks past k hold zeros
      acc = dot16(s.w[i], lds_x4[c < kc ? c : 0], acc);
    }
    acc = group_sum_i32<L>(acc);
    const Where at = where(g);
    if (sub == 0 && g < ngroups && at.row < at.m)
      pick_s(jobs.dst, at.job)[at.row] = rescale(acc, act_scale, __int_as_float(s.sc));
  };
  // groups of this wave: w0, w0 + nwaves, ...
  const int mine = w0 < ngroups ? (ngroups - 1 - w0) / nwaves + 1 : 0;
  for (int i = 0; i < mine; i += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int g = w0 + (i + d) * nwaves;
      process(g, ring[d]);
      load(g + D * nwaves, ring[d]);
    }
  }
}

template <int L, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_f32_kernel(
    GemvJobs jobs, int total, int k, const float *__restrict__ x) {
  extern __shared__ v4f lds_f4[];
  float *lds_f = reinterpret_cast<float *>(lds_f4);
  for (int c = threadIdx.x; c < k; c += kThreads) lds_f[c] = x[c];
  lds_barrier();

  constexpr int kRowsPerWave = 64 / L;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % L;
  const int rloc = lane / L;
  const int stride = gridDim.x * kWaves * kRowsPerWave;

  for (int base = (blockIdx.x * kWaves + wave) * kRowsPerWave; base < total;
       base += stride) {
    const int row = base + rloc;
    float acc = 0.0f;
    int j = 0, r = 0;
    if (row < total) {
      j = job_of(jobs, row, &r);
      const float *w = static_cast<const float *>(pick4(jobs.w, j));
      if (VEC) {
        const int kc = k >> 2;
        const v4f *w4 = reinterpret_cast<const v4f *>(w) + (size_t)r * kc;
#pragma unroll 4
        for (int c = sub; c < kc; c += L) {
          v4f wv = __builtin_nontemporal_load(w4 + c);
          v4f xv = lds_f4[c];
          acc = __builtin_fmaf(wv.x, xv.x, acc);
          acc = __builtin_fmaf(wv.y, xv.y, acc);
          acc = __builtin_fmaf(wv.z, xv.z, acc);
          acc = __builtin_fmaf(wv.w, xv.w, acc);
        }
      } else {
        const float *wr = w + (size_t)r * k;
        for (int c = sub; c < k; c += L)
          acc = __builtin_fmaf(wr[c], lds_f[c], acc);
      }
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (sub == 0 && row < total) pick4(jobs.dst, j)[r] = acc;
  }
}

// fp32 GEMV on the streaming schedule of gemv_i8_stream_kernel (gemv_fpx,
// gemma.c:2730-2752, and gemv_fpx_multi, 2839-2858): groups of R = 64 / L
// consecutive rows of one job dealt round robin to an all-resident grid, raw
// buffer loads whose out-of-range offsets return zeros (rows past a job's
// end, chunks past k, groups past the last), nontemporal weight loads.  A
// row of k floats is kc = k / 4 chunks of 16 bytes; lane `sub` of a row
// takes chunks sub, sub + L, ... in PASSES passes of CPL chunks.  x is
// staged in LDS as fp32.  The sum is fp32 FMAs in two chains per lane, then
// a fixed tree over the L lanes (the reference's order is its compiler's;
// the bound is the fp32 tolerance).  Requires every job's m * k * 4 < 2^31.
template <int L, int CPL, int NT>
__global__ __launch_bounds__(NT) void gemv_f32_stream_kernel(GemvJobs jobs, int ngroups, int k,
                                                             int passes,
                                                             const float *__restrict__ x) {
  extern __shared__ v4f lds_f4[];
  constexpr int R = 64 / L;
  constexpr int kBlockWaves = NT / 64;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane % L;
  const int rloc = lane / L;
  const int kc = k >> 2;
  const int nwaves = gridDim.x * kBlockWaves;
  const int w0 = blockIdx.x * kBlockWaves + wave;

  int gend[kMaxJobs];
  {
    int prev = 0, g = 0;
#pragma unroll
    for (int t = 0; t < kMaxJobs; ++t) {
      if (t < jobs.njobs) g += (jobs.end[t] - prev + R - 1) / R;
      gend[t] = g;
      prev = jobs.end[t];
    }
  }
  struct Where {
    int job, row, m;
  };
  auto where = [&](int g) {
    int j = 0, gs = 0, rs = 0;
#pragma unroll
    for (int t = 0; t < kMaxJobs - 1; ++t)
      if (t + 1 < jobs.njobs && g >= gend[t]) {
        j = t + 1;
        gs = gend[t];
        rs = jobs.end[t];
      }
    return Where{j, (g - gs) * R + rloc, pick4(jobs.end, j) - rs};
  };
  auto pick_s = [&](auto const (&a)[kMaxJobs], int j) {  // j is wave-uniform
    auto v = a[0];
#pragma unroll
    for (int t = 1; t < kMaxJobs; ++t)
      if (j == t) v = a[t];
    return v;
  };
  struct Slot {
    v4f w[CPL];
  };
  auto load = [&](int g, int pass, Slot &s) {
    const Where at = where(g);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(pick_s(jobs.w, at.job)), (short)0, at.m * k * 4, 0x00020000);
    const bool ok = g < ngroups && at.row < at.m;
    const uint32_t row_off = ok ? (uint32_t)at.row * (uint32_t)k * 4u : kOutOfRange;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + (pass * CPL + i) * L;
      s.w[i] = __builtin_bit_cast(
          v4f, __builtin_amdgcn_raw_buffer_load_b128(
                   rw, c < kc ? row_off + (uint32_t)c * 16u : kOutOfRange, 0, kStreamPolicy));
    }
  };

  // work items t = (group i = t / passes of this wave, pass t % passes); the
  // loads of item t+1 are in flight while item t is summed
  const int mine = w0 < ngroups ? (ngroups - 1 - w0) / nwaves + 1 : 0;
  const int items = mine * passes;
  auto item_load = [&](int t, Slot &s) { load(w0 + (t / passes) * nwaves, t % passes, s); };
  Slot buf0, buf1;
  item_load(0, buf0);
  for (int c = threadIdx.x; c < kc; c += NT) lds_f4[c] = reinterpret_cast<const v4f *>(x)[c];
  lds_barrier();

  float a0 = 0.0f, a1 = 0.0f;
  auto item_sum = [&](int t, const Slot &s) {
    const int pass = t % passes;
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      const int c = sub + (pass * CPL + u) * L;  // chunks past k hold zeros
      const v4f xv = lds_f4[c < kc ? c : 0];
      a0 = __builtin_fmaf(s.w[u].x, xv.x, a0);
      a1 = __builtin_fmaf(s.w[u].y, xv.y, a1);
      a0 = __builtin_fmaf(s.w[u].z, xv.z, a0);
      a1 = __builtin_fmaf(s.w[u].w, xv.w, a1);
    }
    if (pass == passes - 1) {
      const int g = w0 + (t / passes) * nwaves;
      const float acc = group_sum_f32<L>(a0 + a1);
      const Where at = where(g);
      if (sub == 0 && g < ngroups && at.row < at.m) pick_s(jobs.dst, at.job)[at.row] = acc;
      a0 = 0.0f;
      a1 = 0.0f;
    }
  };
  for (int t = 0; t < items; t += 2) {
    item_load(t + 1, buf1);
    item_sum(t, buf0);
    if (t + 1 < items) {
      item_load(t + 2, buf0);
      item_sum(t + 1, buf1);
    }
  }
}

// Lanes per row: the widest L whose chunks divide evenly with >= 4 chunks per
// lane, else 8.
int lanes_for(int chunks) {
  for (int lanes = 64; lanes >= 8; lanes >>= 1)
    if (chunks % lanes == 0 && chunks / lanes >= 4) return lanes;
  return 8;
}

int grid_for(int total, int lanes, const DeviceInfo &dev) {
  const int rows_per_block = kWaves * (64 / lanes);
  long blocks = (total + rows_per_block - 1) / rows_per_block;
  long cap = (long)dev.cus * 8;
  return (int)(blocks < cap ? blocks : cap);
}

bool rows_aligned(const GemvJobs &jobs, int k, int elem_bytes, int chunk) {
  if (((long)k * elem_bytes) % chunk != 0) return false;
  for (int j = 0; j < jobs.njobs; ++j)
    if ((uintptr_t)jobs.w[j] % chunk != 0) return false;
  return true;
}

template <bool FUSED, bool VEC>
hipError_t gemv_i8_dispatch(int lanes, dim3 grid, size_t lds,
                            hipStream_t stream, const GemvJobs &jobs,
                            int total, int k, const int8_t *xq,
                            const float *xs, const float *xf, int8_t *xq_out,
                            float *xs_out) {
  switch (lanes) {
    case 64:
      gemv_i8_kernel<64, FUSED, VEC><<<grid, kThreads, lds, stream>>>(
          jobs, total, k, xq, xs, xf, xq_out, xs_out);
      break;
    case 32:
      gemv_i8_kernel<32, FUSED, VEC><<<grid, kThreads, lds, stream>>>(
          jobs, total, k, xq, xs, xf, xq_out, xs_out);
      break;
    case 16:
      gemv_i8_kernel<16, FUSED, VEC><<<grid, kThreads, lds, stream>>>(
          jobs, total, k, xq, xs, xf, xq_out, xs_out);
      break;
    default:
      gemv_i8_kernel<8, FUSED, VEC><<<grid, kThreads, lds, stream>>>(
          jobs, total, k, xq, xs, xf, xq_out, xs_out);
      break;
  }
  return hipGetLastError();
}

template <bool VEC>
hipError_t gemv_f32_dispatch(int lanes, dim3 grid, size_t lds,
                             hipStream_t stream, const GemvJobs &jobs,
                             int total, int k, const float *x) {
  switch (lanes) {
    case 64:
      gemv_f32_kernel<64, VEC><<<grid, kThreads, lds, stream>>>(jobs, total, k, x);
      break;
    case 32:
      gemv_f32_kernel<32, VEC><<<grid, kThreads, lds, stream>>>(jobs, total, k, x);
      break;
    case 16:
      gemv_f32_kernel<16, VEC><<<grid, kThreads, lds, stream>>>(jobs, total, k, x);
      break;
    default:
      gemv_f32_kernel<8, VEC><<<grid, kThreads, lds, stream>>>(jobs, total, k, x);
      break;
  }
  return hipGetLastError();
}

// Launch-shape knobs, read once from the environment (the reference tunes
// its CPU GEMM blocking the same way, GEMM_MC/NC/KC, gemma.c:458-493):
//   GEMMA_HIP_GEMV_LANES         lanes per row of the pipelined GEMV (8..64)
//   GEMMA_HIP_GEMV_BLOCKS_PER_CU workgroups per CU of the pipelined GEMV (a
//                                cap below the occupancy for the streaming one)
//   GEMMA_HIP_GEMV_LOOP=1        use the looping GEMV kernel instead
//   GEMMA_HIP_GEMV_THREADS       256 or 1024 threads per pipelined workgroup
struct Tuning {
  int lanes = 0;
  int blocks_per_cu = 0;  // 0: 8 for 256-thread, 2 for 1024-thread workgroups
  int threads = 0;        // 0: chosen per shape
  bool force_loop = false;
};

const Tuning &tuning() {
  static const Tuning t = [] {
    Tuning v;
    if (const char *e = getenv("GEMMA_HIP_GEMV_LANES")) {
      const int l = atoi(e);
      if (l == 8 || l == 16 || l == 32 || l == 64) v.lanes = l;
    }
    if (const char *e = getenv("GEMMA_HIP_GEMV_BLOCKS_PER_CU")) {
      const int b = atoi(e);
      if (b >= 1 && b <= 64) v.blocks_per_cu = b;
    }
    if (const char *e = getenv("GEMMA_HIP_GEMV_LOOP")) v.force_loop = atoi(e) != 0;
    if (const char *e = getenv("GEMMA_HIP_GEMV_THREADS")) {
      const int t = atoi(e);
      if (t == 256 || t == 1024) v.threads = t;
    }
    return v;
  }();
  return t;
}

using PipeFn = void (*)(dim3, size_t, hipStream_t, const GemvJobs &, int, int,
                        const int8_t *, const float *, const float *, int8_t *,
                        float *);

template <int L, int CPL, bool FUSED, int NT>
void launch_pipe(dim3 grid, size_t lds, hipStream_t stream, const GemvJobs &jobs,
                 int total, int k, const int8_t *xq, const float *xs,
                 const float *xf, int8_t *xq_out, float *xs_out) {
  gemv_i8_pipelined_kernel<L, CPL, FUSED, NT><<<grid, NT, lds, stream>>>(
      jobs, total, k, xq, xs, xf, xq_out, xs_out);
}

template <int L, bool FUSED, int NT>
PipeFn pipe_for(int cpl) {
  switch (cpl) {
    case 1: return &launch_pipe<L, 1, FUSED, NT>;
    case 2: return &launch_pipe<L, 2, FUSED, NT>;
    case 3: return &launch_pipe<L, 3, FUSED, NT>;
    case 4: return &launch_pipe<L, 4, FUSED, NT>;
    case 5: return &launch_pipe<L, 5, FUSED, NT>;
    case 6: return &launch_pipe<L, 6, FUSED, NT>;
    case 7: return &launch_pipe<L, 7, FUSED, NT>;
    case 8: return &launch_pipe<L, 8, FUSED, NT>;
    case 9: return &launch_pipe<L, 9, FUSED, NT>;
    case 10: return &launch_pipe<L, 10, FUSED, NT>;
    case 11: case 12: return NT == 1024 ? nullptr : &launch_pipe<L, 12, FUSED, NT>;
    default: return nullptr;
  }
}

template <int NT>
PipeFn pipe_fn_nt(int lanes, int cpl, bool fused) {
  switch (lanes) {
    case 64: return fused ? pipe_for<64, true, NT>(cpl) : pipe_for<64, false, NT>(cpl);
    case 32: return fused ? pipe_for<32, true, NT>(cpl) : pipe_for<32, false, NT>(cpl);
    case 16: return fused ? pipe_for<16, true, NT>(cpl) : pipe_for<16, false, NT>(cpl);
    default: return fused ? pipe_for<8, true, NT>(cpl) : pipe_for<8, false, NT>(cpl);
  }
}

// The streaming kernel: L lanes per row, the smallest L with at most 10
// chunks per lane, one group in flight per wave (measured at the 1b and 4b
// LM heads and gate/up: a deeper register ring costs more in resident waves
// than it gains).
using StreamFn = hipError_t (*)(const DeviceInfo &, hipStream_t, const GemvJobs &, int, int,
                                const int8_t *, const float *, const float *, int8_t *,
                                float *);
constexpr int kStreamNT = 256;
constexpr int kStreamMaxCpl = 10;

template <int L, int CPL, bool FUSED>
hipError_t launch_stream(const DeviceInfo &dev, hipStream_t stream, const GemvJobs &jobs,
                         int ngroups, int k, const int8_t *xq, const float *xs,
                         const float *xf, int8_t *xq_out, float *xs_out) {
  constexpr int D = 1;
  auto kern = gemv_i8_stream_kernel<L, CPL, D, FUSED, kStreamNT>;
  const size_t lds = (size_t)(k + 15) / 16 * 16;
  // every workgroup resident at once: the groups are dealt round robin, so
  // a second round of workgroups would run as a tail
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStreamNT, lds) !=
          hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  if (tuning().blocks_per_cu > 0 && tuning().blocks_per_cu < per_cu)
    per_cu = tuning().blocks_per_cu;
  const long need = (ngroups + kStreamNT / 64 - 1) / (kStreamNT / 64);
  const long cap = (long)dev.cus * per_cu;
  kern<<<dim3((unsigned)(need < cap ? need : cap)), kStreamNT, lds, stream>>>(
      jobs, ngroups, k, xq, xs, xf, xq_out, xs_out);
  return hipGetLastError();
}

template <int L, bool FUSED, int C>
StreamFn stream_for(int cpl) {
  if (cpl == C) return &launch_stream<L, C, FUSED>;
  if constexpr (C < kStreamMaxCpl) return stream_for<L, FUSED, C + 1>(cpl);
  return nullptr;
}

// chunks per lane: up to 10 at L = 8; above 80 chunks a wider L has 6..10
StreamFn stream_fn(int kc, bool fused, int *lanes) {
  for (int l = 8; l <= 64; l *= 2) {
    const int cpl = (kc + l - 1) / l;
    if (cpl > kStreamMaxCpl) continue;
    *lanes = l;
    switch (l) {
      case 8: return fused ? stream_for<8, true, 1>(cpl) : stream_for<8, false, 1>(cpl);
      case 16: return fused ? stream_for<16, true, 6>(cpl) : stream_for<16, false, 6>(cpl);
      case 32: return fused ? stream_for<32, true, 6>(cpl) : stream_for<32, false, 6>(cpl);
      default: return fused ? stream_for<64, true, 6>(cpl) : stream_for<64, false, 6>(cpl);
    }
  }
  return nullptr;
}

PipeFn pipe_fn(int lanes, int cpl, bool fused, int threads) {
  return threads == 1024 ? pipe_fn_nt<1024>(lanes, cpl, fused)
                         : pipe_fn_nt<256>(lanes, cpl, fused);
}

}  // namespace

hipError_t launch_gemv_i8(const GemvJobs &jobs, int k, const int8_t *xq,
                          const float *xs, const float *xf, int8_t *xq_out,
                          float *xs_out, const DeviceInfo &dev,
                          hipStream_t stream) {
  const int total = jobs.end[jobs.njobs - 1];
  if (total <= 0 || k <= 0) return hipErrorInvalidValue;
  const bool vec = rows_aligned(jobs, k, 1, 16);
  const size_t lds = (size_t)(k + 15) / 16 * 16;
  const bool fused = xf != nullptr;
  // Measured on MI355X (1b and 4b decode shapes): up to ~4096 rows the
  // launch is latency-bound and one row per wave with every load issued up
  // front wins (q/k/v/o, and down with its 6912-byte rows; the 4b o
  // projection's 2560 rows: decoder 604 -> 607 tok/s); above that the
  // streaming kernel's groups amortise the per-row reduction better.
  // Long rows (k >= 4096) with few of them are latency-bound on the x
  // prologue: 1024-thread workgroups pay it 4x less often (measured on the
  // 1b/4b down projections: 8.8 -> 7.9 us and 13.9 -> 10.2 us; the stream
  // kernel there: 4b decoder 604 -> 544 tok/s).
  const bool long_rows = k >= 4096 && total <= 4096;
  const bool pipelined =
      tuning().lanes > 0 || tuning().threads > 0 || total <= 4096 || long_rows;
  if (vec && pipelined && !tuning().force_loop) {
    const int kc = k / 16;
    const int lanes = tuning().lanes > 0 ? tuning().lanes : 64;
    const int threads = tuning().threads > 0 ? tuning().threads : (long_rows ? 1024 : 256);
    const int cpl = (kc + lanes - 1) / lanes;
    PipeFn fn = pipe_fn(lanes, cpl, fused, threads);
    if (fn != nullptr) {
      const int rows_per_block = threads / 64 * (64 / lanes);
      long blocks = (total + rows_per_block - 1) / rows_per_block;
      const int per_cu = tuning().blocks_per_cu > 0 ? tuning().blocks_per_cu
                                                    : (threads == 1024 ? 2 : 8);
      const long cap = (long)dev.cus * per_cu;
      fn(dim3((unsigned)(blocks < cap ? blocks : cap)), lds, stream, jobs, total, k, xq, xs,
         xf, xq_out, xs_out);
      return hipGetLastError();
    }
  }
  if (vec && !tuning().force_loop) {
    bool fits = true;  // buffer offsets are 32-bit
    for (int j = 0, prev = 0; j < jobs.njobs; prev = jobs.end[j], ++j)
      fits = fits && (long)(jobs.end[j] - prev) * k < (long)kOutOfRange;
    int lanes = 0;
    StreamFn fn = fits ? stream_fn(k / 16, fused, &lanes) : nullptr;
    if (fn != nullptr) {
      const int rows = 64 / lanes;
      int ngroups = 0;
      for (int j = 0, prev = 0; j < jobs.njobs; prev = jobs.end[j], ++j)
        ngroups += (jobs.end[j] - prev + rows - 1) / rows;
      return fn(dev, stream, jobs, ngroups, k, xq, xs, xf, xq_out, xs_out);
    }
  }
  const int lanes = vec ? lanes_for(k / 16) : 64;
  const dim3 grid(grid_for(total, lanes, dev));
  if (fused)
    return vec ? gemv_i8_dispatch<true, true>(lanes, grid, lds, stream, jobs,
                                              total, k, xq, xs, xf, xq_out, xs_out)
               : gemv_i8_dispatch<true, false>(lanes, grid, lds, stream, jobs,
                                               total, k, xq, xs, xf, xq_out,
                                               xs_out);
  return vec ? gemv_i8_dispatch<false, true>(lanes, grid, lds, stream, jobs,
                                             total, k, xq, xs, xf, xq_out, xs_out)
             : gemv_i8_dispatch<false, false>(lanes, grid, lds, stream, jobs,
                                              total, k, xq, xs, xf, xq_out,
                                              xs_out);
}

namespace {

template <int L, int CPL>
hipError_t launch_f32_stream(const DeviceInfo &dev, hipStream_t stream, const GemvJobs &jobs,
                             int ngroups, int k, int passes, const float *x) {
  auto kern = gemv_f32_stream_kernel<L, CPL, kStreamNT>;
  const size_t lds = (size_t)(k / 4) * 16;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStreamNT, lds) !=
          hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const long need = (ngroups + kStreamNT / 64 - 1) / (kStreamNT / 64);
  const long cap = (long)dev.cus * per_cu;
  kern<<<dim3((unsigned)(need < cap ? need : cap)), kStreamNT, lds, stream>>>(jobs, ngroups, k,
                                                                              passes, x);
  return hipGetLastError();
}

// jobs with rows split so that every job's m * k * 4 < 2^31 (the stream
// kernel's buffer offsets), or false when that needs more than kMaxJobs jobs
bool split_f32_jobs(const GemvJobs &in, int k, GemvJobs *out) {
  const long max_rows = ((long)kOutOfRange - 1) / ((long)k * 4);
  if (max_rows < 1) return false;
  GemvJobs o{};
  int n = 0;
  for (int j = 0, prev = 0; j < in.njobs; prev = in.end[j], ++j) {
    for (int r0 = prev; r0 < in.end[j]; r0 += (int)max_rows) {
      if (n == kMaxJobs) return false;
      const int r1 = (int)std::min<long>(in.end[j], (long)r0 + max_rows);
      o.w[n] = static_cast<const float *>(in.w[j]) + (size_t)(r0 - prev) * k;
      o.sc[n] = nullptr;
      o.dst[n] = in.dst[j] + (r0 - prev);
      o.end[n] = r1;
      ++n;
    }
  }
  if (n == 0) return false;
  for (int t = n; t < kMaxJobs; ++t) o.end[t] = o.end[n - 1];
  o.njobs = n;
  *out = o;
  return true;
}

}  // namespace

hipError_t launch_gemv_f32(const GemvJobs &jobs, int k, const float *x,
                           const DeviceInfo &dev, hipStream_t stream) {
  const int total = jobs.end[jobs.njobs - 1];
  const bool vec = rows_aligned(jobs, k, 4, 16);
  GemvJobs sj;
  if (vec && ((uintptr_t)x & 15) == 0 && !tuning().force_loop && split_f32_jobs(jobs, k, &sj)) {
    const F32StreamShape sh = f32_stream_shape(k / 4, false, total);
    const int rows = 64 / sh.lanes;
    int ngroups = 0;
    for (int j = 0, prev = 0; j < sj.njobs; prev = sj.end[j], ++j)
      ngroups += (sj.end[j] - prev + rows - 1) / rows;
    auto go = [&](auto lanes) {
      constexpr int L = decltype(lanes)::value;
      switch (sh.cpl) {
        case 8: return launch_f32_stream<L, 8>(dev, stream, sj, ngroups, k, sh.passes, x);
        case 10: return launch_f32_stream<L, 10>(dev, stream, sj, ngroups, k, sh.passes, x);
        default: return launch_f32_stream<L, 12>(dev, stream, sj, ngroups, k, sh.passes, x);
      }
    };
    switch (sh.lanes) {
      case 8: return go(std::integral_constant<int, 8>{});
      case 16: return go(std::integral_constant<int, 16>{});
      case 32: return go(std::integral_constant<int, 32>{});
      default: return go(std::integral_constant<int, 64>{});
    }
  }
  const int lanes = vec ? lanes_for(k / 4) : 64;
  const dim3 grid(grid_for(total, lanes, dev));
  const size_t lds = (size_t)(k + 3) / 4 * 16;
  return vec ? gemv_f32_dispatch<true>(lanes, grid, lds, stream, jobs, total, k, x)
             : gemv_f32_dispatch<false>(lanes, grid, lds, stream, jobs, total, k, x);
}

}  // namespace gh
