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

template <class T>
__device__ __forceinline__ T pick(const T (&arr)[kMaxJobs], int j) {
  T v = arr[0];
#pragma unroll
  for (int t = 1; t < kMaxJobs; ++t)
    if (j == t) v = arr[t];
  return v;
}

__device__ __forceinline__ int32_t dot16(v4i w, v4i x, int32_t acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}

// Stage the activation vector in LDS as int8.  FUSED: quantize x fp32 [k]
// (the quantize_act that precedes every decode GEMV); otherwise copy xq.
// Returns the activation scale.
template <bool FUSED>
__device__ __forceinline__ float stage_x_i8(int8_t *lds, int k,
                                            const int8_t *__restrict__ xq,
                                            const float *__restrict__ xs,
                                            const float *__restrict__ xf,
                                            int8_t *__restrict__ xq_out,
                                            float *__restrict__ xs_out) {
  const int tid = threadIdx.x;
  if (!FUSED) {
    if (((uintptr_t)xq & 15) == 0 && (k & 15) == 0) {
      for (int c = tid; c < k / 16; c += kThreads)
        reinterpret_cast<v4i *>(lds)[c] =
            reinterpret_cast<const v4i *>(xq)[c];
    } else {
      for (int c = tid; c < k; c += kThreads) lds[c] = xq[c];
    }
    __syncthreads();
    return *xs;
  }

  __shared__ float wave_amax[kWaves];
  const bool vec = ((uintptr_t)xf & 15) == 0 && (k & 3) == 0;
  float amax = 0.0f;
  if (vec) {
    for (int c = tid; c < k / 4; c += kThreads) {
      v4f v = reinterpret_cast<const v4f *>(xf)[c];
      amax = fmaxf(amax, fmaxf(fmaxf(abs_daz(v.x), abs_daz(v.y)),
                               fmaxf(abs_daz(v.z), abs_daz(v.w))));
    }
  } else {
    for (int c = tid; c < k; c += kThreads) amax = fmaxf(amax, abs_daz(xf[c]));
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) wave_amax[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wave_amax[0], wave_amax[1]),
               fmaxf(wave_amax[2], wave_amax[3]));
  const QuantParams qp = quant_params(amax);
  if (vec) {
    for (int c = tid; c < k / 4; c += kThreads) {
      v4f v = reinterpret_cast<const v4f *>(xf)[c];
      reinterpret_cast<uint32_t *>(lds)[c] =
          pack4(quant_one(v.x, qp.inv), quant_one(v.y, qp.inv),
                quant_one(v.z, qp.inv), quant_one(v.w, qp.inv));
    }
  } else {
    for (int c = tid; c < k; c += kThreads)
      lds[c] = (int8_t)quant_one(xf[c], qp.inv);
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    if (xq_out != nullptr)
      for (int c = tid; c < k; c += kThreads) xq_out[c] = lds[c];
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
      const int8_t *w = static_cast<const int8_t *>(pick(jobs.w, j));
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
      pick(jobs.dst, j)[r] = rescale(acc, act_scale, pick(jobs.sc, j)[r]);
  }
}

template <int L, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_f32_kernel(
    GemvJobs jobs, int total, int k, const float *__restrict__ x) {
  extern __shared__ v4f lds_f4[];
  float *lds_f = reinterpret_cast<float *>(lds_f4);
  for (int c = threadIdx.x; c < k; c += kThreads) lds_f[c] = x[c];
  __syncthreads();

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
      const float *w = static_cast<const float *>(pick(jobs.w, j));
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
    if (sub == 0 && row < total) pick(jobs.dst, j)[r] = acc;
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

}  // namespace

hipError_t launch_gemv_i8(const GemvJobs &jobs, int k, const int8_t *xq,
                          const float *xs, const float *xf, int8_t *xq_out,
                          float *xs_out, const DeviceInfo &dev,
                          hipStream_t stream) {
  const int total = jobs.end[jobs.njobs - 1];
  const bool vec = rows_aligned(jobs, k, 1, 16);
  const int lanes = vec ? lanes_for(k / 16) : 64;
  const dim3 grid(grid_for(total, lanes, dev));
  const size_t lds = (size_t)(k + 15) / 16 * 16;
  const bool fused = xf != nullptr;
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

hipError_t launch_gemv_f32(const GemvJobs &jobs, int k, const float *x,
                           const DeviceInfo &dev, hipStream_t stream) {
  const int total = jobs.end[jobs.njobs - 1];
  const bool vec = rows_aligned(jobs, k, 4, 16);
  const int lanes = vec ? lanes_for(k / 4) : 64;
  const dim3 grid(grid_for(total, lanes, dev));
  const size_t lds = (size_t)(k + 3) / 4 * 16;
  return vec ? gemv_f32_dispatch<true>(lanes, grid, lds, stream, jobs, total, k, x)
             : gemv_f32_dispatch<false>(lanes, grid, lds, stream, jobs, total, k, x);
}

}  // namespace gh
