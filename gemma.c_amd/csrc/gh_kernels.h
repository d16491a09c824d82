// gh_kernels.h -- launchers of the library's HIP kernels (internal to the
// library; the public interface is include/gemma_hip.h).
//
// Every launcher checks nothing about its arguments beyond what selects a
// kernel variant: gemma_hip.cpp validates shapes, strides and pointers before
// calling, so each launch covers exactly the rows, columns and bytes the
// kernel's grid assumes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gh {

constexpr int kMaxJobs = 4;

// A fused multi-output GEMV: jobs[j] owns output rows [end[j-1], end[j]).
struct GemvJobs {
  const void *w[kMaxJobs];
  const float *sc[kMaxJobs];
  float *dst[kMaxJobs];
  int end[kMaxJobs];
  int njobs;
};

struct DeviceInfo {
  int cus;  // compute units
};

// quantize.hip: rows of src [m][sstr] -> dst [m][n] int8 + dsc [m], and the
// same into the mirror mdst/mdsc when given (pinned host memory)
hipError_t launch_quantize(int8_t *dst, float *dsc, const float *src, int sstr,
                           int m, int n, hipStream_t stream,
                           int8_t *mdst = nullptr, float *mdsc = nullptr);

// gemv.hip: int8 GEMV over jobs.  Either xq/xs (already quantized) or xf
// (fp32, quantized inside the kernel; xq_out/xs_out nullable) is given.
hipError_t launch_gemv_i8(const GemvJobs &jobs, int k, const int8_t *xq,
                          const float *xs, const float *xf, int8_t *xq_out,
                          float *xs_out, const DeviceInfo &dev,
                          hipStream_t stream);

// gemv.hip: fp32 GEMV over jobs (sc unused).
hipError_t launch_gemv_f32(const GemvJobs &jobs, int k, const float *x,
                           const DeviceInfo &dev, hipStream_t stream);

// gemm_i8.hip: dst = rescale(src . mat^T).  hdim > 0 selects the head-major
// output layout dst[((j/hdim)*m + i)*hdim + j%hdim] (dstr ignored).
hipError_t launch_gemm_i8(float *dst, int dstr, int hdim, const int8_t *mat,
                          int mstr, const float *matsc, const int8_t *src,
                          int sstr, const float *ssc, int m, int n, int k,
                          const DeviceInfo &dev, hipStream_t stream);

// gemm_f32.hip: dst = src . mat^T in fp32; bias (nullable) adds bias[col],
// clamp limits every output to [-FLT_MAX, FLT_MAX] (clamp_fpx).
hipError_t launch_gemm_f32(float *dst, int dstr, const float *mat, int mstr,
                           const float *src, int sstr, int m, int n, int k,
                           const float *bias, bool clamp,
                           const DeviceInfo &dev, hipStream_t stream);

// patch.hip: a [npatch][3*psize*psize] = patches of the HWC image, in the K
// order of the SigLIP patch-embedding weight [dim][3][psize][psize].
hipError_t launch_im2col(float *a, const float *img, int img_px, int psize,
                         hipStream_t stream);

}  // namespace gh
