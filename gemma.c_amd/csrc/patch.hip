// patch.hip -- SigLIP patch embedding as im2col + fp32 GEMM
// (gemma.c:4411-4448: the stride-P, PxP convolution of the HWC image).
//
// im2col writes A [npatch][3*P*P] in the K order of the weight pe
// [dim][3][P][P] (k = c*P*P + py*P + px), so the product with pe^T is the
// reference's sum over (py, px, c) for every (patch, out channel); the GEMM
// epilogue adds pe_b and applies clamp_fpx (gemma.c:2504-2506).  Traffic of
// im2col: 4*npatch*3*P*P bytes read and written (9.6 MB at 896 px, P = 14),
// against 5.5 GFLOP of GEMM.
#include "gh_arith.h"
#include "gh_kernels.h"

namespace gh {
namespace {

constexpr int kThreads = 256;

// one workgroup per patch; thread t handles K indices t, t+256, ...
__global__ __launch_bounds__(kThreads) void im2col_kernel(
    float *__restrict__ a, const float *__restrict__ img, int img_px, int psize) {
  const int ppi = img_px / psize;
  const int pi = blockIdx.x;
  const int oy = pi / ppi;
  const int ox = pi - oy * ppi;
  const int pp = psize * psize;
  const int kdim = 3 * pp;
  float *row = a + (size_t)pi * kdim;
  for (int kk = threadIdx.x; kk < kdim; kk += kThreads) {
    const int c = kk / pp;
    const int rem = kk - c * pp;
    const int py = rem / psize;
    const int px = rem - py * psize;
    row[kk] = img[((size_t)(oy * psize + py) * img_px + (ox * psize + px)) * 3 + c];
  }
}

}  // namespace

hipError_t launch_im2col(float *a, const float *img, int img_px, int psize,
                         hipStream_t stream) {
  const int ppi = img_px / psize;
  im2col_kernel<<<dim3(ppi * ppi), kThreads, 0, stream>>>(a, img, img_px, psize);
  return hipGetLastError();
}

}  // namespace gh
