// quantize.hip -- per-row symmetric int8 quantization of activations
// (gemma.c:2586-2674 quantize_act / quantize_acts).
//
// One 256-thread workgroup per row.  Pass 1 reduces amax = max|v| exactly
// (max is order-independent), pass 2 re-reads the row (now L2-resident) and
// writes q.  HBM traffic per row: 4n bytes read, n + 4 written.
// The host entry points also pass a mirror (mdst, mdsc: pinned host memory)
// that receives a second copy of q and the scale, so one launch both leaves
// the result on the device and returns it to the host.
#include "gh_arith.h"
#include "gh_kernels.h"

namespace gh {
namespace {

constexpr int kThreads = 256;

template <bool VEC>
__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(
    int8_t *__restrict__ dst, float *__restrict__ dsc,
    const float *__restrict__ src, int sstr, int n, int8_t *__restrict__ mdst,
    float *__restrict__ mdsc) {
  __shared__ float wave_amax[kThreads / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const float *in = src + (size_t)row * sstr;
  int8_t *out = dst + (size_t)row * n;
  int8_t *mout = mdst != nullptr ? mdst + (size_t)row * n : nullptr;

  float amax = 0.0f;
  if (VEC) {
    const v4f *in4 = reinterpret_cast<const v4f *>(in);
    for (int c = tid; c < n / 4; c += kThreads) {
      v4f v = in4[c];
      amax = fmaxf(amax, fmaxf(fmaxf(abs_daz(v.x), abs_daz(v.y)),
                               fmaxf(abs_daz(v.z), abs_daz(v.w))));
    }
  } else {
    for (int c = tid; c < n; c += kThreads) amax = fmaxf(amax, abs_daz(in[c]));
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) wave_amax[tid >> 6] = amax;
  lds_barrier();
  amax = fmaxf(fmaxf(wave_amax[0], wave_amax[1]),
               fmaxf(wave_amax[2], wave_amax[3]));
  const QuantParams qp = quant_params(amax);

  if (VEC) {
    const v4f *in4 = reinterpret_cast<const v4f *>(in);
    uint32_t *out4 = reinterpret_cast<uint32_t *>(out);
    for (int c = tid; c < n / 4; c += kThreads) {
      v4f v = in4[c];
      const uint32_t q4 = pack4(quant_one(v.x, qp.inv), quant_one(v.y, qp.inv),
                                quant_one(v.z, qp.inv), quant_one(v.w, qp.inv));
      out4[c] = q4;
      if (mout != nullptr) reinterpret_cast<uint32_t *>(mout)[c] = q4;
    }
  } else {
    for (int c = tid; c < n; c += kThreads) {
      const int8_t q = (int8_t)quant_one(in[c], qp.inv);
      out[c] = q;
      if (mout != nullptr) mout[c] = q;
    }
  }
  if (tid == 0) {
    dsc[row] = qp.scale;
    if (mdsc != nullptr) mdsc[row] = qp.scale;
  }
}

}  // namespace

hipError_t launch_quantize(int8_t *dst, float *dsc, const float *src, int sstr,
                           int m, int n, hipStream_t stream, int8_t *mdst,
                           float *mdsc) {
  const bool vec = (n % 4 == 0) && (sstr % 4 == 0) &&
                   ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 4 == 0) &&
                   ((uintptr_t)mdst % 4 == 0);
  if (vec)
    quantize_rows_kernel<true><<<dim3(m), dim3(kThreads), 0, stream>>>(
        dst, dsc, src, sstr, n, mdst, mdsc);
  else
    quantize_rows_kernel<false><<<dim3(m), dim3(kThreads), 0, stream>>>(
        dst, dsc, src, sstr, n, mdst, mdsc);
  return hipGetLastError();
}

}  // namespace gh
