// dec_common.h -- device helpers shared by the decode step (decode.hip) and
// the batched prefill (prefill.hip): workgroup reductions in a fixed order,
// the fp64-evaluated glue of the reference's fp32 formulas (rmsnorm,
// clamp_fpx, gelu_tanh) and the residual + norm + quantize prologue.
#pragma once

#include <float.h>
#include <math.h>

#include "gh_arith.h"
#include "gh_kernels.h"

namespace gh {
namespace {

constexpr int kNT = 256;
constexpr int kWaves = kNT / 64;
constexpr int kAttB = kDecAttnBlock;  // keys per attention workgroup

// Workgroup sum / max, the same bits in every thread (and in every
// workgroup that reduces the same values): wave reductions in a fixed DPP
// order, then the waves' results in wave order.
template <int NT = kNT>
__device__ __forceinline__ double block_sum(double v, double *red) {
  v = wave_sum_f64(v);
  lds_barrier();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_barrier();
  double s = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) s += red[w];
  return s;
}

template <int NT = kNT>
__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max_dpp(v);
  lds_barrier();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_barrier();
  float s = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) s = fmaxf(s, red[w]);
  return s;
}

// clamp_fpx (gemma.c:2504-2506) for fp32
__device__ __forceinline__ float clamp_f32(float v) {
  return fminf(FLT_MAX, fmaxf(-FLT_MAX, v));
}

// 1 / sqrt(mean(x^2) + eps) of rmsnorm (gemma.c:2512-2516)
__device__ __forceinline__ double rms_of(double sqsum, int dim, float eps) {
  return 1.0 / sqrt(sqsum / (double)dim + (double)eps);
}

// one rmsnorm output element: x * rms * (w + 1), rounded once
__device__ __forceinline__ float norm_one(float x, double rms, float w) {
  return (float)((double)x * rms * ((double)w + 1.0));
}

// gelu_tanh (gemma.c:4139-4145) with the reference's fp32 constants
__device__ __forceinline__ double gelu_tanh(double x) {
  const double c = (double)0.79788456080287f;
  const double k = (double)0.044715f;
  return 0.5 * x * (1.0 + tanh(c * (x + k * x * x * x)));
}

// Reads the step's token and position; false when they are out of range
// (the host checks them, this keeps a bad value from addressing memory).
__device__ __forceinline__ bool step_ok(const int *step, int nvocab, int clen,
                                        int *token, int *pos) {
  *token = step[0];
  *pos = step[1];
  return *token >= 0 && *token < nvocab && *pos >= 0 && *pos < clen;
}

// x_new = clamp(x_res + post(y)), h = rmsnorm(x_new, w_pre), and h
// quantized into xq (LDS, int8) exactly as quantize_act does (gemma.c:
// 2590-2650).  Split in two so the caller can issue its own (HBM) loads
// between them: norm_load issues every load the prologue needs (NPT
// 16-byte chunks per vector per thread, dim <= NPT * 4 * NT); vector loads
// return in issue order, so loads issued after it do not delay it.
template <int NPT>
struct NormIn {
  v4f y[NPT], xr[NPT], wp[NPT], wq[NPT];
};

template <int NPT, int NT>
__device__ __forceinline__ void norm_load(const DecNorm &a, NormIn<NPT> &in) {
  const int tid = threadIdx.x;
  const int n4 = a.dim >> 2;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
    const bool ok = c < n4;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    in.xr[j] = ok ? reinterpret_cast<const v4f *>(a.x_res)[c] : zero;
    in.wq[j] = ok ? reinterpret_cast<const v4f *>(a.w_pre)[c] : zero;
    in.y[j] = (ok && a.y != nullptr) ? reinterpret_cast<const v4f *>(a.y)[c] : zero;
    in.wp[j] = (ok && a.w_post != nullptr) ? reinterpret_cast<const v4f *>(a.w_post)[c] : zero;
  }
}

// The arithmetic of the prologue; returns the activation scale.  Workgroup 0
// (every workgroup with kEvery, when each normalizes its own row) stores
// x_new to x_out and h to h_out (each nullable); xq may be null (the final
// norm only stores h).
template <int NPT, int NT, bool kEvery = false>
__device__ float norm_quant(const DecNorm &a, NormIn<NPT> &in, int8_t *xq, double *red,
                            float *redf) {
  const int tid = threadIdx.x;
  const int n4 = a.dim >> 2;
  if (a.y != nullptr) {
    double rms = 1.0;
    if (a.w_post != nullptr) {
      double ss = 0.0;
#pragma unroll
      for (int j = 0; j < NPT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) ss += (double)in.y[j][e] * (double)in.y[j][e];
      rms = rms_of(block_sum<NT>(ss, red), a.dim, a.eps);
    }
#pragma unroll
    for (int j = 0; j < NPT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float t = a.w_post != nullptr ? norm_one(in.y[j][e], rms, in.wp[j][e]) : in.y[j][e];
        in.xr[j][e] = clamp_f32(t + in.xr[j][e]);
      }
  }
  if ((kEvery || blockIdx.x == 0) && a.x_out != nullptr)
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      if (tid + j * NT < n4) reinterpret_cast<v4f *>(a.x_out)[tid + j * NT] = in.xr[j];
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += (double)in.xr[j][e] * (double)in.xr[j][e];
  const double rms = rms_of(block_sum<NT>(ss, red), a.dim, a.eps);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      in.y[j][e] = norm_one(in.xr[j][e], rms, in.wq[j][e]);  // h; padding lanes stay 0
      amax = fmaxf(amax, abs_daz(in.y[j][e]));
    }
  if ((kEvery || blockIdx.x == 0) && a.h_out != nullptr)
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      if (tid + j * NT < n4) reinterpret_cast<v4f *>(a.h_out)[tid + j * NT] = in.y[j];
  if (xq == nullptr) return 1.0f;
  amax = block_max<NT>(amax, redf);
  const QuantParams qp = quant_params(amax);
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
    if (c < n4)
      reinterpret_cast<uint32_t *>(xq)[c] =
          pack4(quant_one(in.y[j].x, qp.inv), quant_one(in.y[j].y, qp.inv),
                quant_one(in.y[j].z, qp.inv), quant_one(in.y[j].w, qp.inv));
  }
  lds_barrier();
  return qp.scale;
}

__device__ __forceinline__ int32_t dot16(v4i w, v4i x, int32_t acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}

}  // namespace
}  // namespace gh
