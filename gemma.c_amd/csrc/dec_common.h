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


// e^x in fp64 by Tang's table-driven method (P. T. P. Tang, "Table-driven
// implementation of the exponential function in IEEE floating-point
// arithmetic", ACM TOMS 15(2), 1989): x = (128 e + j) ln2/128 + r with
// |r| <= ln2/256, e^x = 2^e * 2^(j/128) * e^r, e^r by its Taylor polynomial of
// degree 5 (truncation below 6e-19 relative); ln2/128 is split so that
// k * hi is exact for |k| < 2^21.  The result is within about 2 ulp of e^x.
// Arguments are clamped to [-800, 800], where e^x is 0 or inf.  kExp2Tab
// holds 2^(j/128) correctly rounded; the caller copies it into LDS
// (exp_tab_load) and passes the constants from scalar registers
// (exp_consts).
__constant__ double kExp2Tab[128] = {
    0x1.0000000000000p+0, 0x1.0163da9fb3335p+0, 0x1.02c9a3e778061p+0, 0x1.04315e86e7f85p+0,
    0x1.059b0d3158574p+0, 0x1.0706b29ddf6dep+0, 0x1.0874518759bc8p+0, 0x1.09e3ecac6f383p+0,
    0x1.0b5586cf9890fp+0, 0x1.0cc922b7247f7p+0, 0x1.0e3ec32d3d1a2p+0, 0x1.0fb66affed31bp+0,
    0x1.11301d0125b51p+0, 0x1.12abdc06c31ccp+0, 0x1.1429aaea92de0p+0, 0x1.15a98c8a58e51p+0,
    0x1.172b83c7d517bp+0, 0x1.18af9388c8deap+0, 0x1.1a35beb6fcb75p+0, 0x1.1bbe084045cd4p+0,
    0x1.1d4873168b9aap+0, 0x1.1ed5022fcd91dp+0, 0x1.2063b88628cd6p+0, 0x1.21f49917ddc96p+0,
    0x1.2387a6e756238p+0, 0x1.251ce4fb2a63fp+0, 0x1.26b4565e27cddp+0, 0x1.284dfe1f56381p+0,
    0x1.29e9df51fdee1p+0, 0x1.2b87fd0dad990p+0, 0x1.2d285a6e4030bp+0, 0x1.2ecafa93e2f56p+0,
    0x1.306fe0a31b715p+0, 0x1.32170fc4cd831p+0, 0x1.33c08b26416ffp+0, 0x1.356c55f929ff1p+0,
    0x1.371a7373aa9cbp+0, 0x1.38cae6d05d866p+0, 0x1.3a7db34e59ff7p+0, 0x1.3c32dc313a8e5p+0,
    0x1.3dea64c123422p+0, 0x1.3fa4504ac801cp+0, 0x1.4160a21f72e2ap+0, 0x1.431f5d950a897p+0,
    0x1.44e086061892dp+0, 0x1.46a41ed1d0057p+0, 0x1.486a2b5c13cd0p+0, 0x1.4a32af0d7d3dep+0,
    0x1.4bfdad5362a27p+0, 0x1.4dcb299fddd0dp+0, 0x1.4f9b2769d2ca7p+0, 0x1.516daa2cf6642p+0,
    0x1.5342b569d4f82p+0, 0x1.551a4ca5d920fp+0, 0x1.56f4736b527dap+0, 0x1.58d12d497c7fdp+0,
    0x1.5ab07dd485429p+0, 0x1.5c9268a5946b7p+0, 0x1.5e76f15ad2148p+0, 0x1.605e1b976dc09p+0,
    0x1.6247eb03a5585p+0, 0x1.6434634ccc320p+0, 0x1.6623882552225p+0, 0x1.68155d44ca973p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6c012750bdabfp+0, 0x1.6dfb23c651a2fp+0, 0x1.6ff7df9519484p+0,
    0x1.71f75e8ec5f74p+0, 0x1.73f9a48a58174p+0, 0x1.75feb564267c9p+0, 0x1.780694fde5d3fp+0,
    0x1.7a11473eb0187p+0, 0x1.7c1ed0130c132p+0, 0x1.7e2f336cf4e62p+0, 0x1.80427543e1a12p+0,
    0x1.82589994cce13p+0, 0x1.8471a4623c7adp+0, 0x1.868d99b4492edp+0, 0x1.88ac7d98a6699p+0,
    0x1.8ace5422aa0dbp+0, 0x1.8cf3216b5448cp+0, 0x1.8f1ae99157736p+0, 0x1.9145b0b91ffc6p+0,
    0x1.93737b0cdc5e5p+0, 0x1.95a44cbc8520fp+0, 0x1.97d829fde4e50p+0, 0x1.9a0f170ca07bap+0,
    0x1.9c49182a3f090p+0, 0x1.9e86319e32323p+0, 0x1.a0c667b5de565p+0, 0x1.a309bec4a2d33p+0,
    0x1.a5503b23e255dp+0, 0x1.a799e1330b358p+0, 0x1.a9e6b5579fdbfp+0, 0x1.ac36bbfd3f37ap+0,
    0x1.ae89f995ad3adp+0, 0x1.b0e07298db666p+0, 0x1.b33a2b84f15fbp+0, 0x1.b59728de5593ap+0,
    0x1.b7f76f2fb5e47p+0, 0x1.ba5b030a1064ap+0, 0x1.bcc1e904bc1d2p+0, 0x1.bf2c25bd71e09p+0,
    0x1.c199bdd85529cp+0, 0x1.c40ab5fffd07ap+0, 0x1.c67f12e57d14bp+0, 0x1.c8f6d9406e7b5p+0,
    0x1.cb720dcef9069p+0, 0x1.cdf0b555dc3fap+0, 0x1.d072d4a07897cp+0, 0x1.d2f87080d89f2p+0,
    0x1.d5818dcfba487p+0, 0x1.d80e316c98398p+0, 0x1.da9e603db3285p+0, 0x1.dd321f301b460p+0,
    0x1.dfc97337b9b5fp+0, 0x1.e264614f5a129p+0, 0x1.e502ee78b3ff6p+0, 0x1.e7a51fbc74c83p+0,
    0x1.ea4afa2a490dap+0, 0x1.ecf482d8e67f1p+0, 0x1.efa1bee615a27p+0, 0x1.f252b376bba97p+0,
    0x1.f50765b6e4540p+0, 0x1.f7bfdad9cbe14p+0, 0x1.fa7c1819e90d8p+0, 0x1.fd3c22b8f71f1p+0,
};

struct ExpConsts {
  double inv, hi, lo, c5, c4, c3;
};

__device__ __forceinline__ ExpConsts exp_consts() {
  ExpConsts c;
  c.inv = in_sgpr(0x1.71547652b82fep+7);  // 128 / ln2
  c.hi = in_sgpr(0x1.62e42fee00000p-8);   // ln2 / 128, 32 significant bits
  c.lo = in_sgpr(0x1.a39ef35793c76p-40);  // ln2 / 128 - hi
  c.c5 = in_sgpr(1.0 / 120.0);
  c.c4 = in_sgpr(1.0 / 24.0);
  c.c3 = in_sgpr(1.0 / 6.0);
  return c;
}

// every thread of the workgroup takes part; a barrier must follow
__device__ __forceinline__ void exp_tab_load(double *tab) {
  for (int i = threadIdx.x; i < 128; i += blockDim.x) tab[i] = kExp2Tab[i];
}

__device__ __forceinline__ double exp_tab(double x, const double *tab, const ExpConsts &c) {
  x = fmin(fmax(x, -800.0), 800.0);  // e^x is 0 below -745 and inf above 710
  const double kf = rint(x * c.inv);
  double r = fma(-kf, c.hi, x);
  r = fma(-kf, c.lo, r);
  double p = fma(r, c.c5, c.c4);
  p = fma(r, p, c.c3);
  p = fma(r, p, 0.5);
  p = fma(r, p, 1.0);
  p = fma(r, p, 1.0);
  const int k = (int)kf;
  return ldexp(tab[k & 127] * p, k >> 7);
}

// gelu_tanh (gemma.c:4139-4145) with the reference's fp32 constants, in
// fp64: 0.5 x (1 + tanh(u)) with u = c (x + k x^3) is the same function as
// x / (1 + e^(-2u)) (1 + tanh(u) = 2 / (1 + e^(-2u))), which costs one table
// exponential and one reciprocal instead of tanh.  The two forms differ only
// by fp64 rounding; at x -> -inf both give -0, at x -> +inf both give x.
__device__ __forceinline__ double gelu(double x, const double *etab, const ExpConsts &ec) {
  const double c = (double)0.79788456080287f;
  const double k = (double)0.044715f;
  const double u = c * (x + k * x * x * x);
  // x / d by v_rcp_f64 and two Newton steps (each squares the relative
  // error, so the reciprocal is within an ulp or two of fp64), instead of
  // the correctly rounded fp64 division sequence: the result is rounded to
  // fp32 once anyway.  d is capped at 1e300, where x / d and x * (1 / d)
  // both round to a zero of x's sign in fp32 (d = inf would give NaN in
  // the Newton steps).
  const double d = fmin(1.0 + exp_tab(-2.0 * u, etab, ec), 1e300);
  double r = __builtin_amdgcn_rcp(d);
  r = fma(r, fma(-d, r, 1.0), r);
  r = fma(r, fma(-d, r, 1.0), r);
  return x * r;
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

// Every load is issued (a chunk past dim reloads chunk 0, an absent vector
// reads x_res) and the unused values are zeroed after they return: a
// conditional load makes the compiler's wait counts wait for it, and for
// everything issued before it, at its first use.
template <int NPT, int NT>
__device__ __forceinline__ void norm_load(const DecNorm &a, NormIn<NPT> &in) {
  const int tid = threadIdx.x;
  const int n4 = a.dim >> 2;
  const v4f *y = reinterpret_cast<const v4f *>(a.y != nullptr ? a.y : a.x_res);
  const v4f *wp = reinterpret_cast<const v4f *>(a.w_post != nullptr ? a.w_post : a.x_res);
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT < n4 ? tid + j * NT : 0;
    in.xr[j] = reinterpret_cast<const v4f *>(a.x_res)[c];
    in.wq[j] = reinterpret_cast<const v4f *>(a.w_pre)[c];
    in.y[j] = y[c];
    in.wp[j] = wp[c];
  }
}

// Zeroes what norm_load read past dim or from an absent vector (call once
// the values are needed).
template <int NPT, int NT>
__device__ __forceinline__ void norm_fix(const DecNorm &a, NormIn<NPT> &in) {
  const int tid = threadIdx.x;
  const int n4 = a.dim >> 2;
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const bool ok = tid + j * NT < n4;
    if (!ok) in.xr[j] = in.wq[j] = zero;
    if (!ok || a.y == nullptr) in.y[j] = zero;
    if (!ok || a.w_post == nullptr) in.wp[j] = zero;
  }
}

// Kernel arguments into scalar registers at once.  The compiler otherwise
// loads each argument where it is first used, and an argument read behind a
// branch (a job's end, a nullable vector) costs a dependent scalar-memory
// round trip before the loads that follow it can issue.
__device__ __forceinline__ void hold_args(const DecNorm &n) {
  asm volatile("" ::"s"(n.x_res), "s"(n.y), "s"(n.w_post), "s"(n.w_pre), "s"(n.x_out),
               "s"(n.h_out), "s"(n.dim), "s"(n.eps));
}
__device__ __forceinline__ void hold_args(const GemvJobs &j) { hold_jobs(j); }
__device__ __forceinline__ void hold_args(const DecAttn &a) {
  asm volatile("" ::"s"(a.xq), "s"(a.xk), "s"(a.xv), "s"(a.nq), "s"(a.nk), "s"(a.rope),
               "s"(a.kc), "s"(a.vc), "s"(a.step), "s"(a.part));
  asm volatile("" ::"s"(a.xo), "s"(a.n_heads), "s"(a.nkv), "s"(a.hdim), "s"(a.clen),
               "s"(a.slide), "s"(a.max_blocks), "s"(a.nvocab), "s"(a.asc), "s"(a.sc_att),
               "s"(a.eps));
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
  norm_fix<NPT, NT>(a, in);
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

// This workgroup's share (part `part` of `parts`) of the regions, read and
// discarded: four 16-byte loads in flight per thread, their values fed to an
// empty asm statement.  Called at the end of a kernel, so that its waits
// delay only the workgroup's exit.
__device__ __forceinline__ void warm_share(const WarmRegions &w, int part, int parts, int tid,
                                           int nt) {
  for (int j = 0; j < w.n; ++j) {
    const v4i *p = static_cast<const v4i *>(w.p[j]);
    const size_t n = w.bytes[j] / 16;
    const size_t per = (n + parts - 1) / parts;
    const size_t lo = (size_t)part * per, hi = lo + per < n ? lo + per : n;
    const size_t st = (size_t)nt;
    for (size_t i = lo + tid; i < hi; i += 4 * st) {
      auto at = [&](size_t u) { return i + u * st < hi ? i + u * st : hi - 1; };
      const v4i x0 = p[i], x1 = p[at(1)], x2 = p[at(2)], x3 = p[at(3)];
      asm volatile("" ::"v"(x0), "v"(x1), "v"(x2), "v"(x3));
    }
  }
}

}  // namespace
}  // namespace gh
