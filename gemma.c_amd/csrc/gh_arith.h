// gh_arith.h -- device arithmetic that reproduces the reference build's fp32
// results bit for bit on gfx950.
//
// The reference (gemma.c, built by gcc with -ffast-math) runs with FTZ and DAZ
// set in MXCSR and truncates with cvttss2si.  gfx950 keeps fp32 denormals and
// saturates on conversion, so the differences are written out here:
//  - DAZ: a subnormal operand is read as a zero of its sign.
//  - FTZ: x86 flushes a product whose value, rounded to 24 bits with an
//    unbounded exponent, is below FLT_MIN.  The GPU's gradual underflow gives
//    the same answer except when its denormal rounding lands on exactly
//    FLT_MIN; that case is settled with the exact double product.
//  - cvttss2si returns INT_MIN for NaN and out-of-range values.
// Files including this header are compiled with -ffp-contract=off, so every
// a*b and a+b below is one IEEE round-to-nearest operation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gh {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float daz(float v) {
  uint32_t bits = __float_as_uint(v);
  return (bits & 0x7f800000u) == 0 ? __uint_as_float(bits & 0x80000000u) : v;
}

// a*b under FTZ/DAZ (gemma.c's rescale products, gemma.c:2762, 3629, 3862)
__device__ __forceinline__ float mul_ftz(float a, float b) {
  a = daz(a);
  b = daz(b);
  float p = a * b;
  if (fabsf(p) <= 1.17549435e-38f) {
    double exact = (double)a * (double)b;  // exact: 24+24 bits fit in 53
    float scaled = (float)(exact * 0x1p64);  // 24-bit rounding, no underflow
    p = fabsf(scaled) < 0x1p-62f
            ? (__double_as_longlong(exact) < 0 ? -0.0f : 0.0f)
            : (float)exact;
  }
  return p;
}

// x86 cvttss2si
__device__ __forceinline__ int32_t cvtt(float v) {
  return fabsf(v) < 2147483648.0f ? (int32_t)v : INT32_MIN;
}

// Scale and reciprocal of one activation row from its amax
// (gemma.c:2616-2617 as gcc -ffast-math evaluates it: scale = amax*(1/127),
// inv = 127/amax; both 1 when amax == 0).  The division is done in double:
// a 53-bit quotient rounded to 24 bits equals the correctly rounded float
// quotient (double rounding is innocuous for p' >= 2p+2).
struct QuantParams {
  float scale;
  float inv;
};

__device__ __forceinline__ QuantParams quant_params(float amax) {
  QuantParams qp;
  if (amax > 0.0f) {
    qp.scale = mul_ftz(amax, 1.0f / 127.0f);
    qp.inv = (float)(127.0 / (double)amax);
  } else {
    qp.scale = 1.0f;
    qp.inv = 1.0f;
  }
  return qp;
}

// One quantized element (gemma.c:2625-2633 and 2642-2646):
// q = clamp(trunc(v*inv + copysign(0.5, v*inv)), -127, 127)
__device__ __forceinline__ int32_t quant_one(float v, float inv) {
  float x = daz(v) * inv;
  float t = x + copysignf(0.5f, x);
  int32_t q = cvtt(t);
  return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// |v| with DAZ, for the exact amax reduction (gemma.c:2596-2615)
__device__ __forceinline__ float abs_daz(float v) { return fabsf(daz(v)); }

// Rescale of one int32 accumulator: (float)acc * (act_scale * w_scale)
__device__ __forceinline__ float rescale(int32_t acc, float act_scale,
                                         float w_scale) {
  return mul_ftz((float)acc, mul_ftz(act_scale, w_scale));
}

// True when act_scale*w_scale can take the plain IEEE path in rescale():
// neither scale is subnormal (DAZ would zero it) and their product is not a
// nonzero value at or below FLT_MIN (FTZ territory).  Then for every int32
// acc, |acc*p| >= |p| (acc == 0 gives an exact signed zero), so
// (float)acc * p equals the FTZ/DAZ result bit for bit.
__device__ __forceinline__ bool rescale_is_plain(float act_scale, float w_scale) {
  const float p = act_scale * w_scale;
  return daz(act_scale) == act_scale && daz(w_scale) == w_scale &&
         (p == 0.0f || fabsf(p) > 1.17549435e-38f);
}

// rescale_is_plain() for every pair of a set of activation scales and a set
// of weight scales, from their extremes: plain unless some scale is
// subnormal or the smallest nonzero |product| is at or below FLT_MIN.
// mins are the smallest nonzero magnitudes (+inf when all are zero) and
// sub flags a subnormal scale.
__device__ __forceinline__ bool rescale_all_plain(float act_min, bool act_sub,
                                                  float w_min, bool w_sub) {
  return !act_sub && !w_sub && act_min * w_min > 1.17549435e-38f;
}

__device__ __forceinline__ void scale_extremes(float v, float *min_nz, bool *sub) {
  const float a = fabsf(v);
  if (a != 0.0f) *min_nz = fminf(*min_nz, a);
  *sub = *sub || (a != 0.0f && a < 1.17549435e-38f);
}

// Packs four quantized values into one little-endian 32-bit word.
__device__ __forceinline__ uint32_t pack4(int32_t a, int32_t b, int32_t c,
                                          int32_t d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) |
         ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}

// s_waitcnt vmcnt(N): at most N of this wave's vector memory operations
// still outstanding (lgkmcnt and expcnt not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Workgroup barrier for LDS traffic only: this wave's LDS operations are
// complete (lgkmcnt(0)) before the barrier, and nothing moves across it.
// __syncthreads() also waits for the wave's outstanding global loads
// (vmcnt(0)), which would stall a kernel that has weight loads in flight
// behind a reduction over LDS.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited on
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Pins a wave-uniform value to scalar registers.  Choosing one of several
// kernel-argument pointers by a per-lane index otherwise compiles to a
// per-lane load from the argument segment, and its wait also drains every
// global load issued before it.
template <class T>
__device__ __forceinline__ T in_sgpr(T v) {
  asm("" : "+s"(v));
  return v;
}

// a[j] of a four-entry kernel-argument array for a per-lane j, as a chain of
// v_cndmask over copies of the entries pinned to scalar registers.  A select
// over the argument array itself is folded into a per-lane load from the
// argument segment, whose wait drains every global load issued before it.
template <class T>
__device__ __forceinline__ T pick4(T const (&a)[4], int j) {
  T v0 = a[0], v1 = a[1], v2 = a[2], v3 = a[3];
  asm("" : "+s"(v0), "+s"(v1), "+s"(v2), "+s"(v3));
  return j == 3 ? v3 : j == 2 ? v2 : j == 1 ? v1 : v0;
}

// A GemvJobs argument in scalar registers at once: the compiler otherwise
// loads each field where it is first used, and a field read behind a branch
// (a job's end) costs a dependent scalar-memory round trip before the loads
// that follow it can issue.
template <class Jobs>
__device__ __forceinline__ void hold_jobs(const Jobs &j) {
  asm volatile("" ::"s"(j.w[0]), "s"(j.w[1]), "s"(j.w[2]), "s"(j.w[3]), "s"(j.sc[0]),
               "s"(j.sc[1]), "s"(j.sc[2]), "s"(j.sc[3]));
  asm volatile("" ::"s"(j.dst[0]), "s"(j.dst[1]), "s"(j.dst[2]), "s"(j.dst[3]), "s"(j.end[0]),
               "s"(j.end[1]), "s"(j.end[2]), "s"(j.end[3]), "s"(j.njobs));
}

// The global-memory view of a pointer.  After in_sgpr the compiler no longer
// knows a pointer is global, and flat accesses through it count against both
// vmcnt and lgkmcnt, so waits for them cannot be partial.
template <class T>
using gptr = T __attribute__((address_space(1))) *;
template <class T>
__device__ __forceinline__ gptr<T> as_global(T *p) {
  return (gptr<T>)p;
}

// Wavefront (64 lanes) reductions.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// DPP lane moves within rows of 16 lanes (every source lane exists for the
// patterns used here): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror,
// row_mirror.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)b, lane);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// Sum over the 64 lanes of a wave, the same value in every lane.  The order
// of the additions is fixed, so every wave (and every workgroup) that sums
// the same values gets the same bits.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_f64<kDppXor1>(v);
  v += dpp_f64<kDppXor2>(v);
  v += dpp_f64<kDppHalfMirror>(v);
  v += dpp_f64<kDppMirror>(v);
  return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the L consecutive lanes of a row group (L = 8, 16, 32 or 64), in
// a fixed tree: every lane of the group ends with the sum.
template <int L>
__device__ __forceinline__ float group_sum_f32(float v) {
  static_assert(L == 8 || L == 16 || L == 32 || L == 64, "L is 8, 16, 32 or 64");
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppHalfMirror>(v);
  if (L >= 16) v += dpp_f32<kDppMirror>(v);
  if (L >= 32) v += __shfl_xor(v, 16, 64);
  if (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Sum over each aligned group of L lanes (L = 8, 16, 32 or 64), the same
// value in every lane of the group.  Integer sums are exact, so the order
// of the additions does not matter.
template <int L>
__device__ __forceinline__ int32_t group_sum_i32(int32_t v) {
  static_assert(L == 8 || L == 16 || L == 32 || L == 64, "L is 8, 16, 32 or 64");
  v += __builtin_amdgcn_update_dpp(0, v, kDppXor1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppXor2, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppHalfMirror, 0xF, 0xF, false);
  if (L >= 16) v += __builtin_amdgcn_update_dpp(0, v, kDppMirror, 0xF, 0xF, false);
  if (L >= 32) v += __shfl_xor(v, 16, 64);
  if (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Max over the 64 lanes of a wave, the same value in every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppMirror>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Split precision on the bf16 matrix cores: x = p0 + p1 + p2, each piece
// rounded to nearest bf16 from the remainder of the ones before it (the
// subtractions are exact: x and p0 agree in their leading bits, and so do the
// remainder and p1), so the three together carry x's 24 significant bits.
// A product a.b summed from the six piece products whose orders add up to at
// most 2 (a0 b0, a0 b1, a1 b0, a0 b2, a1 b1, a2 b0) drops terms below
// 3 * 2^-24 |a b|; each bf16 x bf16 product is exact in fp32.
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// The pieces of two values a, b, each piece pair packed as a bf16x2 dword (a
// in the low half): one v_cvt_pk_bf16_f32 per piece pair, and each piece's
// fp32 value taken back from the packed dword by a shift or a mask.
struct Bf3x2 {
  uint32_t q0, q1, q2;
};
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, h2));
}
__device__ __forceinline__ float bf16_lo(uint32_t q) { return __uint_as_float(q << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t q) { return __uint_as_float(q & 0xffff0000u); }
__device__ __forceinline__ Bf3x2 split3x2(float a, float b) {
  Bf3x2 r;
  r.q0 = cvt_pk_bf16(a, b);
  const float a1 = a - bf16_lo(r.q0), b1 = b - bf16_hi(r.q0);
  r.q1 = cvt_pk_bf16(a1, b1);
  r.q2 = cvt_pk_bf16(a1 - bf16_lo(r.q1), b1 - bf16_hi(r.q1));
  return r;
}
__device__ __forceinline__ bf8 as_bf8(u4 v) { return __builtin_bit_cast(bf8, v); }

}  // namespace gh
