/*
 * gemma_oracle.c -- CPU restatement of the reference's W8A8 hot path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT (see gemma_oracle.h).  Plain C, scalar,
 * single-threaded, compiled with -ffp-contract=off and without fast-math.
 *
 * The reference's floating-point environment is restated explicitly:
 *  - DAZ: a subnormal input operand counts as a zero of the same sign.
 *  - FTZ: a product that is tiny becomes a zero of its sign.  x86 detects
 *    tininess after rounding to 24 bits with an unbounded exponent: a product
 *    just below FLT_MIN that rounds up to FLT_MIN survives, while one that is
 *    exactly representable below FLT_MIN is flushed even where gradual
 *    underflow would have rounded it up to FLT_MIN.  float*float is exact in
 *    double; scaling it by 2^64 before the conversion to float gives the
 *    24-bit rounding without the exponent limit.
 *  - cvttss2si: NaN, infinities and out-of-range values convert to INT_MIN
 *    ("integer indefinite"), which the clamp then maps to -127.
 */
#include "gemma_oracle.h"

#include <float.h>
#include <math.h>
#include <string.h>

static float daz(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof(bits));
  if ((bits & 0x7f800000u) == 0) {
    bits &= 0x80000000u;
    memcpy(&value, &bits, sizeof(bits));
  }
  return value;
}

/* a*b rounded to float under FTZ/DAZ; the double product is exact */
static float mul_ftz(float a, float b) {
  double exact = (double)daz(a) * (double)daz(b);
  float scaled = (float)(exact * 0x1p64); /* 2^64 * FLT_MIN = 2^-62 */
  if (fabsf(scaled) < 0x1p-62f) {
    return signbit(exact) ? -0.0f : 0.0f;
  }
  return (float)exact;
}

/* x86 cvttss2si */
static int32_t cvtt(float value) {
  if (!(fabsf(value) < 2147483648.0f)) {
    return INT32_MIN;
  }
  return (int32_t)value;
}

/* gemma.c:2590-2650.  The reference computes amax with an exact max over
 * |v| (2596-2615), then scale = amax/127 and inv = 1/scale (2616-2617) which
 * gcc -ffast-math evaluates as amax*(1/127) and 127/amax, and clang as
 * amax*(1/127) and 1/(amax*(1/127)); a zero amax gives scale = inv = 1.
 * q = (int)(v*inv + copysign(0.5, v*inv)) clamped to [-127, 127]
 * (2625-2633, 2642-2646). */
float oracle_quantize_act(int8_t *dst, const float *vec, int dim, int flavor) {
  float amax = 0.0f;
  for (int d = 0; d < dim; d++) {
    float mag = fabsf(daz(vec[d]));
    if (mag > amax) {
      amax = mag;
    }
  }

  float scale = 1.0f;
  float inv = 1.0f;
  if (amax > 0.0f) {
    scale = mul_ftz(amax, 1.0f / 127.0f);
    if (flavor == GEMMA_ORACLE_CLANG) {
      inv = (float)(1.0 / (double)scale); /* 1/0 -> inf, as on x86 */
    } else {
      inv = (float)(127.0 / (double)amax);
    }
  }

  for (int d = 0; d < dim; d++) {
    /* |x| < FLT_MIN gives q = 0 whether or not it is flushed, and
     * 0*inf = NaN as on x86, so a plain float multiply is exact enough */
    float x = daz(vec[d]) * inv;
    float t = x + copysignf(0.5f, x);
    int32_t q = cvtt(t);
    dst[d] = (int8_t)(q > 127 ? 127 : (q < -127 ? -127 : q));
  }
  return scale;
}

/* gemma.c:2656-2674 */
void oracle_quantize_acts(int8_t *dst, float *dsc, const float *src, int sstr,
                          int m, int n, int flavor) {
  if (sstr == 0) {
    sstr = n;
  }
  for (int i = 0; i < m; i++) {
    dsc[i] = oracle_quantize_act(dst + (size_t)i * n, src + (size_t)i * sstr,
                                 n, flavor);
  }
}

/* gemma.c:2757-2761 and 3624-3628: int32 sum of int8 products */
int32_t oracle_dot_i8(const int8_t *a, const int8_t *b, int k) {
  int32_t sum = 0;
  for (int l = 0; l < k; l++) {
    sum += (int32_t)a[l] * (int32_t)b[l];
  }
  return sum;
}

/* gemma.c:2762, 3629, 3862: the source writes (float)acc * xs * ws; gcc
 * -ffast-math evaluates acc*(xs*ws), clang (acc*xs)*ws */
float oracle_rescale(int32_t acc, float act_scale, float w_scale, int flavor) {
  if (flavor == GEMMA_ORACLE_CLANG) {
    return mul_ftz(mul_ftz((float)acc, act_scale), w_scale);
  }
  return mul_ftz((float)acc, mul_ftz(act_scale, w_scale));
}

/* gemma.c:2765-2788 */
void oracle_gemv_int8(float *dst, int32_t *acc, const int8_t *mat,
                      const float *matsc, const int8_t *vec, float vsc, int m,
                      int n, int flavor) {
  for (int i = 0; i < m; i++) {
    int32_t sum = oracle_dot_i8(mat + (size_t)i * n, vec, n);
    if (acc != NULL) {
      acc[i] = sum;
    }
    dst[i] = oracle_rescale(sum, vsc, matsc[i], flavor);
  }
}

/* gemma.c:3937-4054.  The reference splits the work into 8x8-aligned
 * micro-tiles and scalar remainders (4035-4044), but every cell gets the same
 * integer sum and the same rescale (measured: 0 mismatches between the
 * remainder path and the tile path), so the restatement is one loop nest.
 * Cells of dst outside [m][n] (the stride gap) are left untouched. */
void oracle_gemm_int8(float *dst, int dstr, int32_t *acc, const int8_t *mat,
                      int mstr, const float *matsc, const int8_t *src,
                      int sstr, const float *ssc, int m, int n, int k,
                      int flavor) {
  if (dstr == 0) {
    dstr = n;
  }
  if (mstr == 0) {
    mstr = k;
  }
  if (sstr == 0) {
    sstr = k;
  }
  for (int i = 0; i < m; i++) {
    for (int j = 0; j < n; j++) {
      int32_t sum = oracle_dot_i8(src + (size_t)i * sstr,
                                  mat + (size_t)j * mstr, k);
      if (acc != NULL) {
        acc[(size_t)i * n + j] = sum;
      }
      dst[(size_t)i * dstr + j] = oracle_rescale(sum, ssc[i], matsc[j], flavor);
    }
  }
}

/* The flush of gemm_int8 (gemma.c:3854-3865, scalar tails 3617-3634) over a
 * matrix of int32 sums computed elsewhere: dst[i][j] = rescale(acc[i][j],
 * ssc[i], matsc[j]).  Lets a test form the exact sums of a large product with
 * any exact method and still take every rounding step from this file. */
void oracle_rescale_matrix(float *dst, const int32_t *acc, const float *ssc,
                           const float *matsc, int m, int n, int flavor) {
  for (int i = 0; i < m; i++) {
    for (int j = 0; j < n; j++) {
      dst[(size_t)i * n + j] =
          oracle_rescale(acc[(size_t)i * n + j], ssc[i], matsc[j], flavor);
    }
  }
}

/* gemma.c:2718-2728 / 3074-3112 / 3154-3302, in float64 */
void oracle_gemm_f64(double *dst, double *absdst, const float *mat, int mstr,
                     const float *src, int sstr, int m, int n, int k) {
  if (mstr == 0) {
    mstr = k;
  }
  if (sstr == 0) {
    sstr = k;
  }
  for (int i = 0; i < m; i++) {
    for (int j = 0; j < n; j++) {
      const float *arow = src + (size_t)i * sstr;
      const float *brow = mat + (size_t)j * mstr;
      double sum = 0.0, mag = 0.0;
      for (int l = 0; l < k; l++) {
        double prod = (double)arow[l] * (double)brow[l];
        sum += prod;
        mag += fabs(prod);
      }
      dst[(size_t)i * n + j] = sum;
      if (absdst != NULL) {
        absdst[(size_t)i * n + j] = mag;
      }
    }
  }
}

/* gemma.c:4419-4447: loops patch (oy, ox), out channel, py, px, c */
void oracle_patch_embed_f64(double *dst, double *absdst, const float *img,
                            const float *pe, const float *pe_b, int img_px,
                            int psize, int dim) {
  int ppi = img_px / psize;
  int idim = 3 * psize * psize;
  for (int pi = 0; pi < ppi * ppi; pi++) {
    int oy = pi / ppi, ox = pi % ppi;
    for (int oc = 0; oc < dim; oc++) {
      double sum = 0.0, mag = 0.0;
      for (int py = 0; py < psize; py++) {
        for (int px = 0; px < psize; px++) {
          for (int c = 0; c < 3; c++) {
            size_t in_idx = ((size_t)(oy * psize + py) * img_px + (ox * psize + px)) * 3 + c;
            size_t w_idx = (size_t)oc * idim + c * psize * psize + py * psize + px;
            double prod = (double)pe[w_idx] * (double)img[in_idx];
            sum += prod;
            mag += fabs(prod);
          }
        }
      }
      dst[(size_t)pi * dim + oc] = sum + (double)pe_b[oc];
      absdst[(size_t)pi * dim + oc] = mag + fabs((double)pe_b[oc]);
    }
  }
}
