/*
 * gemma_oracle.h -- CPU restatement of the reference's W8A8 matmul hot path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this; the HIP library never does.
 *
 * Each function restates one reference function of /root/reference/gemma.c as
 * the reference's own build computes it.  The reference Makefile compiles with
 * -O3 -ffast-math (Makefile:106,120), which re-associates the source's
 * arithmetic, and whose start-up code sets FTZ and DAZ in MXCSR.  The
 * restatement writes that effective arithmetic out explicitly and is compiled
 * strictly (-ffp-contract=off, no fast-math), so its results do not depend on
 * the compiler that builds it.
 *
 * Two "flavours" exist because gcc and clang re-associate differently:
 *   GEMMA_ORACLE_GCC   scale = amax*(1/127), inv = 127/amax, y = acc*(xs*ws)
 *   GEMMA_ORACLE_CLANG scale = amax*(1/127), inv = 1/scale,  y = (acc*xs)*ws
 * The gcc flavour is the one the reference's published numbers were built
 * with and is the default everywhere.
 */
#ifndef GEMMA_ORACLE_H
#define GEMMA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { GEMMA_ORACLE_GCC = 0, GEMMA_ORACLE_CLANG = 1 };

/* gemma.c:2586-2650 quantize_act; returns the scale */
float oracle_quantize_act(int8_t *dst, const float *vec, int dim, int flavor);

/* gemma.c:2652-2674 quantize_acts (sstr == 0 means sstr = n) */
void oracle_quantize_acts(int8_t *dst, float *dsc, const float *src, int sstr,
                          int m, int n, int flavor);

/* exact int32 dot product of two int8 rows (the full-K group accumulator) */
int32_t oracle_dot_i8(const int8_t *a, const int8_t *b, int k);

/* dequantization of one accumulator: gemma.c:2762 (gemv_int8_row),
 * 3630 (gemm_int8_scalar_row), 3862 (gemm_int8_flush_block) */
float oracle_rescale(int32_t acc, float act_scale, float w_scale, int flavor);

/* gemma.c:2765-2788 gemv_int8: m = output rows, n = reduction length.
 * acc (nullable) receives the int32 sums. */
void oracle_gemv_int8(float *dst, int32_t *acc, const int8_t *mat,
                      const float *matsc, const int8_t *vec, float vsc, int m,
                      int n, int flavor);

/* gemma.c:3937-4054 gemm_int8: C[i][j] = rescale(sum_l A[i][l]*B[j][l]).
 * Strides of 0 mean dense.  acc (nullable) receives the int32 sums, dense
 * [m][n]. */
void oracle_gemm_int8(float *dst, int dstr, int32_t *acc, const int8_t *mat,
                      int mstr, const float *matsc, const int8_t *src,
                      int sstr, const float *ssc, int m, int n, int k,
                      int flavor);

/* fp32 fallback (gemma.c:2718-2752 gemv_fpx, 3304-3399 gemm_fpx): no
 * bit-exact target exists (the reference's summation order is whatever its
 * compiler vectorises), so the oracle gives the float64 dot product and the
 * float64 sum of |a|*|b| that bounds any fp32 summation's rounding error.
 * Strides of 0 mean dense; dst/absdst are dense [m][n]. */
/* rescale of precomputed int32 sums (the flush, gemma.c:3854-3865) */
void oracle_rescale_matrix(float *dst, const int32_t *acc, const float *ssc,
                           const float *matsc, int m, int n, int flavor);

void oracle_gemm_f64(double *dst, double *absdst, const float *mat, int mstr,
                     const float *src, int sstr, int m, int n, int k);

/* gemma.c:4411-4448, the SigLIP patch embedding, in float64: dst and
 * absdst are [npatch][dim] with npatch = (img_px/psize)^2; dst = bias +
 * sum over (py, px, c) of pe[oc][c][py][px] * img[oy*P+py][ox*P+px][c],
 * absdst = |bias| + the sum of |products| (the fp32 rounding bound). */
void oracle_patch_embed_f64(double *dst, double *absdst, const float *img,
                            const float *pe, const float *pe_b, int img_px,
                            int psize, int dim);

#ifdef __cplusplus
}
#endif

#endif
