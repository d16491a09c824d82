/*
 * e2e_shim.h -- forced-included (-include) at the top of the HIP build of the
 * end-to-end harness.  TEST INFRASTRUCTURE ONLY (see e2e_harness.c).
 *
 * The HIP build compiles the reference's gemma.c with the call sites of its
 * forward passes (the "forward passes" section, gemma.c:4386-5595) renamed
 * from quantize_act / quantize_acts / gemv_int8 / gemv_int8_multi / gemm_int8
 * and gemv_fpx / gemv_fpx_multi / gemm_fpx to the GH_ names below; e2e_harness.c defines them on top of the
 * libgemma_hip host entry points.  They are declared here, before any of the
 * reference's types exist, so PerfBench* and GemvJob* travel as void*; the
 * argument order and meaning are the reference's own (gemma.c:2590, 2656,
 * 2770, 2818, 3943).
 */
#ifndef GEMMA_E2E_SHIM_H
#define GEMMA_E2E_SHIM_H

#include <stdbool.h>
#include <stdint.h>

#include "../include/gemma_hip.h"

static float GH_quantize_act(int8_t *dst, const float *vec, int dim,
                             void *perf);
static void GH_quantize_acts(int8_t *dst, float *dsc, const float *src,
                             int sstr, int m, int n, bool omp, int threads,
                             void *perf);
static void GH_gemv_int8(float *dst, const int8_t *mat, const float *matsc,
                         const int8_t *vec, float vsc, int m, int n, bool omp,
                         int threads, void *perf);
static void GH_gemv_int8_multi(const void *jobs, int njobs, const int8_t *vec,
                               float vsc, int n, int threads, void *perf);
static int GH_gemm_int8(float *dst, int dstr, const int8_t *mat, int mstr,
                        const float *matsc, const int8_t *src, int sstr,
                        const float *ssc, int m, int n, int k, bool omp,
                        int threads, void *perf);
/* the fp32 twins (gemma.c:2734, 2840, 3308) */
static void GH_gemv_fpx(float *dst, const float *mat, const float *vec, int m,
                        int n, bool omp, int threads, void *perf);
static void GH_gemv_fpx_multi(const void *jobs, int njobs, const float *vec,
                              int n, int threads, void *perf);
static int GH_gemm_fpx(float *dst, int dstr, const float *mat, int mstr,
                       const float *src, int sstr, int m, int n, int k,
                       bool omp, int threads, void *perf);

#endif
