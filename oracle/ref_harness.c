/*
 * ref_harness.c -- drives the REFERENCE's own hot-path functions, compiled from
 * /root/reference/gemma.c where it lies (never copied).  TEST INFRASTRUCTURE
 * ONLY: it is the oracle's cross-check and the "reference" CPU baseline of
 * bench.py.  Nothing in the product links or runs it.
 *
 * The reference's functions are `static`, so this translation unit includes
 * gemma.c and calls them directly.  The include sits on top of the file and
 * everything below it uses identifiers of three characters or more: the stb
 * blob at the end of gemma.c (gemma.c:7494-8769) defines ~200 one- and
 * two-letter macros that would otherwise rewrite this code.
 *
 * It is built as an executable, not a shared library, so that gcc's
 * -ffast-math start-up code (crtfastmath: FTZ + DAZ in MXCSR) runs exactly as
 * it does for the reference's own `gemma` binary, and so that loading it can
 * never change the floating-point mode of a test process.
 *
 * Usage:
 *   gemma_ref <op> <input-file> <output-file> [integer params...]
 * Inputs and outputs are raw little-endian arrays laid back to back, in the
 * order documented for each op in run_op() below.
 *   gemma_ref bench <op> [integer params...]
 * runs the op on synthetic data and prints one JSON line with the time per
 * call (see run_bench()).
 */
#define main gemma_reference_main
#include GEMMA_REF_SOURCE
#undef main

/* ---- everything below: identifiers of length >= 3 only ------------------ */

static unsigned char *input_base;
static size_t input_size;
static size_t input_cursor;

static void *take_input(size_t nbytes) {
  if (input_cursor + nbytes > input_size) {
    fprintf(stderr, "gemma_ref: input file too short (need %zu more bytes)\n",
            input_cursor + nbytes - input_size);
    exit(2);
  }
  void *ptr = input_base + input_cursor;
  input_cursor += nbytes;
  return ptr;
}

static void *alloc_or_die(size_t nbytes) {
  void *ptr = calloc(nbytes > 0 ? nbytes : 1, 1);
  if (ptr == NULL) {
    fprintf(stderr, "gemma_ref: out of memory (%zu bytes)\n", nbytes);
    exit(2);
  }
  return ptr;
}

static void load_input(const char *path) {
  FILE *file = fopen(path, "rb");
  if (file == NULL) {
    fprintf(stderr, "gemma_ref: cannot open %s\n", path);
    exit(2);
  }
  fseek(file, 0, SEEK_END);
  long length = ftell(file);
  fseek(file, 0, SEEK_SET);
  input_size = (size_t)(length > 0 ? length : 0);
  input_base = alloc_or_die(input_size);
  if (input_size > 0 && fread(input_base, 1, input_size, file) != input_size) {
    fprintf(stderr, "gemma_ref: short read on %s\n", path);
    exit(2);
  }
  fclose(file);
  input_cursor = 0;
}

static FILE *output_file;

static void put_output(const void *ptr, size_t nbytes) {
  if (nbytes > 0 && fwrite(ptr, 1, nbytes, output_file) != nbytes) {
    fprintf(stderr, "gemma_ref: short write\n");
    exit(2);
  }
}

static int param_at(int argc, char **argv, int index) {
  if (index >= argc) {
    fprintf(stderr, "gemma_ref: missing integer parameter #%d\n", index);
    exit(2);
  }
  return atoi(argv[index]);
}

static int thread_count(void) {
  const char *env = getenv("OMP_NUM_THREADS");
  int value = env != NULL ? atoi(env) : 0;
  return value > 0 ? value : 1;
}

/*
 * ops (P = integer params after the file names):
 *  quantize_act     P: dim                in: f32[dim]
 *                   out: i8[dim], f32 scale                  (gemma.c:2590)
 *  quantize_acts    P: rows cols sstr omp in: f32[rows*sstr]
 *                   out: i8[rows*cols], f32[rows]            (gemma.c:2656)
 *  gemv_int8        P: nout kin omp       in: i8[nout*kin], f32[nout],
 *                   i8[kin], f32 vsc       out: f32[nout]     (gemma.c:2770)
 *  gemv_int8_multi  P: kin njobs nout_0..  in: per job i8[nout*kin],
 *                   f32[nout]; then i8[kin], f32 vsc
 *                   out: f32[sum nout] in job order          (gemma.c:2818)
 *  gemm_int8        P: rows nout kin dstr mstr sstr omp
 *                   in: i8[nout*mstr], f32[nout], i8[rows*sstr], f32[rows],
 *                   f32[rows*dstr] (initial dst)
 *                   out: f32[rows*dstr], i32 return code     (gemma.c:3943)
 *  gemv_fpx         P: nout kin omp       in: f32[nout*kin], f32[kin]
 *                   out: f32[nout]                           (gemma.c:2734)
 *  gemv_fpx_multi   P: kin njobs nout_0.. in: per job f32[nout*kin];
 *                   then f32[kin]          out: f32[sum nout] (gemma.c:2840)
 *  gemm_fpx         P: rows nout kin dstr mstr sstr omp
 *                   in: f32[nout*mstr], f32[rows*sstr], f32[rows*dstr]
 *                   out: f32[rows*dstr], i32 return code     (gemma.c:3308)
 */
static int run_op(const char *opname_arg, int argc, char **argv) {
  int threads = thread_count();

  if (strcmp(opname_arg, "quantize_act") == 0) {
    int dim = param_at(argc, argv, 4);
    float *vec = take_input((size_t)dim * 4);
    int8_t *qout = alloc_or_die((size_t)dim);
    float scale = quantize_act(qout, vec, dim, NULL);
    put_output(qout, (size_t)dim);
    put_output(&scale, 4);
    return 0;
  }
  if (strcmp(opname_arg, "quantize_acts") == 0) {
    int rows = param_at(argc, argv, 4), cols = param_at(argc, argv, 5);
    int sstr = param_at(argc, argv, 6), use_omp = param_at(argc, argv, 7);
    int stride = sstr == 0 ? cols : sstr;
    float *src = take_input((size_t)rows * stride * 4);
    int8_t *qout = alloc_or_die((size_t)rows * cols);
    float *scales = alloc_or_die((size_t)rows * 4);
    quantize_acts(qout, scales, src, sstr, rows, cols, use_omp != 0, threads,
                  NULL);
    put_output(qout, (size_t)rows * cols);
    put_output(scales, (size_t)rows * 4);
    return 0;
  }
  if (strcmp(opname_arg, "gemv_int8") == 0) {
    int nout = param_at(argc, argv, 4), kin = param_at(argc, argv, 5);
    int use_omp = param_at(argc, argv, 6);
    int8_t *mat = take_input((size_t)nout * kin);
    float *matsc = take_input((size_t)nout * 4);
    int8_t *vec = take_input((size_t)kin);
    float vsc = *(float *)take_input(4);
    float *dst = alloc_or_die((size_t)nout * 4);
    gemv_int8(dst, mat, matsc, vec, vsc, nout, kin, use_omp != 0, threads,
              NULL);
    put_output(dst, (size_t)nout * 4);
    return 0;
  }
  if (strcmp(opname_arg, "gemv_int8_multi") == 0 ||
      strcmp(opname_arg, "gemv_fpx_multi") == 0) {
    int is_int8 = strcmp(opname_arg, "gemv_int8_multi") == 0;
    int kin = param_at(argc, argv, 4), njobs = param_at(argc, argv, 5);
    GemvJob jobs[8];
    int total = 0;
    if (njobs < 1 || njobs > 8) {
      fprintf(stderr, "gemma_ref: njobs out of range\n");
      return 2;
    }
    for (int job = 0; job < njobs; job++) {
      int nout = param_at(argc, argv, 6 + job);
      if (is_int8) {
        jobs[job].w = take_input((size_t)nout * kin);
        jobs[job].sc = take_input((size_t)nout * 4);
      } else {
        jobs[job].w = take_input((size_t)nout * kin * 4);
        jobs[job].sc = NULL;
      }
      jobs[job].m = nout;
      total += nout;
    }
    float *dst = alloc_or_die((size_t)total * 4);
    int offset = 0;
    for (int job = 0; job < njobs; job++) {
      jobs[job].dst = dst + offset;
      offset += jobs[job].m;
    }
    if (is_int8) {
      int8_t *vec = take_input((size_t)kin);
      float vsc = *(float *)take_input(4);
      gemv_int8_multi(jobs, njobs, vec, vsc, kin, threads, NULL);
    } else {
      float *vec = take_input((size_t)kin * 4);
      gemv_fpx_multi(jobs, njobs, vec, kin, threads, NULL);
    }
    put_output(dst, (size_t)total * 4);
    return 0;
  }
  if (strcmp(opname_arg, "gemm_int8") == 0 ||
      strcmp(opname_arg, "gemm_fpx") == 0) {
    int is_int8 = strcmp(opname_arg, "gemm_int8") == 0;
    int rows = param_at(argc, argv, 4), nout = param_at(argc, argv, 5);
    int kin = param_at(argc, argv, 6), dstr = param_at(argc, argv, 7);
    int mstr = param_at(argc, argv, 8), sstr = param_at(argc, argv, 9);
    int use_omp = param_at(argc, argv, 10);
    int dst_stride = dstr == 0 ? nout : dstr;
    int mat_stride = mstr == 0 ? kin : mstr;
    int src_stride = sstr == 0 ? kin : sstr;
    size_t dst_bytes = (size_t)rows * dst_stride * 4;
    int status;
    float *dst = alloc_or_die(dst_bytes);
    if (is_int8) {
      int8_t *mat = take_input((size_t)nout * mat_stride);
      float *matsc = take_input((size_t)nout * 4);
      int8_t *src = take_input((size_t)rows * src_stride);
      float *ssc = take_input((size_t)rows * 4);
      memcpy(dst, take_input(dst_bytes), dst_bytes);
      status = gemm_int8(dst, dstr, mat, mstr, matsc, src, sstr, ssc, rows,
                         nout, kin, use_omp != 0, threads, NULL);
    } else {
      float *mat = take_input((size_t)nout * mat_stride * 4);
      float *src = take_input((size_t)rows * src_stride * 4);
      memcpy(dst, take_input(dst_bytes), dst_bytes);
      status = gemm_fpx(dst, dstr, mat, mstr, src, sstr, rows, nout, kin,
                        use_omp != 0, threads, NULL);
    }
    put_output(dst, dst_bytes);
    put_output(&status, 4);
    return 0;
  }
  if (strcmp(opname_arg, "gemv_fpx") == 0) {
    int nout = param_at(argc, argv, 4), kin = param_at(argc, argv, 5);
    int use_omp = param_at(argc, argv, 6);
    float *mat = take_input((size_t)nout * kin * 4);
    float *vec = take_input((size_t)kin * 4);
    float *dst = alloc_or_die((size_t)nout * 4);
    gemv_fpx(dst, mat, vec, nout, kin, use_omp != 0, threads, NULL);
    put_output(dst, (size_t)nout * 4);
    return 0;
  }
  fprintf(stderr, "gemma_ref: unknown op %s\n", opname_arg);
  return 2;
}

/* ---- timing mode --------------------------------------------------------- */

static uint64_t lcg_state = 0x9E3779B97F4A7C15ull;

static uint32_t lcg_next(void) {
  lcg_state = lcg_state * 6364136223846793005ull + 1442695040888963407ull;
  return (uint32_t)(lcg_state >> 33);
}

static void fill_int8(int8_t *ptr, size_t count) {
  for (size_t idx = 0; idx < count; idx++)
    ptr[idx] = (int8_t)((int)(lcg_next() % 255u) - 127);
}

static void fill_float(float *ptr, size_t count, float low, float high) {
  for (size_t idx = 0; idx < count; idx++)
    ptr[idx] = low + (high - low) * (float)(lcg_next() & 0xFFFFFF) / 16777216.0f;
}

/*
 * bench gemv_int8 <nout> <kin> <copies> <min_calls>
 *   W8A8 GEMV (quantize_act + gemv_int8, as at the decode call sites
 *   gemma.c:4858-4859) over `copies` distinct weight matrices in rotation.
 * bench gemv_int8_multi <kin> <copies> <min_calls> <njobs> <nout_0> ...
 *   quantize_act + gemv_int8_multi over njobs matrices, as at the decode q/k/v
 *   and gate/up call sites (gemma.c:4768-4773, 4911-4915).
 * bench gemm_int8 <rows> <nout> <kin> <min_calls>
 *   quantize_acts + gemm_int8 (prefill call sites gemma.c:5365-5370).
 * Prints {"op":..., "calls":..., "seconds":..., "threads":...}.
 */
static int run_bench(int argc, char **argv) {
  const char *what = argc > 2 ? argv[2] : "";
  int threads = thread_count();

  if (strcmp(what, "gemv_int8") == 0) {
    int nout = param_at(argc, argv, 3), kin = param_at(argc, argv, 4);
    int copies = param_at(argc, argv, 5), min_calls = param_at(argc, argv, 6);
    int8_t *weights = alloc_or_die((size_t)copies * nout * kin);
    float *scales = alloc_or_die((size_t)copies * nout * 4);
    float *activ = alloc_or_die((size_t)kin * 4);
    int8_t *qact = alloc_or_die((size_t)kin);
    float *dst = alloc_or_die((size_t)nout * 4);
    fill_int8(weights, (size_t)copies * nout * kin);
    fill_float(scales, (size_t)copies * nout, 1e-3f, 1e-2f);
    fill_float(activ, (size_t)kin, -3.0f, 3.0f);
    for (int warm = 0; warm < 2; warm++) {
      float vsc = quantize_act(qact, activ, kin, NULL);
      gemv_int8(dst, weights, scales, qact, vsc, nout, kin, true, threads,
                NULL);
    }
    double start = now_sec();
    int calls = 0;
    while (calls < min_calls) {
      int copy = calls % copies;
      float vsc = quantize_act(qact, activ, kin, NULL);
      gemv_int8(dst, weights + (size_t)copy * nout * kin,
                scales + (size_t)copy * nout, qact, vsc, nout, kin, true,
                threads, NULL);
      calls++;
    }
    double seconds = now_sec() - start;
    printf("{\"op\": \"gemv_int8\", \"nout\": %d, \"kin\": %d, \"calls\": %d, "
           "\"seconds\": %.6f, \"threads\": %d, \"checksum\": %.6e}\n",
           nout, kin, calls, seconds, threads, (double)dst[nout / 2]);
    return 0;
  }
  if (strcmp(what, "gemv_int8_multi") == 0) {
    int kin = param_at(argc, argv, 3), copies = param_at(argc, argv, 4);
    int min_calls = param_at(argc, argv, 5), njobs = param_at(argc, argv, 6);
    if (njobs < 1 || njobs > 8 || copies < 1) {
      fprintf(stderr, "gemma_ref: njobs or copies out of range\n");
      return 2;
    }
    int nouts[8], total = 0;
    for (int job = 0; job < njobs; job++) {
      nouts[job] = param_at(argc, argv, 7 + job);
      total += nouts[job];
    }
    int8_t *weights = alloc_or_die((size_t)copies * total * kin);
    float *scales = alloc_or_die((size_t)copies * total * 4);
    float *activ = alloc_or_die((size_t)kin * 4);
    int8_t *qact = alloc_or_die((size_t)kin);
    float *dst = alloc_or_die((size_t)total * 4);
    fill_int8(weights, (size_t)copies * total * kin);
    fill_float(scales, (size_t)copies * total, 1e-3f, 1e-2f);
    fill_float(activ, (size_t)kin, -3.0f, 3.0f);
    GemvJob jobs[8];
    double start = 0.0;
    int calls = 0;
    for (int iter = -2; iter < min_calls; iter++) {  /* two warm-up calls */
      if (iter == 0) start = now_sec();
      int copy = (iter + 2) % copies, row = 0;
      for (int job = 0; job < njobs; job++) {
        jobs[job].w = weights + ((size_t)copy * total + row) * kin;
        jobs[job].sc = scales + (size_t)copy * total + row;
        jobs[job].dst = dst + row;
        jobs[job].m = nouts[job];
        row += nouts[job];
      }
      float vsc = quantize_act(qact, activ, kin, NULL);
      gemv_int8_multi(jobs, njobs, qact, vsc, kin, threads, NULL);
      if (iter >= 0) calls++;
    }
    double seconds = now_sec() - start;
    printf("{\"op\": \"gemv_int8_multi\", \"kin\": %d, \"njobs\": %d, \"calls\": %d, "
           "\"seconds\": %.6f, \"threads\": %d, \"checksum\": %.6e}\n",
           kin, njobs, calls, seconds, threads, (double)dst[total / 2]);
    return 0;
  }
  if (strcmp(what, "gemm_int8") == 0) {
    int rows = param_at(argc, argv, 3), nout = param_at(argc, argv, 4);
    int kin = param_at(argc, argv, 5), min_calls = param_at(argc, argv, 6);
    int8_t *weights = alloc_or_die((size_t)nout * kin);
    float *scales = alloc_or_die((size_t)nout * 4);
    float *activ = alloc_or_die((size_t)rows * kin * 4);
    int8_t *qact = alloc_or_die((size_t)rows * kin);
    float *qsc = alloc_or_die((size_t)rows * 4);
    float *dst = alloc_or_die((size_t)rows * nout * 4);
    fill_int8(weights, (size_t)nout * kin);
    fill_float(scales, (size_t)nout, 1e-3f, 1e-2f);
    fill_float(activ, (size_t)rows * kin, -3.0f, 3.0f);
    quantize_acts(qact, qsc, activ, 0, rows, kin, true, threads, NULL);
    gemm_int8(dst, 0, weights, 0, scales, qact, 0, qsc, rows, nout, kin, true,
              threads, NULL);
    double start = now_sec();
    int calls = 0;
    while (calls < min_calls) {
      quantize_acts(qact, qsc, activ, 0, rows, kin, true, threads, NULL);
      gemm_int8(dst, 0, weights, 0, scales, qact, 0, qsc, rows, nout, kin,
                true, threads, NULL);
      calls++;
    }
    double seconds = now_sec() - start;
    printf("{\"op\": \"gemm_int8\", \"rows\": %d, \"nout\": %d, \"kin\": %d, "
           "\"calls\": %d, \"seconds\": %.6f, \"threads\": %d}\n",
           rows, nout, kin, calls, seconds, threads);
    return 0;
  }
  fprintf(stderr, "gemma_ref: unknown bench %s\n", what);
  return 2;
}

int main(int argc, char **argv) {
  if (argc >= 2 && strcmp(argv[1], "bench") == 0)
    return run_bench(argc, argv);
  if (argc < 4) {
    fprintf(stderr, "usage: gemma_ref <op> <in> <out> [params...]\n"
                    "       gemma_ref bench <op> [params...]\n");
    return 2;
  }
  load_input(argv[2]);
  output_file = fopen(argv[3], "wb");
  if (output_file == NULL) {
    fprintf(stderr, "gemma_ref: cannot create %s\n", argv[3]);
    return 2;
  }
  int status = run_op(argv[1], argc, argv);
  fclose(output_file);
  return status;
}
