/*
 * e2e_harness.c -- greedy generation through the REFERENCE program, built
 * twice from /root/reference/gemma.c where it lies (never copied).  TEST
 * INFRASTRUCTURE ONLY: the product is libgemma_hip; this harness shows it is
 * a drop-in at the reference's own call sites.
 *
 *   gemma_e2e_cpu  the reference source as it is: every quantize and int8
 *                  matmul runs on the CPU (the reference's own kernels).
 *   gemma_e2e_hip  the same source with the forward passes' calls to
 *                  quantize_act, quantize_acts, gemv_int8, gemv_int8_multi
 *                  and gemm_int8, and to the fp32 twins gemv_fpx,
 *                  gemv_fpx_multi and gemm_fpx (unquantized 'U' model
 *                  files), renamed to the GH_ shims below (the rename
 *                  is a sed script applied while the source is piped into
 *                  the compiler, e2e_retarget.sed), which call the library's
 *                  host entry points.  Everything else -- embedding, norms,
 *                  RoPE, attention, GELU, residuals, argmax -- is the
 *                  reference's code in both builds, compiled with the same
 *                  flags.
 *
 * Because the library's quantize and int8 matmul results are bit-identical
 * to the reference's, both builds must produce the same logits, bit for bit,
 * at every step, and so the same greedy token stream, on a W8A8 ('Q')
 * file.  On an fp32 ('U') file the sums' order differs (the reference's is
 * its compiler's), so the logits agree to fp32 rounding, not bit for bit.
 *
 * The run follows sample() (gemma.c:5978-6075) with temperature 0: prefill
 * <bos> without logits (6010-6014), prefill the prompt with logits, then
 * decode one token per step; the next token is argmax(logits) (5600-5630).
 * The prompt is `prompt_len` ids drawn uniformly from [0, nvocab) by
 * splitmix64 (Steele, Lea and Flood, "Fast splittable pseudorandom number
 * generators", OOPSLA 2014) seeded with `seed`.
 *
 * Usage:
 *   gemma_e2e <model.bin> <prompt_len> <decode_steps> <seed> <threads> [chunk]
 * prints one JSON line: the generated tokens, an FNV-1a hash of the bits of
 * every step's logits, and the wall time of each phase.
 *
 * Environment:
 *   GEMMA_E2E_DECODE_ONLY=1  feed <bos> and the prompt one token at a time
 *                            through forward_gemma_decode instead of the
 *                            chunked prefill (the decode path at every
 *                            position, as the device-resident decoder runs)
 *   GEMMA_E2E_LOGITS=<path>  write every step's logits (nvocab float32 each,
 *                            in step order) to <path>
 *   GEMMA_E2E_VISION_IMAGE=<path>, GEMMA_E2E_VISION_OUT=<path>
 *                            (CPU build, multimodal model) instead of the text
 *                            run: read the image (float32 [img_px][img_px][3],
 *                            normalized as gemma.c:4271-4273 leaves it) from the
 *                            first file, run forward_vision (4394-4725) and
 *                            write the image's soft tokens (float32 [img_tok]
 *                            [dim], tb->x) to the second
 *   GEMMA_E2E_IMAGE=<path>   (CPU build, multimodal model) an image prompt, as
 *                            sample() (5978-6075) takes one: prefill <bos>,
 *                            then forward_gemma_image (5561-5595: the vision
 *                            tower, then its soft tokens through the decoder
 *                            with mask=false), then the text prompt (chunked
 *                            prefill), then the decode steps.  The logits
 *                            after the image, after the prompt and after each
 *                            step go to GEMMA_E2E_LOGITS (required here)
 *
 * Everything below the include uses identifiers of three characters or more
 * (the stb blob at the end of gemma.c defines one- and two-letter macros,
 * among them `x`), and touches no struct field of one or two letters that
 * the blob redefines.
 */
#define main gemma_reference_main
#include GEMMA_REF_SOURCE
#undef main

#include <inttypes.h>

static void die_with(const char *what, const char *detail) {
  fprintf(stderr, "gemma_e2e: %s: %s\n", what, detail);
  exit(3);
}

#ifdef GEMMA_E2E_HIP

static void hip_or_die(int status, const char *what) {
  if (status != 0) {
    die_with(what, gemma_hip_last_error());
  }
}

/* quantize_act (gemma.c:2590) */
static float GH_quantize_act(int8_t *dst, const float *vec, int dim,
                             void *perf_any) {
  PerfBench *perf = perf_any;
  double tic = PERF_TIC(perf);
  float scale = 1.0f;
  hip_or_die(gemma_hip_quantize_act_host(dst, &scale, vec, dim),
             "quantize_act");
  PERF_TOC(perf, PERF_OP_QUANTIZE_ACT, tic);
  return scale;
}

/* quantize_acts (gemma.c:2656); the reference times each row as one
 * quantize_act call, this times the batch as one */
static void GH_quantize_acts(int8_t *dst, float *dsc, const float *src,
                             int sstr, int rows, int cols, bool omp,
                             int threads, void *perf_any) {
  (void)omp;
  (void)threads;
  PerfBench *perf = perf_any;
  double tic = PERF_TIC(perf);
  hip_or_die(gemma_hip_quantize_acts_host(dst, dsc, src, sstr, rows, cols),
             "quantize_acts");
  PERF_TOC(perf, PERF_OP_QUANTIZE_ACT, tic);
}

/* gemv_int8 (gemma.c:2770) */
static void GH_gemv_int8(float *dst, const int8_t *mat, const float *matsc,
                         const int8_t *vec, float vsc, int rows, int cols,
                         bool omp, int threads, void *perf_any) {
  (void)omp;
  (void)threads;
  PerfBench *perf = perf_any;
  double tic = PERF_TIC(perf);
  hip_or_die(gemma_hip_gemv_int8_host(dst, mat, matsc, vec, vsc, rows, cols),
             "gemv_int8");
  PERF_TOC(perf, PERF_OP_GEMV_INT8, tic);
}

/* gemv_int8_multi (gemma.c:2818) */
static void GH_gemv_int8_multi(const void *jobs_any, int njobs,
                               const int8_t *vec, float vsc, int cols,
                               int threads, void *perf_any) {
  (void)threads;
  const GemvJob *jobs = jobs_any;
  PerfBench *perf = perf_any;
  double tic = PERF_TIC(perf);
  gemma_hip_job hjobs[GEMMA_HIP_MAX_JOBS];
  if (njobs < 1 || njobs > GEMMA_HIP_MAX_JOBS) {
    die_with("gemv_int8_multi", "too many jobs");
  }
  for (int idx = 0; idx < njobs; idx++) {
    hjobs[idx].w = jobs[idx].w;
    hjobs[idx].sc = jobs[idx].sc;
    hjobs[idx].dst = jobs[idx].dst;
    hjobs[idx].m = jobs[idx].m;
  }
  hip_or_die(gemma_hip_gemv_int8_multi_host(hjobs, njobs, vec, vsc, cols),
             "gemv_int8_multi");
  PERF_TOC(perf, PERF_OP_GEMV_INT8, tic);
}

/* gemm_int8 (gemma.c:3943): 0 = ok, 1 = failure with the message in the
 * reference's error channel, as its callers expect */
static int GH_gemm_int8(float *dst, int dstr, const int8_t *mat, int mstr,
                        const float *matsc, const int8_t *src, int sstr,
                        const float *ssc, int rows, int cols, int depth,
                        bool omp, int threads, void *perf_any) {
  (void)omp;
  (void)threads;
  PerfBench *perf = perf_any;
  double tic = PERF_TIC(perf);
  if (gemma_hip_gemm_int8_host(dst, dstr, mat, mstr, matsc, src, sstr, ssc,
                               rows, cols, depth) != 0) {
    log_error("gemm_int8 (hip): %s", gemma_hip_last_error());
    return 1;
  }
  PERF_TOC(perf, PERF_OP_GEMM_INT8, tic);
  return 0;
}

/* gemv_fpx (gemma.c:2734): every call site passes a weight matrix */
static void GH_gemv_fpx(float *dst, const float *mat, const float *vec, int rows,
                        int cols, bool omp, int threads, void *perf_any) {
  (void)omp;
  (void)threads;
  PerfBench *perf = perf_any;
  double tic = PERF_TIC(perf);
  hip_or_die(gemma_hip_gemv_fpx_host(dst, mat, vec, rows, cols), "gemv_fpx");
  PERF_TOC(perf, PERF_OP_GEMV_FPX, tic);
}

/* gemv_fpx_multi (gemma.c:2840) */
static void GH_gemv_fpx_multi(const void *jobs_any, int njobs, const float *vec,
                              int cols, int threads, void *perf_any) {
  (void)threads;
  const GemvJob *jobs = jobs_any;
  PerfBench *perf = perf_any;
  double tic = PERF_TIC(perf);
  gemma_hip_job hjobs[GEMMA_HIP_MAX_JOBS];
  if (njobs < 1 || njobs > GEMMA_HIP_MAX_JOBS) {
    die_with("gemv_fpx_multi", "too many jobs");
  }
  for (int idx = 0; idx < njobs; idx++) {
    hjobs[idx].w = jobs[idx].w;
    hjobs[idx].sc = NULL;
    hjobs[idx].dst = jobs[idx].dst;
    hjobs[idx].m = jobs[idx].m;
  }
  hip_or_die(gemma_hip_gemv_fpx_multi_host(hjobs, njobs, vec, cols), "gemv_fpx_multi");
  PERF_TOC(perf, PERF_OP_GEMV_FPX, tic);
}

/* gemm_fpx (gemma.c:3308).  The forward passes also use it for products of
 * two activations (the attention scores of the vision tower and of the
 * prefill, gemma.c:4538, 5222, 5271), which are outside the library's scope:
 * a `mat` that is not a registered weight goes to the reference's own
 * gemm_fpx (which times itself). */
static int GH_gemm_fpx(float *dst, int dstr, const float *mat, int mstr,
                       const float *src, int sstr, int rows, int cols,
                       int depth, bool omp, int threads, void *perf_any) {
  PerfBench *perf = perf_any;
  if (gemma_hip_device_ptr(mat) == NULL) {
    return gemm_fpx(dst, dstr, mat, mstr, src, sstr, rows, cols, depth, omp,
                    threads, perf);
  }
  double tic = PERF_TIC(perf);
  if (gemma_hip_gemm_fpx_host(dst, dstr, mat, mstr, src, sstr, rows, cols,
                              depth) != 0) {
    log_error("gemm_fpx (hip): %s", gemma_hip_last_error());
    return 1;
  }
  PERF_TOC(perf, PERF_OP_GEMM_FPX, tic);
  return 0;
}

/* one device copy per tensor: the int8 rows and the scales are separate
 * ranges, so each lands 256-byte aligned on the device even though the
 * mmapped file places them at arbitrary byte offsets */
static size_t register_qtensor(const QTensor *tensor, size_t rows,
                               size_t cols) {
  if (!tensor->quant) {  /* an fp32 ('U') model file */
    hip_or_die(gemma_hip_register_weights(tensor->fpx, rows * cols * sizeof(float)),
               "register fp32 weights");
    return rows * cols * sizeof(float);
  }
  hip_or_die(gemma_hip_register_weights(tensor->i8.q, rows * cols),
             "register int8 weights");
  hip_or_die(gemma_hip_register_weights(tensor->i8.scales,
                                        rows * sizeof(float)),
             "register weight scales");
  return rows * cols + rows * sizeof(float);
}

static size_t register_decoder(const TextDecoder *dec) {
  const TextConfig *cfg = dec->config;
  size_t dim = cfg->dim, hdim = cfg->hdim, mlp = cfg->mlp_dim;
  size_t q_sz = cfg->n_heads * hdim, kv_sz = cfg->nkv * hdim;
  size_t total = register_qtensor(dec->emb, cfg->nvocab, dim);
  for (int lyr = 0; lyr < cfg->nl; lyr++) {
    const TextDecoderLayer *layer = dec->layers[lyr];
    total += register_qtensor(layer->wq, q_sz, dim);
    total += register_qtensor(layer->wk, kv_sz, dim);
    total += register_qtensor(layer->wv, kv_sz, dim);
    total += register_qtensor(layer->wo, dim, q_sz);
    total += register_qtensor(layer->w1, mlp, dim);
    total += register_qtensor(layer->w2, mlp, dim);
    total += register_qtensor(layer->w3, dim, mlp);
  }
  return total;
}

#endif /* GEMMA_E2E_HIP */

static uint64_t mix_state;

static uint64_t splitmix_next(void) {
  uint64_t val = (mix_state += 0x9E3779B97F4A7C15ull);
  val = (val ^ (val >> 30)) * 0xBF58476D1CE4E5B9ull;
  val = (val ^ (val >> 27)) * 0x94D049BB133111EBull;
  return val ^ (val >> 31);
}

/* FNV-1a over the bytes of the logits, chained across steps */
static uint64_t fnv_chain(uint64_t hash, const float *vals, size_t count) {
  const unsigned char *bytes = (const unsigned char *)vals;
  for (size_t idx = 0; idx < count * sizeof(float); idx++) {
    hash ^= bytes[idx];
    hash *= 0x100000001B3ull;
  }
  return hash;
}

/* The reference's vision tower on one image (see GEMMA_E2E_VISION_IMAGE).
 * The stb blob's `x` macro is no longer needed here: TextBuffer's field x
 * (gemma.c's soft-token output) is reached through it. */
#undef x
static int run_vision(const char *model_path, const char *img_path,
                      const char *out_path, int threads) {
  GemmaModel *model = mmap_gemma_model(model_path, true);
  if (model == NULL || model->encoder == NULL) {
    die_with("load (multimodal)", model == NULL ? get_error() : "no vision tower");
  }
  TextConfig *cfg = model->decoder->config;
  VisionConfig *vcfg = model->encoder->config;
  int img_tok = (int)cfg->img_tok;
  TextBuffer *buf = malloc_text_buffer(cfg, vcfg, img_tok + 1, img_tok, true,
                                       model->quant);
  VisionBuffer *vbuf = malloc_vision_buffer(vcfg, model->quant);
  if (buf == NULL || vbuf == NULL) {
    die_with("buffers", get_error());
  }
  size_t npix = (size_t)vcfg->img_px * vcfg->img_px * 3;
  float *img = malloc(npix * sizeof(float));
  FILE *fin = fopen(img_path, "rb");
  if (img == NULL || fin == NULL || fread(img, sizeof(float), npix, fin) != npix) {
    die_with("image", img_path);
  }
  fclose(fin);
  PerfBench perf;
  memset(&perf, 0, sizeof(perf));
  double tic = now_sec();
  if (forward_vision(model->encoder, cfg, buf, vbuf, img, model->quant, threads,
                     &perf) != 0) {
    die_with("forward_vision", get_error());
  }
  double vision_sec = now_sec() - tic;
  FILE *fout = fopen(out_path, "wb");
  if (fout == NULL ||
      fwrite(buf->x, sizeof(float), (size_t)img_tok * cfg->dim, fout) !=
          (size_t)img_tok * cfg->dim) {
    die_with("output", out_path);
  }
  fclose(fout);
  printf("{\"build\": \"cpu\", \"model\": \"%s\", \"vision_s\": %.6f, "
         "\"img_tok\": %d, \"dim\": %d, \"threads\": %d}\n",
         model_path, vision_sec, img_tok, (int)cfg->dim, threads);
  free(img);
  free_vision_buffer(vbuf, model->quant);
  free_text_buffer(buf, model->quant);
  munmap_gemma_model(model);
  return 0;
}

/* sample() with an image prompt (see GEMMA_E2E_IMAGE); prints one JSON line
 * with the greedy tokens. */
static int run_image(const char *model_path, const char *img_path,
                     const char *logits_path, int prompt_len, int decode_steps,
                     uint64_t seed, int threads) {
  GemmaModel *model = mmap_gemma_model(model_path, true);
  if (model == NULL || model->encoder == NULL) {
    die_with("load (multimodal)", model == NULL ? get_error() : "no vision tower");
  }
  TextConfig *cfg = model->decoder->config;
  VisionConfig *vcfg = model->encoder->config;
  int img_tok = (int)cfg->img_tok;
  int nvocab = (int)cfg->nvocab;
  int chunk = img_tok > prompt_len ? img_tok : prompt_len;
  TextBuffer *buf = malloc_text_buffer(cfg, vcfg, 1 + img_tok + prompt_len + decode_steps,
                                       chunk, true, model->quant);
  VisionBuffer *vbuf = malloc_vision_buffer(vcfg, model->quant);
  if (buf == NULL || vbuf == NULL) {
    die_with("buffers", get_error());
  }
  size_t npix = (size_t)vcfg->img_px * vcfg->img_px * 3;
  float *img = malloc(npix * sizeof(float));
  int *prompt = malloc((size_t)(prompt_len + 1) * sizeof(int));
  FILE *fin = fopen(img_path, "rb");
  if (img == NULL || prompt == NULL || fin == NULL ||
      fread(img, sizeof(float), npix, fin) != npix) {
    die_with("image", img_path);
  }
  fclose(fin);
  FILE *dump = fopen(logits_path, "wb");
  if (dump == NULL) {
    die_with("logits file", logits_path);
  }
  mix_state = seed;
  for (int idx = 0; idx < prompt_len; idx++) {
    prompt[idx] = (int)(splitmix_next() % (uint64_t)nvocab);
  }
  PerfBench perf;
  memset(&perf, 0, sizeof(perf));
  int pos = 0;
  int bos_tok = model->tok->bos;
  if (forward_gemma_prefill(model, buf, &bos_tok, 1, &pos, chunk, NULL, false, threads,
                            &perf) != 0) {
    die_with("prefill <bos>", get_error());
  }
  if (forward_gemma_image(model, buf, vbuf, img, &pos, true, threads, &perf) != 0) {
    die_with("forward_gemma_image", get_error());
  }
  fwrite(buf->logits, sizeof(float), (size_t)nvocab, dump);
  if (prompt_len > 0) {
    if (forward_gemma_prefill(model, buf, prompt, prompt_len, &pos, chunk, NULL, true,
                              threads, &perf) != 0) {
      die_with("prefill", get_error());
    }
    fwrite(buf->logits, sizeof(float), (size_t)nvocab, dump);
  }
  printf("{\"build\": \"cpu\", \"model\": \"%s\", \"img_tok\": %d, \"bos\": %d, "
         "\"prompt\": [", model_path, img_tok, bos_tok);
  for (int idx = 0; idx < prompt_len; idx++) {
    printf("%s%d", idx ? ", " : "", prompt[idx]);
  }
  printf("], \"tokens\": [");
  int token = argmax(buf->logits, nvocab, threads);
  for (int step = 0; step <= decode_steps; step++) {
    printf("%s%d", step ? ", " : "", token);
    if (step == decode_steps) {
      break;
    }
    if (forward_gemma_decode(model, buf, token, pos, threads, &perf) != 0) {
      die_with("decode", get_error());
    }
    pos++;
    fwrite(buf->logits, sizeof(float), (size_t)nvocab, dump);
    token = argmax(buf->logits, nvocab, threads);
  }
  printf("]}\n");
  fclose(dump);
  free(prompt);
  free(img);
  free_vision_buffer(vbuf, model->quant);
  free_text_buffer(buf, model->quant);
  munmap_gemma_model(model);
  return 0;
}

int main(int argc, char **argv) {
  const char *image_prompt = getenv("GEMMA_E2E_IMAGE");
  if (image_prompt != NULL) {
    const char *dump_to = getenv("GEMMA_E2E_LOGITS");
    if (dump_to == NULL || argc < 6) {
      fprintf(stderr, "gemma_e2e: GEMMA_E2E_IMAGE needs GEMMA_E2E_LOGITS and "
                      "<model.bin> <prompt_len> <decode_steps> <seed> <threads>\n");
      return 2;
    }
    return run_image(argv[1], image_prompt, dump_to, atoi(argv[2]), atoi(argv[3]),
                     strtoull(argv[4], NULL, 10), atoi(argv[5]));
  }
  const char *vis_img = getenv("GEMMA_E2E_VISION_IMAGE");
  const char *vis_out = getenv("GEMMA_E2E_VISION_OUT");
  if (vis_img != NULL && vis_out != NULL && argc >= 2) {
    return run_vision(argv[1], vis_img, vis_out, argc > 5 ? atoi(argv[5]) : 1);
  }
  if (argc < 6) {
    fprintf(stderr, "usage: %s <model.bin> <prompt_len> <decode_steps> "
                    "<seed> <threads> [chunk]\n", argv[0]);
    return 2;
  }
  const char *model_path = argv[1];
  int prompt_len = atoi(argv[2]);
  int decode_steps = atoi(argv[3]);
  uint64_t seed = strtoull(argv[4], NULL, 10);
  int threads = atoi(argv[5]);
  int chunk = argc > 6 ? atoi(argv[6]) : DEFAULT_CHUNK_SIZE;
  if (prompt_len < 1 || decode_steps < 0 || threads < 1 || chunk < 1) {
    fprintf(stderr, "gemma_e2e: bad arguments\n");
    return 2;
  }

  GemmaModel *model = mmap_gemma_model(model_path, false);
  if (model == NULL) {
    die_with("load", get_error());
  }
  TextConfig *cfg = model->decoder->config;
  int nvocab = (int)cfg->nvocab;
  int seqlen = 1 + prompt_len + decode_steps;
  TextBuffer *buf = malloc_text_buffer(cfg, NULL, seqlen, chunk, false,
                                       model->quant);
  if (buf == NULL) {
    die_with("text buffer", get_error());
  }

  double setup_sec = 0.0;
  size_t weight_bytes = 0;
  const char *build = "cpu";
#ifdef GEMMA_E2E_HIP
  build = "hip";
  double setup_tic = now_sec();
  hip_or_die(gemma_hip_init(0), "init");
  weight_bytes = register_decoder(model->decoder);
  setup_sec = now_sec() - setup_tic;
  hip_or_die(gemma_hip_perf_enable(1), "perf");
#endif
/* device-side per-op timing follows the reference's phases (PERF_PHASE) */
#ifdef GEMMA_E2E_HIP
#define E2E_PHASE(ph) hip_or_die(gemma_hip_perf_phase(ph), "perf phase")
#else
#define E2E_PHASE(ph) ((void)0)
#endif

  int *prompt = malloc((size_t)prompt_len * sizeof(int));
  int *generated = malloc((size_t)(decode_steps + 1) * sizeof(int));
  if (prompt == NULL || generated == NULL) {
    die_with("alloc", "out of memory");
  }
  mix_state = seed;
  for (int idx = 0; idx < prompt_len; idx++) {
    prompt[idx] = (int)(splitmix_next() % (uint64_t)nvocab);
  }

  PerfBench perf;
  memset(&perf, 0, sizeof(perf));
  int pos = 0;
  int bos_tok = model->tok->bos;
  const char *only = getenv("GEMMA_E2E_DECODE_ONLY");
  const bool decode_only = only != NULL && only[0] == '1';
  const char *dump_path = getenv("GEMMA_E2E_LOGITS");
  FILE *dump = NULL;
  if (dump_path != NULL && (dump = fopen(dump_path, "wb")) == NULL) {
    die_with("logits file", dump_path);
  }
  uint64_t hash = 0xCBF29CE484222325ull;
  double bos_sec = 0.0, prefill_sec = 0.0;

  if (decode_only) {
    /* every position through the decode path, <bos> first */
    E2E_PHASE(PERF_PHASE_DECODE);
    double tic = now_sec();
    for (int idx = 0; idx <= prompt_len; idx++) {
      int tok = idx == 0 ? bos_tok : prompt[idx - 1];
      if (forward_gemma_decode(model, buf, tok, pos, threads, &perf) != 0) {
        die_with("decode (prompt)", get_error());
      }
      pos++;
      if (dump != NULL) {
        fwrite(buf->logits, sizeof(float), (size_t)nvocab, dump);
      }
      if (idx == 0) {
        bos_sec = now_sec() - tic;
        tic = now_sec();
      } else {
        hash = fnv_chain(hash, buf->logits, (size_t)nvocab);
      }
    }
    prefill_sec = now_sec() - tic;
  } else {
    E2E_PHASE(PERF_PHASE_PREFILL);
    double tic = now_sec();
    if (forward_gemma_prefill(model, buf, &bos_tok, 1, &pos, chunk, NULL, false,
                              threads, &perf) != 0) {
      die_with("prefill <bos>", get_error());
    }
    bos_sec = now_sec() - tic;

    tic = now_sec();
    if (forward_gemma_prefill(model, buf, prompt, prompt_len, &pos, chunk, NULL,
                              true, threads, &perf) != 0) {
      die_with("prefill", get_error());
    }
    prefill_sec = now_sec() - tic;
    hash = fnv_chain(hash, buf->logits, (size_t)nvocab);
    if (dump != NULL) {
      fwrite(buf->logits, sizeof(float), (size_t)nvocab, dump);
    }
  }

  int token = argmax(buf->logits, nvocab, threads);
  generated[0] = token;

  E2E_PHASE(PERF_PHASE_DECODE);
  double tic = now_sec();
  for (int step = 0; step < decode_steps; step++) {
    if (forward_gemma_decode(model, buf, token, pos, threads, &perf) != 0) {
      die_with("decode", get_error());
    }
    pos++;
    hash = fnv_chain(hash, buf->logits, (size_t)nvocab);
    if (dump != NULL) {
      fwrite(buf->logits, sizeof(float), (size_t)nvocab, dump);
    }
    token = argmax(buf->logits, nvocab, threads);
    generated[step + 1] = token;
  }
  double decode_sec = now_sec() - tic;
  if (dump != NULL) {
    fclose(dump);
  }

  printf("{\"build\": \"%s\", \"model\": \"%s\", \"nl\": %d, \"dim\": %d, "
         "\"prompt_len\": %d, \"decode_steps\": %d, \"seed\": %" PRIu64
         ", \"threads\": %d, \"chunk\": %d, ",
         build, model_path, (int)cfg->nl, (int)cfg->dim, prompt_len,
         decode_steps, seed, threads, chunk);
  printf("\"setup_s\": %.6f, \"weight_bytes\": %zu, \"bos_s\": %.6f, "
         "\"prefill_s\": %.6f, \"decode_s\": %.6f, \"prefill_tok_s\": %.3f, "
         "\"decode_tok_s\": %.3f, \"decode_only\": %d, ",
         setup_sec, weight_bytes, bos_sec, prefill_sec, decode_sec,
         prompt_len / prefill_sec,
         decode_steps > 0 ? decode_steps / decode_sec : 0.0, (int)decode_only);
  printf("\"ops\": {");
  for (int phase = 0; phase < 2; phase++) {
    printf("%s\"%s\": {", phase ? ", " : "", phase ? "decode" : "prefill");
    int first = 1;
    for (int opi = 0; opi < PERF_OP_COUNT; opi++) {
      if (perf.op[phase][opi].cnt == 0) {
        continue;
      }
      printf("%s\"%s\": [%.6f, %ld]", first ? "" : ", ", opname[opi],
             perf.op[phase][opi].sec, perf.op[phase][opi].cnt);
      first = 0;
    }
    printf("}");
  }
  printf("}, ");
#ifdef GEMMA_E2E_HIP
  /* the library's GPU time of the same ops (HIP events, no PCIe copies) */
  gemma_hip_perf_entry dev_ops[32];
  int ndev = 0;
  hip_or_die(gemma_hip_perf_read(dev_ops, 32, &ndev), "perf read");
  printf("\"device_ops\": {");
  for (int phase = 0; phase < 2; phase++) {
    printf("%s\"%s\": {", phase ? ", " : "", phase ? "decode" : "prefill");
    int first = 1;
    for (int i = 0; i < ndev && i < 32; i++) {
      if (dev_ops[i].phase != phase) {
        continue;
      }
      printf("%s\"%s\": [%.6f, %ld]", first ? "" : ", ", dev_ops[i].op, dev_ops[i].sec,
             dev_ops[i].calls);
      first = 0;
    }
    printf("}");
  }
  printf("}, ");
#endif
  printf("\"bos\": %d, \"logits_fnv\": \"%016" PRIx64 "\", \"prompt\": [",
         bos_tok, hash);
  for (int idx = 0; idx < prompt_len; idx++) {
    printf("%s%d", idx ? ", " : "", prompt[idx]);
  }
  printf("], \"tokens\": [");
  for (int idx = 0; idx <= decode_steps; idx++) {
    printf("%s%d", idx ? ", " : "", generated[idx]);
  }
  printf("]}\n");

#ifdef GEMMA_E2E_HIP
  gemma_hip_shutdown();
#endif
  free(prompt);
  free(generated);
  free_text_buffer(buf, model->quant);
  munmap_gemma_model(model);
  return 0;
}
