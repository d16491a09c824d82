/*
 * gemma_hip.h -- C ABI of the MI355X (gfx950) W8A8 matmul library.
 *
 * The library replaces the matmul hot path of Gemma.c's forward passes:
 * runtime activation quantization, int8 x int8 -> int32 dot products over the
 * full K row (one fp32 scale per output channel and one per activation row),
 * the fp32 rescale, and the fp32 GEMV/GEMM fallback used for unquantized
 * model files.  Every numbered comment names the reference function an entry
 * point replaces, as /root/reference/gemma.c:<line>.
 *
 * Arithmetic contract (bit-exact with the reference built by gcc with
 * -ffast-math, whose start-up code sets FTZ and DAZ):
 *   amax  = max |v| over the row (subnormal v count as 0)
 *   scale = amax * (1/127)   (1 when amax == 0; a result below FLT_MIN is 0)
 *   inv   = 127 / amax       (1 when amax == 0; correctly rounded)
 *   x     = v * inv,  t = x + copysign(0.5, x)
 *   q     = clamp(trunc_x86(t), -127, 127)   (NaN/out of range -> -127)
 *   acc   = sum_k (int32)a[k] * (int32)w[k]  (exact int32)
 *   y     = (float)acc * (act_scale * w_scale)   (two roundings, FTZ)
 * The fp32 fallback has no bit-exact target (the reference's summation order
 * is whatever its compiler vectorises); it matches within a relative error of
 * 1e-5 of sum_k |a_k w_k|.
 *
 * Conventions shared by every entry point:
 *  - Return 0 on success and 1 on failure; the failure's message is kept in a
 *    thread-local buffer read by gemma_hip_last_error() (the reference's
 *    log_error/get_error convention, gemma.c:577-587).  Nothing aborts.
 *  - Matrices are row-major.  A stride of 0 means "dense" (the row length),
 *    as in the reference (gemma.c:3951-3956).
 *  - "n" of gemv_* is the reference's m (output rows) and "k" its n
 *    (reduction length): the names here follow the GEMM contract.
 *  - Entry points without the _host suffix take DEVICE pointers (HBM) and
 *    enqueue their work on `stream` (a hipStream_t; NULL is HIP's default
 *    stream) without synchronising.
 *  - Entry points with the _host suffix take the reference call sites' host
 *    buffers for activations and outputs, resolve weight pointers through the
 *    registry below, and return after the result is back in host memory.
 *  - Device entry points and the decoder are called from one host thread at
 *    a time; the _host entry points serialise among themselves.
 */
#ifndef GEMMA_HIP_H
#define GEMMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GEMMA_HIP_MAX_JOBS 4

/* One projection of a fused multi-output GEMV: replaces GemvJob
 * (gemma.c:2790-2800) field for field.  w is int8 [m][k] (or fp32 [m][k] for
 * the fp32 entry points), sc its fp32 [m] row scales (unused for fp32),
 * dst the fp32 [m] output. */
typedef struct {
  const void *w;
  const float *sc;
  float *dst;
  int m;
} gemma_hip_job;

/* ---- lifecycle --------------------------------------------------------- */

/* Select the GPU and create the library's stream.  Replaces nothing in the
 * reference (its kernels need no set-up); called from setup_gemma_model
 * (gemma.c:6867). */
int gemma_hip_init(int device);

/* Free every registered weight and the staging buffers.  Called from
 * cleanup_gemma_model (gemma.c:6909), next to gemm_free_thread_scratch
 * (gemma.c:4056-4065). */
void gemma_hip_shutdown(void);

/* Message of the last failure on this thread (gemma.c:577-587 get_error). */
const char *gemma_hip_last_error(void);

/* Block until all work enqueued on `stream` (NULL: HIP's default stream)
 * has finished. */
int gemma_hip_sync(void *stream);

/* ---- per-op GPU timing ------------------------------------------------- */
/* The reference's PerfBench (gemma.c:2402-2431, accumulated by PERF_TOC,
 * 2468-2476) on the device: while enabled, the GPU time of every device
 * entry point's launches (HIP events on its stream, so PCIe copies of the
 * _host calls are not included) is summed per phase and op, under the
 * reference's op names and report order: "quantize_act" (gemma_hip_quantize
 * and the _host quantizes), "gemv_int8" (matmul with m == 1, matmul_multi,
 * and quantize_matmul, whose quantize is fused into the GEMV launch),
 * "gemm_int8" (matmul with m > 1, matmul_cols, matmul_heads), "gemv_fpx" and
 * "gemm_fpx" (the fp32 entry points).
 *
 * The device-resident decoder and vision tower time each launch as the
 * reference op it stands for, fused kernels as the op they open with:
 * "rmsnorm" (the residual + norm (+ quantize) rows, the final norm, the
 * tower's pooling RMSNorm), "layernorm" (the tower's residual + layer norm
 * rows), "gemv_int8" (the decode GEMVs, their norm-fused forms and the LM
 * head), "gemm_int8" (the prompt pass's and the tower's GEMMs),
 * "quantize_act", "gelu" (GELU(gate) * up + quantize, bias + GELU +
 * quantize), "rope" (the prompt pass's q/k norm + RoPE + cache append),
 * "softmax" (the attention kernels, which also hold the reference's score
 * and value products and, in the decode step, its RoPE), "gemm_fpx" (the
 * tower's im2col + patch GEMM; with 'U' weights every GEMM, q|k|v and
 * gate|up one launch each), "gemv_fpx" (with 'U' weights the decode GEMVs,
 * their norm-fused forms, GELU fused, and the LM head) and
 * "sample_from_logits" (softcap + argmax,
 * counted in the decode phase as the reference does).  They set the phase
 * themselves as the reference's forward_gemma_* do: decoder_prefill and
 * prefill_rows with mask != 0 prefill; decoder_step and decoder_generate
 * decode (run eagerly, not as the captured graph, while timing is on);
 * vision_forward, gemma_image and prefill_rows with mask == 0 vision.
 * Launches on a stream under graph capture are not timed. */

/* One (phase, op) total: seconds of GPU time over `calls` calls. */
typedef struct {
  const char *op; /* static string: one of the names above */
  int phase;      /* the reference's PerfPhase: 0 prefill, 1 decode, 2 vision */
  double sec;
  long calls;
} gemma_hip_perf_entry;

/* Start (on != 0, clearing the totals) or stop timing. */
int gemma_hip_perf_enable(int on);

/* Attribute the calls that follow to `phase` (PERF_PHASE, gemma.c:2479-2485). */
int gemma_hip_perf_phase(int phase);

/* Waits for the timed launches, then writes up to `max` non-empty totals to
 * out (phase-major, ops in the reference's report order) and their number to
 * *count. */
int gemma_hip_perf_read(gemma_hip_perf_entry *out, int max, int *count);

/* ---- weights: uploaded once, addressed by their host pointers ---------- */

/* Copy [host, host+bytes) to a new device allocation.  Registered ranges are
 * looked up by the _host entry points, which accept any pointer inside a
 * range (the prefill QKV site passes w->i8.q + hd*hdim*dim, gemma.c:5084).
 * Called once per QTensor array after read_qtensor/mmap_qtensor
 * (gemma.c:1134-1171). */
int gemma_hip_register_weights(const void *host, size_t bytes);

/* Free the device copy of the range that starts at `host`. */
int gemma_hip_release_weights(const void *host);

/* Device address of a host pointer inside a registered range, or NULL. */
void *gemma_hip_device_ptr(const void *host);

/* ---- device entry points (the hot path) -------------------------------- */

/* quantize_acts (gemma.c:2652-2674), and quantize_act (gemma.c:2586-2650)
 * for m == 1: quantize m rows of n values, read with row stride sstr, into
 * dst [m][n] int8 and dsc [m] fp32 scales. */
int gemma_hip_quantize(int8_t *dst, float *dsc, const float *src, int sstr,
                       int m, int n, void *stream);

/* gemm_int8 (gemma.c:3937-4054), and gemv_int8 (gemma.c:2765-2788) when
 * m == 1: dst[i][j] = (float)sum_l src[i][l]*mat[j][l] * (ssc[i]*matsc[j]).
 * src int8 [m][sstr], mat int8 [n][mstr], dst fp32 [m][dstr]; cells outside
 * [m][n] are not written. */
int gemma_hip_matmul(float *dst, int dstr, const int8_t *mat, int mstr,
                     const float *matsc, const int8_t *src, int sstr,
                     const float *ssc, int m, int n, int k, void *stream);

/* gemma_hip_matmul without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops): no
 * counterpart in the reference.  Same arguments, result bit-identical to
 * gemma_hip_matmul.  The split-K partial tiles and tile counters that some
 * shapes use live in a static device array of 32 MiB that each GPU the
 * library runs on holds until the process ends; a shape whose launch plan
 * needs more fails with an error naming both sizes.  The counters are
 * cleared by a kernel on every call (no memset, so the call may be captured).
 * All calls on one GPU share that array: calls that overlap in time on one
 * GPU (several streams, or several host threads) race. */
int gemma_hip_matmul_noalloc(float *dst, int dstr, const int8_t *mat, int mstr,
                             const float *matsc, const int8_t *src, int sstr,
                             const float *ssc, int m, int n, int k, void *stream);

/* The prefill QKV site (gemma.c:5045-5089) as one launch: the same product
 * as gemma_hip_matmul with n = heads*hdim and dense operands, written
 * head-major, dst[(h*m + i)*hdim + j] for output column h*hdim + j. */
int gemma_hip_matmul_heads(float *dst, const int8_t *mat, const float *matsc,
                           const int8_t *src, const float *ssc, int m,
                           int heads, int hdim, int k, void *stream);

/* gemm_int8 (gemma.c:3937-4054) of one activation block against several
 * weight matrices that share its K, as adjacent prefill call sites issue
 * them (up and gate at gemma.c:5365-5372; q, k and v per head at 5084-5087):
 * the multi-job form of gemma_hip_matmul, as gemma_hip_matmul_multi is of the
 * GEMV.  Job j (j < njobs <= 3) holds int8 [jobs[j].m][k] dense weights
 * jobs[j].w and their scales jobs[j].sc, and fills dst columns
 * [c_j, c_j + jobs[j].m), c_j the sum of the earlier jobs' m; jobs[j].dst is
 * not used.  src int8 [m][sstr], dst fp32 [m][dstr] (0 strides: dense).
 * Bit-identical to one gemma_hip_matmul per job. */
int gemma_hip_matmul_cols(float *dst, int dstr, const gemma_hip_job *jobs, int njobs,
                          const int8_t *src, int sstr, const float *ssc, int m, int k,
                          void *stream);

/* gemv_int8_multi (gemma.c:2813-2837): njobs (<= GEMMA_HIP_MAX_JOBS)
 * projections of the one quantized vector x [k] with scale xs (a device
 * pointer to one float). */
int gemma_hip_matmul_multi(const gemma_hip_job *jobs, int njobs,
                           const int8_t *x, const float *xs, int k,
                           void *stream);

/* The decode call sites' quantize_act followed by gemv_int8_multi / gemv_int8
 * (gemma.c:4768-4773, 4858-4859, 4911-4915, 4929-4930, 4964-4965) in one
 * launch: x fp32 [k] is quantized inside the kernel.  xq [k] and xs [1]
 * (both nullable) receive the quantized vector and its scale. */
int gemma_hip_quantize_matmul(const gemma_hip_job *jobs, int njobs,
                              const float *x, int k, int8_t *xq, float *xs,
                              void *stream);

/* gemm_fpx (gemma.c:3304-3399) and gemv_fpx (gemma.c:2730-2752) when
 * m == 1: dst[i][j] = sum_l src[i][l]*mat[j][l] in fp32. */
int gemma_hip_matmul_f32(float *dst, int dstr, const float *mat, int mstr,
                         const float *src, int sstr, int m, int n, int k,
                         void *stream);

/* gemm_fpx (gemma.c:3304-3399) of one fp32 activation block against several
 * fp32 weight matrices that share its K, as the unquantized prompt pass's
 * adjacent call sites issue them (q, k and v at gemma.c:5079; gate and up at
 * 5358): the fp32 form of gemma_hip_matmul_cols.  Job j (j < njobs <= 3)
 * holds fp32 [jobs[j].m][k] dense weights jobs[j].w and fills dst columns
 * [c_j, c_j + jobs[j].m), c_j the sum of the earlier jobs' m; jobs[j].sc and
 * jobs[j].dst are not used.  src fp32 [m][sstr], dst fp32 [m][dstr] (0
 * strides: dense).  Same tolerance as gemma_hip_matmul_f32. */
int gemma_hip_matmul_f32_cols(float *dst, int dstr, const gemma_hip_job *jobs, int njobs,
                              const float *src, int sstr, int m, int k, void *stream);

/* gemv_fpx_multi (gemma.c:2839-2858). */
int gemma_hip_matmul_f32_multi(const gemma_hip_job *jobs, int njobs,
                               const float *x, int k, void *stream);

/* The SigLIP patch embedding (gemma.c:4411-4448): the stride-psize,
 * psize x psize convolution of an HWC fp32 image img [img_px][img_px][3]
 * with pe [dim][3][psize][psize] plus pe_b [dim], as im2col + fp32 GEMM.
 * dst [npatch][dim], npatch = (img_px/psize)^2, each value clamped to
 * [-FLT_MAX, FLT_MAX] (clamp_fpx, gemma.c:2504).  work is a device
 * workspace of npatch*3*psize*psize floats, or NULL to use one the library
 * allocates on first need.  fp32: matches within the fp32 tolerance. */
int gemma_hip_patch_embed(float *dst, const float *img, const float *pe,
                          const float *pe_b, int img_px, int psize, int dim,
                          float *work, void *stream);

/* ---- host drop-ins for the reference call sites ------------------------ */
/* Same argument order and meaning as the reference functions named; weight
 * pointers (mat, matsc, job w/sc) must lie in registered ranges, activation
 * and output pointers are ordinary host memory.  They may be called from
 * several threads at once (the prefill QKV site calls gemm_int8 inside an
 * OpenMP loop, gemma.c:5050-5089); such calls run one after another. */

/* quantize_act (gemma.c:2590); the scale goes to *scale. */
int gemma_hip_quantize_act_host(int8_t *dst, float *scale, const float *vec,
                                int dim);

/* quantize_acts (gemma.c:2656). */
int gemma_hip_quantize_acts_host(int8_t *dst, float *dsc, const float *src,
                                 int sstr, int m, int n);

/* gemv_int8 (gemma.c:2770): m output rows, reduction length n. */
int gemma_hip_gemv_int8_host(float *dst, const int8_t *mat, const float *matsc,
                             const int8_t *vec, float vsc, int m, int n);

/* gemv_int8_multi (gemma.c:2818); job dst pointers are host memory. */
int gemma_hip_gemv_int8_multi_host(const gemma_hip_job *jobs, int njobs,
                                   const int8_t *vec, float vsc, int n);

/* gemm_int8 (gemma.c:3943). */
int gemma_hip_gemm_int8_host(float *dst, int dstr, const int8_t *mat, int mstr,
                             const float *matsc, const int8_t *src, int sstr,
                             const float *ssc, int m, int n, int k);

/* gemv_fpx (gemma.c:2734). */
int gemma_hip_gemv_fpx_host(float *dst, const float *mat, const float *vec,
                            int m, int n);

/* gemv_fpx_multi (gemma.c:2840). */
int gemma_hip_gemv_fpx_multi_host(const gemma_hip_job *jobs, int njobs,
                                  const float *vec, int n);

/* gemm_fpx (gemma.c:3308). */
int gemma_hip_gemm_fpx_host(float *dst, int dstr, const float *mat, int mstr,
                            const float *src, int sstr, int m, int n, int k);

/* forward_vision's patch embedding (gemma.c:4411-4448) on a host image;
 * pe and pe_b must be registered. */
int gemma_hip_patch_embed_host(float *dst, const float *img, const float *pe,
                               const float *pe_b, int img_px, int psize, int dim);

/* ---- device-resident decoder ------------------------------------------- */
/* One greedy decode step with every tensor resident in HBM: the embedding
 * lookup, all layers (norms, q/k/v, q/k norm, RoPE, KV cache, attention,
 * o, gate/up, GELU, down, residuals), the final norm, the LM head and the
 * argmax run on the GPU, captured once into a HIP graph.  Replaces
 * forward_gemma_decode (gemma.c:5456) + forward_text_decode (4727) for W8A8
 * model files, and argmax (5600) for greedy sampling.  The int8 products are
 * bit-exact as above; the fp32 glue (norms, RoPE, softmax, GELU) follows
 * the reference's formulas in its own summation order, so logits agree with
 * the reference to fp32 rounding amplified by int8 requantization, not bit
 * for bit. */

/* The reference's TextConfig (gemma.c:740-761) as plain fields. */
typedef struct {
  int nl, n_heads, nkv, hdim, dim, mlp_dim, q_scale, slide, nvocab;
  float theta_l, theta_g, eps, sc_att, sc_log;
  int qk_norm, mlp_pre, mlp_pst; /* flags, 0 or 1 */
  const unsigned char *swa;      /* nl flags: 1 = sliding-window layer */
} gemma_hip_text_config;

/* One TextDecoderLayer (gemma.c:1173-1195) of a W8A8 file: int8 weights and
 * their row scales are host pointers inside registered ranges; the norm
 * weights (stored as w, applied as w + 1) are host arrays the decoder copies
 * (nq/nk only read when qk_norm, n3 when mlp_pre, n4 when mlp_pst). */
typedef struct {
  const int8_t *wq, *wk, *wv, *wo, *w1, *w2, *w3;
  const float *wq_s, *wk_s, *wv_s, *wo_s, *w1_s, *w2_s, *w3_s;
  const float *nq, *nk, *n1, *n2, *n3, *n4;
} gemma_hip_layer;

typedef struct gemma_hip_decoder gemma_hip_decoder;

/* Builds a decoder for a context of clen positions: resolves the registered
 * weights (emb int8 [nvocab][dim] + emb_s [nvocab] is also the tied LM head),
 * copies the norms, allocates the KV cache [nl][2][nkv][clen][hdim] and the
 * activations, and captures the step graph.  NULL on failure. */
gemma_hip_decoder *gemma_hip_decoder_create(const gemma_hip_text_config *cfg,
                                            const gemma_hip_layer *layers,
                                            const int8_t *emb, const float *emb_s,
                                            const float *fnorm, int clen);
void gemma_hip_decoder_destroy(gemma_hip_decoder *dec);

/* One TextDecoderLayer of an unquantized ('U') file: fp32 weights [out][in]
 * (QTensor.fpx, gemma.c:1125-1131) as host pointers inside registered
 * ranges; the norms as for gemma_hip_layer. */
typedef struct {
  const float *wq, *wk, *wv, *wo, *w1, *w2, *w3;
  const float *nq, *nk, *n1, *n2, *n3, *n4;
} gemma_hip_layer_f32;

/* gemma_hip_decoder_create for a 'U' file: the reference's !quant branches
 * (decode gemma.c:4762, 4855, 4906, 4925, 4960; prefill 5079, 5297, 5358,
 * 5384, 5431) on the device: emb is the fp32 [nvocab][dim] table (also the
 * tied LM head), the projections run as fp32 GEMVs (gemv_fpx) in the step
 * (the norms fused into the q/k/v and gate/up GEMVs, GELU into gate/up, as
 * in the W8A8 step) and as fp32 GEMMs (gemm_fpx: on the bf16 matrix cores in
 * split precision, fp32 accuracy) in the prompt pass, with no activation
 * quantize.  Every other decoder entry point takes the result as it takes a
 * W8A8 decoder. */
gemma_hip_decoder *gemma_hip_decoder_create_f32(const gemma_hip_text_config *cfg,
                                                const gemma_hip_layer_f32 *layers,
                                                const float *emb, const float *fnorm,
                                                int clen);

/* One step at position pos (0 <= pos < clen, token < nvocab): logits (host,
 * nvocab floats) and next (the argmax) are written when non-NULL. */
int gemma_hip_decoder_step(gemma_hip_decoder *dec, int token, int pos,
                           float *logits, int *next);

/* The prompt pass: n tokens (host array) at positions pos .. pos+n-1 go
 * through every layer as one batch, as forward_gemma_prefill (gemma.c:5501)
 * with forward_text_chunk (4985-5453) does -- the int8 projections as GEMMs,
 * causal (sliding-window) attention over the KV cache -- filling the KV
 * cache, so step/generate continue at pos + n.  logits and next (nullable)
 * receive the last token's logits and argmax.  n >= 1, pos + n <= clen; head
 * dim 128 or 256, q heads per kv head dividing 32, mlp_dim <= 24576.  Its
 * row buffers are allocated on the first call (regrown for a larger n). */
int gemma_hip_decoder_prefill(gemma_hip_decoder *dec, const int *tokens, int n, int pos,
                              float *logits, int *next);

/* The prompt pass over n rows given as embeddings (n x dim fp32, a host or
 * a device pointer) instead of token ids: forward_text_chunk (gemma.c:4985)
 * on what its callers place in tb->x.  mask != 0 is the causal
 * (sliding-window) attention of text tokens; mask == 0 the dense path
 * (gemma.c:5258-5290) forward_gemma_image (5561-5595) takes for image soft
 * tokens: every row attends to every cached key up to pos + n - 1, with no
 * window.  Rows are used as given (no embedding scale).  Otherwise as
 * gemma_hip_decoder_prefill; the step record's token is 0 (next, when
 * given, is the argmax of the last row). */
int gemma_hip_decoder_prefill_rows(gemma_hip_decoder *dec, const float *x, int n, int pos,
                                   int mask, float *logits, int *next);

/* The arithmetic of the prompt passes' attention (prefill, prefill_rows,
 * image), kept until changed: GEMMA_HIP_ATTN_F32 (the default; fp32
 * throughout as the reference's gemm_fpx/softmax/gemm_fpx_nn,
 * gemma.c:5198-5255, in its own summation order: agrees with the exact
 * result to fp32 rounding, amplified where a later int8 quantization flips)
 * or GEMMA_HIP_ATTN_F64 (fp64 matrix cores, each output rounded once from
 * the exact sum: the verification mode, equal to an fp64 evaluation of the
 * same formulas).  The fp32 mode runs on the bf16 matrix cores in split
 * precision (each fp32 operand three bf16 pieces, each product summed from
 * the six piece products down to 2^-16 of the leading one, fp32
 * accumulation), or, for passes too small to give that kernel 32 workgroups,
 * on the fp32 matrix cores; the environment variable GEMMA_HIP_PF_ATTN=bf3
 * or =f32, read at every launch, forces either.  The decode step's attention
 * is fp64 either way.  0 or 1 on an unknown mode. */
#define GEMMA_HIP_ATTN_F64 0
#define GEMMA_HIP_ATTN_F32 1
int gemma_hip_decoder_set_attention(gemma_hip_decoder *dec, int mode);

/* n greedy steps without host round trips: step i consumes the token step
 * i-1 produced (the first consumes `token` at `pos`); tokens[i] receives the
 * argmax of step i (host, n ints).  pos + n <= clen. */
int gemma_hip_decoder_generate(gemma_hip_decoder *dec, int token, int pos, int n,
                               int *tokens);

/* Device pointer of the last step's logits (nvocab floats). */
const float *gemma_hip_decoder_logits(const gemma_hip_decoder *dec);

/* ---- device-resident vision tower --------------------------------------- */
/* forward_vision (gemma.c:4394-4725) with every tensor resident in HBM: the
 * patch embedding, the position embedding, all SigLIP encoder layers (layer
 * norms, q/k/v/o with biases, attention over all patches, fc1 + GELU, fc2,
 * residuals), the post layer norm, average pooling to the image tokens, the
 * soft-embedding RMSNorm and the projection to the text width.  W8A8 files:
 * the int8 products are bit-exact as above; the fp32 glue follows the
 * reference's formulas, evaluated in fp64 and rounded once. */

/* The reference's VisionConfig (gemma.c:713-721), plus the two TextConfig
 * fields the tower feeds: img_tok (a square number of pooled tokens) and the
 * text model's dim (the projection's width). */
typedef struct {
  int nl, n_heads, img_px, psize, dim, mlp_dim;
  float eps;
  int img_tok, text_dim;
} gemma_hip_vision_config;

/* One VisionEncoderLayer (gemma.c:1234-1256) of a W8A8 file: int8 weights and
 * their row scales are host pointers inside registered ranges (wq..wo
 * [dim][dim], w1 [mlp_dim][dim], w2 [dim][mlp_dim]); biases and layer-norm
 * weights are host arrays the tower copies. */
typedef struct {
  const int8_t *wq, *wk, *wv, *wo, *w1, *w2;
  const float *wq_s, *wk_s, *wv_s, *wo_s, *w1_s, *w2_s;
  const float *bq, *bk, *bv, *bo, *b1, *b2;
  const float *n1, *n1_b, *n2, *n2_b;
} gemma_hip_vision_layer;

typedef struct gemma_hip_vision gemma_hip_vision;

/* Builds the tower of a VisionEncoder (gemma.c:1565-1585): pe [dim][3][psize]
 * [psize] and pe_b [dim] (fp32), post_n/post_nb/norm [dim] are copied;
 * pos_q [npatch][dim] + pos_s [npatch] and proj [text_dim][dim] + proj_s
 * [text_dim] must be registered.  Head dim (dim / n_heads) 16, 32, 64, 72 or
 * 128; dim and mlp_dim multiples of 16 (dim <= 6144, mlp_dim <= 24576).
 * NULL on failure. */
gemma_hip_vision *gemma_hip_vision_create(const gemma_hip_vision_config *cfg,
                                          const gemma_hip_vision_layer *layers,
                                          const float *pe, const float *pe_b,
                                          const int8_t *pos_q, const float *pos_s,
                                          const float *post_n, const float *post_nb,
                                          const float *norm, const int8_t *proj,
                                          const float *proj_s);
void gemma_hip_vision_destroy(gemma_hip_vision *vis);

/* One VisionEncoderLayer of an unquantized ('U') file: fp32 projections
 * [out][in] (registered), biases and norms as for gemma_hip_vision_layer. */
typedef struct {
  const float *wq, *wk, *wv, *wo, *w1, *w2;
  const float *bq, *bk, *bv, *bo, *b1, *b2;
  const float *n1, *n1_b, *n2, *n2_b;
} gemma_hip_vision_layer_f32;

/* gemma_hip_vision_create for a 'U' file: forward_vision's !quant branches
 * (gemma.c:4454, 4488, 4562, 4604, 4626, 4709) on the device: pos
 * [npatch][dim] and proj [text_dim][dim] fp32 (registered), every
 * projection an fp32 matrix-core GEMM (gemm_fpx; fp64 in the verification
 * mode of gemma_hip_vision_set_attention), no activation quantize.  Every
 * other vision entry point takes the result as it takes a W8A8 tower. */
gemma_hip_vision *gemma_hip_vision_create_f32(const gemma_hip_vision_config *cfg,
                                              const gemma_hip_vision_layer_f32 *layers,
                                              const float *pe, const float *pe_b,
                                              const float *pos, const float *post_n,
                                              const float *post_nb, const float *norm,
                                              const float *proj);

/* One image: img (host, [img_px][img_px][3] fp32, normalized as gemma.c:
 * 4271-4273 leaves it) in, out (host, [img_tok][text_dim] fp32: the image's
 * soft tokens, what forward_vision leaves in tb->x) out. */
int gemma_hip_vision_forward(gemma_hip_vision *vis, const float *img, float *out);

/* The arithmetic of the tower's two fp32 products, its attention
 * (gemma.c:4533-4561) and its patch embedding (4411-4448, im2col and a GEMM
 * with the bias, clamp and position embedding of 4452-4468 in its epilogue);
 * set before forward, kept until changed:
 *   GEMMA_HIP_ATTN_F32 (the default) -- fp32 throughout as the reference
 *     computes it (its summation order differs), so results agree with the
 *     exact form to fp32 rounding, amplified where a later int8 quantization
 *     flips.  The patch GEMM runs on the fp32 matrix cores; the attention on
 *     the bf16 ones in split precision: each fp32 operand is the sum of three
 *     bf16 pieces and every product is summed from the six piece products
 *     down to 2^-16 of the leading one, which leaves an error per product of
 *     order 2^-23 relative, the size of an fp32 rounding, with fp32
 *     accumulation (the environment variable GEMMA_HIP_VIS_ATTN=f32, read
 *     once, selects the plain fp32 matrix-core kernel instead);
 *   GEMMA_HIP_ATTN_F64 -- fp64 (matrix cores for the attention), every
 *     output rounded once from the exact sum: the verification mode, equal
 *     to an fp64 evaluation of the same formulas.
 * The rest of the tower is unchanged.  0 or 1 on an unknown mode. */
int gemma_hip_vision_set_attention(gemma_hip_vision *vis, int mode);

/* The tower's attention block alone (gemma.c:4527-4561) on device buffers:
 * qkv [n][3*dim] holds the q, k and v GEMM outputs of each patch, bias
 * [3*dim] their biases (added in fp32, 4517-4526); out [n][dim] receives, per
 * head of dim/n_heads (16, 32, 64, 72 or 128), softmax(q.k * scale) v over all
 * n patches with scale = 1/sqrtf(head dim).  mode as above.  On `stream`
 * (NULL: the library's). */
int gemma_hip_vision_attention(float *out, const float *qkv, const float *bias, int n,
                               int n_heads, int dim, int mode, void *stream);

/* The prompt pass's attention block alone (forward_text_chunk's blockwise
 * attention, gemma.c:5152-5293, and its dense form 5258-5290), as
 * gemma_hip_vision_attention is for the tower, so that its kernels can be
 * checked before any int8 requantization: no counterpart function in the
 * reference.  q [n][q_stride] holds the n rows' q heads after RoPE (head h
 * at column h*hdim, n_heads*hdim <= q_stride); kc / vc [nkv][clen][hdim]
 * hold the keys and values of positions 0 .. pos0+n-1 (the rows' own at
 * pos0 .. pos0+n-1); out [n][n_heads*hdim].  Row i sits at position pos0+i:
 * dense == 0 attends causally to keys max(0, pos0+i+1-slide) .. pos0+i
 * (slide 0: no window), dense == 1 to every key 0 .. pos0+n-1.  Scores are
 * q.k * asc, capped as tanh(s / sc_att) * sc_att when sc_att != 0; mode is
 * GEMMA_HIP_ATTN_F32 or GEMMA_HIP_ATTN_F64 as for the decoder.  hdim 128 or
 * 256; n_heads / nkv must divide 32; n_heads * hdim <= 6144.  Allocates its
 * key-split workspace. */
int gemma_hip_prefill_attention(float *out, const float *q, int q_stride, const float *kc,
                                const float *vc, int n, int pos0, int n_heads, int nkv,
                                int hdim, int clen, int slide, float asc, float sc_att,
                                int dense, int mode, void *stream);

/* forward_gemma_image (gemma.c:5561-5595) on the device: the vision tower on
 * img, its img_tok soft tokens handed to the decoder in HBM, and the dense
 * (mask=false) prompt pass at *pos, which advances by img_tok on success.
 * logits / next (nullable) as gemma_hip_decoder_prefill.  The tower's
 * text_dim must be the decoder's dim. */
int gemma_hip_gemma_image(gemma_hip_decoder *dec, gemma_hip_vision *vis, const float *img,
                          int *pos, float *logits, int *next);

#ifdef __cplusplus
}
#endif

#endif
