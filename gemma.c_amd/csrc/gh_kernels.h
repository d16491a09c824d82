// gh_kernels.h -- launchers of the library's HIP kernels (internal to the
// library; the public interface is include/gemma_hip.h).
//
// Every launcher checks nothing about its arguments beyond what selects a
// kernel variant: gemma_hip.cpp validates shapes, strides and pointers before
// calling, so each launch covers exactly the rows, columns and bytes the
// kernel's grid assumes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gh {

constexpr int kMaxJobs = 4;  // Pick4 (gh_arith.h) selects among exactly four

// A fused multi-output GEMV: jobs[j] owns output rows [end[j-1], end[j]).
struct GemvJobs {
  const void *w[kMaxJobs];
  const float *sc[kMaxJobs];
  float *dst[kMaxJobs];
  int end[kMaxJobs];
  int njobs;
};

struct DeviceInfo {
  int cus;  // compute units
};

// quantize.hip: rows of src [m][sstr] -> dst [m][n] int8 + dsc [m], and the
// same into the mirror mdst/mdsc when given (pinned host memory)
hipError_t launch_quantize(int8_t *dst, float *dsc, const float *src, int sstr,
                           int m, int n, hipStream_t stream,
                           int8_t *mdst = nullptr, float *mdsc = nullptr);

// gemv.hip: int8 GEMV over jobs.  Either xq/xs (already quantized) or xf
// (fp32, quantized inside the kernel; xq_out/xs_out nullable) is given.
hipError_t launch_gemv_i8(const GemvJobs &jobs, int k, const int8_t *xq,
                          const float *xs, const float *xf, int8_t *xq_out,
                          float *xs_out, const DeviceInfo &dev,
                          hipStream_t stream);

// gemv.hip: fp32 GEMV over jobs (sc unused).
// Lanes per row and 16-byte chunks per lane and pass of the fp32 stream
// GEMVs (gemv_f32_stream_kernel, dec_norm_f32_kernel) for `rows` rows of kc
// chunks; gelu pairs gate and up rows in one wave, so at most 32 lanes.  Up
// to 65536 rows, a row that fits in one pass of at most 12 chunks per lane
// takes one (the fewest lanes, then the fewest chunks that cover it):
// measured at gemma-3-1b (rows of 1152 floats, same box, alternating runs),
// q/k/v 5.4 -> 5.1 us, gate/up 15.5 -> 13.7 us, the 'U' decode step 701 ->
// 716 tok/s.  Otherwise 8 chunks and the fewest lanes that cover a row in at
// most two passes: on the 262144-row LM head one pass of 10 ran 2-4%
// slower, and on the 6912-float down rows three passes of 10 ran 4% slower
// than four of 8.
struct F32StreamShape {
  int lanes, cpl, passes;
};
inline F32StreamShape f32_stream_shape(int kc, bool gelu, long rows) {
  const int lmax = gelu ? 32 : 64;
  if (rows <= 65536)
    for (int l = 8; l <= lmax; l *= 2)
      for (int c : {8, 10, 12})
        if (kc <= l * c) return {l, c, 1};
  int lanes = lmax;
  for (int l = 8; l <= lmax; l *= 2)
    if ((kc + l * 8 - 1) / (l * 8) <= 2) {
      lanes = l;
      break;
    }
  return {lanes, 8, (kc + lanes * 8 - 1) / (lanes * 8)};
}

hipError_t launch_gemv_f32(const GemvJobs &jobs, int k, const float *x,
                           const DeviceInfo &dev, hipStream_t stream);

// Workspace of split-K GEMM launches (int32 partial tiles + tile counters).
struct GemmWs {
  int *base;
  size_t bytes;
};
// Size of the caller-free workspace (gemm_i8.hip's static `scratch`).
constexpr size_t kGemmScratchBytes = (size_t)32 << 20;
// Resolves the device address of `scratch` on `device`, which must be the
// current device (once per device; later calls return at once).
hipError_t gemm_scratch_init(int device);
// The caller-free workspace of `device` ({nullptr, 0} before init).
GemmWs gemm_scratch(int device);

// gemm_i8.hip: dst = rescale(src . mat^T).  hdim > 0 selects the head-major
// output layout dst[((j/hdim)*m + i)*hdim + j%hdim] (dstr ignored).  With
// `fixed` the launch takes its workspace from there (and returns
// hipErrorOutOfMemory if it needs more), else from a per-stream one the
// library allocates on first need.
hipError_t launch_gemm_i8(float *dst, int dstr, int hdim, const int8_t *mat,
                          int mstr, const float *matsc, const int8_t *src,
                          int sstr, const float *ssc, int m, int n, int k,
                          const DeviceInfo &dev, hipStream_t stream,
                          const GemmWs *fixed = nullptr);
// Workspace bytes launch_gemm_i8 needs for this shape (0: none).
size_t gemm_i8_scratch_bytes(int m, int n, int k, bool heads, const int8_t *mat, int mstr,
                             const int8_t *src, int sstr, int dstr, const DeviceInfo &dev);

// B as up to kMaxGemmSegs separate [rows][k] matrices (q, k, v; or gate,
// up) whose outputs are adjacent column ranges of one dst: segment t holds
// output columns [end[t-1], end[t]) (end[-1] = 0), scales s[t] per row.
constexpr int kMaxGemmSegs = 3;
struct GemmSegs {
  const int8_t *w[kMaxGemmSegs];
  const float *s[kMaxGemmSegs];
  int end[kMaxGemmSegs];
  int nseg;
};
// One launch over all segments when every inner segment boundary is a
// multiple of the tile width; otherwise one launch per segment.
// Frees the split-K workspaces of every (device, stream) (library shutdown).
void release_gemm_workspaces();

hipError_t launch_gemm_i8_segs(float *dst, int dstr, const GemmSegs &b, const int8_t *src,
                               int sstr, const float *ssc, int m, int k, const DeviceInfo &dev,
                               hipStream_t stream);

// gemm_f32.hip: dst = src . mat^T in fp32; bias (nullable) adds bias[col],
// clamp limits every output to [-FLT_MAX, FLT_MAX] (clamp_fpx).
hipError_t launch_gemm_f32(float *dst, int dstr, const float *mat, int mstr,
                           const float *src, int sstr, int m, int n, int k,
                           const float *bias, bool clamp,
                           const DeviceInfo &dev, hipStream_t stream);

// What the fp32 GEMM does with a finished sum s of output (row, col):
//   y = s (+ bias[col]), clamped to [-FLT_MAX, FLT_MAX] when clamp is set;
//   with pos_q: y = clamp(y + (float)pos_q[row][col] * pos_s[row]) -- the
//   dequantized position embedding of the SigLIP patch embedding
//   (gemma.c:4411-4468), whose rows are dstr wide.
struct F32Epilogue {
  const float *bias;
  bool clamp;
  const int8_t *pos_q;
  const float *pos_s;
  const float *pos_f;  // an fp32 position embedding [rows][dstr] ('U' files)
  __device__ __forceinline__ float finish(float y, int row, int col, int dstr) const {
    if (clamp) y = fminf(3.40282347e38f, fmaxf(-3.40282347e38f, y));
    if (pos_q != nullptr || pos_f != nullptr) {
      const float pos = pos_f != nullptr ? pos_f[(size_t)row * dstr + col]
                                         : (float)pos_q[(size_t)row * dstr + col] * pos_s[row];
      y = fminf(3.40282347e38f, fmaxf(-3.40282347e38f, y + pos));
    }
    return y;
  }
  // an fp32 sum: the bias is one fp32 addition
  __device__ __forceinline__ float apply(float s, int row, int col, int dstr) const {
    return finish(bias != nullptr ? s + bias[col] : s, row, col, dstr);
  }
  // an fp64 sum: the sum and the bias rounded once
  __device__ __forceinline__ float apply_f64(double s, int row, int col, int dstr) const {
    return finish((float)(bias != nullptr ? s + (double)bias[col] : s), row, col, dstr);
  }
};
// ... with a full epilogue; f64 selects the fp64 twin (every output rounded
// once from its fp64 sum), the verification mode of the vision tower.
hipError_t launch_gemm_f32(float *dst, int dstr, const float *mat, int mstr,
                           const float *src, int sstr, int m, int n, int k,
                           const F32Epilogue &ep, const DeviceInfo &dev, hipStream_t stream,
                           bool f64);

// B as up to kMaxGemmSegs separate fp32 [rows][mstr] matrices whose outputs
// are adjacent column ranges of one dst (q, k, v; or gate, up): segment t
// holds output columns [end[t-1], end[t]) (end[-1] = 0).  The split-bf16
// kernel runs all segments in one launch (split-K when its tiles leave CUs
// idle); the fp32-MFMA and fp64 kernels run one launch per segment.
struct F32Segs {
  const float *w[kMaxGemmSegs];
  int end[kMaxGemmSegs];
  int nseg;
};
hipError_t launch_gemm_f32_segs(float *dst, int dstr, const F32Segs &b, int mstr,
                                const float *src, int sstr, int m, int k,
                                const F32Epilogue &ep, const DeviceInfo &dev, hipStream_t stream,
                                bool f64);

// gemm_i8.hip: the split-K workspace of (device, stream) with at least
// ws_ints ints of partials and ncnt tile counters (zero between launches;
// each launch must leave them at zero), grown on demand (the stream is
// synchronized first, so not while it is being captured).
hipError_t split_workspace(hipStream_t stream, size_t ws_ints, int ncnt, int **ws, int **cnt);

// patch.hip: a [npatch][3*psize*psize] = patches of the HWC image, in the K
// order of the SigLIP patch-embedding weight [dim][3][psize][psize].
hipError_t launch_im2col(float *a, const float *img, int img_px, int psize,
                         hipStream_t stream);

// decode.hip: the device-resident decode step.
// Residual update and rmsnorm in front of an int8 GEMV:
//   x_new = clamp(x_res + (w_post ? rmsnorm(y, w_post) : y))   (x_res when y is null)
//   h     = rmsnorm(x_new, w_pre)
// workgroup 0 stores x_new to x_out and h to h_out (each nullable).
struct DecNorm {
  const float *x_res;
  const float *y;
  const float *w_post;
  const float *w_pre;
  float *x_out;
  float *h_out;
  int dim;
  float eps;
};

// x = emb_q[token] * (esc * emb_s[token]), or emb_f[token] * esc for an
// fp32 table (emb_f non-null); step = {token, pos, count}
struct DecEmbed {
  const int8_t *emb_q;
  const float *emb_s;
  float *x;
  const int *step;
  int dim, nvocab, clen;
  float esc;
  const float *emb_f;
};

// Keys per attention workgroup, and its LDS bytes for hn q heads per kv head.
constexpr int kDecAttnBlock = 16;
inline size_t dec_attn_lds(int hn, int hdim) {
  return (size_t)hn * kDecAttnBlock * 8 +
         ((size_t)hn * hdim + 2 * (size_t)hdim + (size_t)kDecAttnBlock * (2 * hdim + 16)) * 4;
}

// Byte regions (16-byte aligned) that a kernel reads and discards after its
// own work, so that a later kernel finds them in the memory-side cache
// (the Infinity Cache) rather than in HBM.
constexpr int kMaxWarm = 4;
struct WarmRegions {
  const void *p[kMaxWarm];
  size_t bytes[kMaxWarm];
  int n;
};

// One layer's attention: q/k/v rows in, xo out; kc/vc are the layer's cache
// [nkv][clen][hdim]; rope the table [clen][hdim] (cos, sin interleaved) of
// the layer's base; part holds [n_heads][max_blocks][hdim + 2] fp64 partials.
struct DecAttn {
  const float *xq, *xk, *xv, *nq, *nk, *rope;
  float *kc, *vc;
  double *part;
  float *xo;
  const int *step;
  int n_heads, nkv, hdim, clen, slide, max_blocks, nvocab;
  float asc, sc_att, eps;
};

// norm prologue + int8 GEMV over jobs (gelu: jobs.w[0]/w[1] are gate/up,
// total = 2 * rows, output gelu(gate) * up to jobs.dst[0]); k % 16 == 0,
// k <= 6144 (k <= 4096 for gelu), rows 16-byte aligned
hipError_t launch_dec_norm_gemv(const DecNorm &na, const GemvJobs &jobs, int total, int k,
                                bool gelu, const DeviceInfo &dev, hipStream_t stream);
// The same for fp32 weights (the unquantized decode step): jobs.w fp32 rows
// (16-byte aligned), k = na.dim <= 6144 and a multiple of 4; gelu as above.
// Every workgroup normalizes into LDS as fp32; workgroup 0 stores x_out.
hipError_t launch_dec_norm_gemv_f32(const DecNorm &na, const GemvJobs &jobs, int total, int k,
                                    bool gelu, const DeviceInfo &dev, hipStream_t stream);
hipError_t launch_dec_embed(const DecEmbed &a, hipStream_t stream);
hipError_t launch_dec_final_norm(const DecNorm &na, hipStream_t stream);
hipError_t launch_dec_attention(const DecAttn &a, hipStream_t stream);
hipError_t launch_dec_softcap(float *logits, int n, float cap, hipStream_t stream);
// argmax over logits; writes step[0] = token, step[1] += 1, tokens[step[2]++]
hipError_t launch_dec_argmax(const float *logits, int n, float *pval, int *pidx, int nparts,
                             int *step, int *tokens, int max_tokens, hipStream_t stream);

// prefill.hip: the batched prompt pass (forward_text_chunk).
// Rows of x [n][dim] (in place), y [n][dim] nullable: the per-row form of
// DecNorm; h of every row is quantized into xq [n][dim] + xs [n].
// per row: x = clamp(x + post(y)), h = rmsnorm(x; w_pre) quantized into
// xq/xs, or, when xq is null, stored to h (fp32 rows [n][dim])
struct PfNorm {
  float *x;
  const float *y;
  const float *w_post;
  const float *w_pre;
  int8_t *xq;
  float *xs;
  int dim;
  float eps;
  float *h;
};
// qkv [n][stride]: q heads at column h*hdim, k heads from q_sz, v heads from
// q_sz + kv_sz; rows sit at positions pos0 .. pos0+n-1; kc/vc [nkv][clen][hdim]
struct PfRope {
  float *qkv;
  int stride, q_sz;
  const float *nq, *nk, *rope;
  float *kc, *vc;
  int clen, pos0, n_heads, nkv;
  float eps;
};
// attention of the n rows of qkv (q part) over kc/vc; xo [n][q_sz]
struct PfAttn {
  const float *qkv;
  int stride;
  const float *kc, *vc;
  float *xo;
  int q_sz, n, pos0, n_heads, nkv, clen, slide;
  float asc, sc_att;
  // key-range split: fp64 partials [kPfMaxSplit][n][q_sz] (unnormalized
  // value sums) then [kPfMaxSplit][n][n_heads][2] (reference max, sum);
  // chunk and nsplit are set by launch_pf_attention
  double *part;
  int chunk, nsplit;
  int qpb;  // query vectors per workgroup (set by launch_pf_attention)
  // 0: causal, sliding-window rows (forward_text_chunk with mask=true);
  // 1: every row sees keys 0 .. pos0+n-1, no window (mask=false, the image
  // tokens' bidirectional attention, gemma.c:5258-5290)
  int dense;
  // non-null: every output row is quantized into xq [n][q_sz] / xs [n] as
  // quantize_acts does (the o projection's input), in the merge pass, and
  // xo then holds only the rows the attention kernel wrote whole
  int8_t *xq;
  float *xs;
};
constexpr int kPfMaxSplit = 8;
constexpr int kPfMaxMergeHeads = 64;  // q heads the key-split merge handles
// doubles of PfAttn::part for n rows
inline size_t pf_attn_part_doubles(size_t n, size_t n_heads, size_t hdim) {
  return (size_t)kPfMaxSplit * n * n_heads * (hdim + 2);
}
// float4 chunks per thread of the row kernels: dim <= 6144 (256 threads),
// mlp <= 24576 (1024 threads)
constexpr int kPfMaxNpt = 6;
// emb_f non-null: an fp32 table (rows emb_f[token] * esc), else int8 rows
// scaled by esc * emb_s[token]
hipError_t launch_pf_embed(const int *tokens, int n, const int8_t *emb_q, const float *emb_s,
                           const float *emb_f, float *x, int dim, float esc, hipStream_t stream);
hipError_t launch_pf_norm_rows(const PfNorm &a, int n, hipStream_t stream);
hipError_t launch_pf_qk_rope(const PfRope &a, int n, int hdim, hipStream_t stream);
// hdim 128 or 256; the q heads per kv head must divide 32; a.part must hold
// pf_attn_part_doubles(n, n_heads, hdim) doubles
// f32: on the fp32 matrix cores (otherwise fp64, rounded once)
hipError_t launch_pf_attention(const PfAttn &a, int hdim, bool f32, const DeviceInfo &dev,
                               hipStream_t stream);
hipError_t launch_pf_gelu_quant(const float *g, int n, int mlp, int8_t *xq, float *xs,
                                const WarmRegions &warm, hipStream_t stream);
// rows g [n][2 * mlp] = (gate | up): gate = gelu(gate) * up in place (the
// fp32-weight path, where no quantize follows); mlp % 4 == 0
hipError_t launch_gelu_mul_rows(float *g, int n, int mlp, hipStream_t stream);

// vision.hip: the SigLIP tower (forward_vision).
// per row: x = clamp((y + bias) + x) when y is given; LayerNorm(x; w, b) into
// xq/xs (quantized) or, when xq is null, into h
struct VisLn {
  float *x;
  const float *y, *bias, *w, *b;
  int8_t *xq;
  float *xs;
  float *h;
  int dim;
  float eps;
};
// qkv [n][stride] (q | k | v, head h at column h*hdim of each), bias [3*dim]
struct VisAttn {
  const float *qkv;
  int stride;
  const float *bias;
  float *out;
  int n, n_heads, dim;
  float scale;
};
// h [ppi*ppi][dim] -> xq/xs [(ppi/ksize)^2][dim]: mean pooling, RMSNorm(w);
// when xq is null the normalized rows go to out (fp32)
struct VisPool {
  const float *h, *w;
  int8_t *xq;
  float *xs;
  int dim, ppi, ksize;
  float eps;
  float *out;
};
hipError_t launch_vis_ln_rows(const VisLn &a, int n, hipStream_t stream);
// head dim 16, 32, 64, 72 or 128
// f32: on the fp32 matrix cores (otherwise fp64, rounded once)
hipError_t launch_vis_attention(const VisAttn &a, int hdim, bool f32, hipStream_t stream);
hipError_t launch_vis_gelu_quant(const float *h, const float *bias, int n, int mlp, int8_t *xq,
                                 float *xs, const WarmRegions &warm, hipStream_t stream);
hipError_t launch_vis_pool(const VisPool &a, int ntok, hipStream_t stream);
// h [n][mlp] = gelu(h + bias) in place (the fp32-weight tower, where no
// quantize follows); mlp % 4 == 0
hipError_t launch_vis_bias_gelu(float *h, const float *bias, int n, int mlp, hipStream_t stream);

}  // namespace gh
