// decode.hip -- the kernels of the device-resident decode step
// (forward_gemma_decode + forward_text_decode, gemma.c:5456-5499 and
// 4727-4983): the fp32 work between two int8 GEMVs runs on the GPU too, so a
// token costs no PCIe round trip.
//
// Per layer the step is six launches (captured once into a HIP graph):
//   norm-GEMV q/k/v   residual add of the previous MLP output (post-FFN
//                     norm n4), pre-attention norm n1, quantize, q/k/v GEMV
//   attention         q/k norm, RoPE, KV-cache append, scores, softmax and
//                     the value sum over one block of keys per workgroup
//   combine           the per-block softmax partials -> attention output
//   GEMV o            (gemv.hip, quantize fused)
//   norm-GEMV gate/up residual add of the attention output (post-attention
//                     norm n2), pre-FFN norm n3, quantize, gate and up rows
//                     in pairs, GELU(gate) * up fused into the epilogue
//   GEMV down         (gemv.hip, quantize fused)
// The residual update and the norms are computed by every workgroup of the
// norm-GEMV from the same inputs in the same order (the vector is at most a
// few thousand floats), so no extra launch or grid-wide sync is needed;
// workgroup 0 stores the new residual for the next layer.
//
// Arithmetic.  The int8 parts (quantize, dot products, rescale) use the
// bit-exact arithmetic of gh_arith.h.  The fp32 glue follows the reference's
// formulas (rmsnorm 2508-2521, clamp_fpx 2504-2506, RoPE 4223-4246, scores,
// att_finalize and softmax 4091-4131, gelu_tanh 4139-4145) but is evaluated
// in fp64 and rounded to fp32 once, where the reference stores an fp32
// tensor; residual adds and the embedding scale are single fp32 operations.
// The reference leaves its fp32 summation order to the compiler, so no fp32
// bit pattern is canonical for the glue; the correctly rounded value is, and
// it is what the decode oracle computes.  This matters because the next
// quantize turns a 1-ulp difference that straddles a rounding boundary into
// a whole int8 step.
#include <float.h>
#include <math.h>

#include "gh_arith.h"
#include "gh_kernels.h"

namespace gh {
namespace {

constexpr int kNT = 256;
constexpr int kWaves = kNT / 64;

__device__ __forceinline__ double block_sum(double v, double *red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) s += red[w];
  return s;
}

__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) s = fmaxf(s, red[w]);
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

// x_new = clamp(x_res + post(y)), then h = rmsnorm(x_new, w_pre) into xs.
// Every thread handles elements i = tid, tid + 256, ...; workgroup 0 stores
// x_new (and h when h_out is given).
__device__ void norm_prologue(const DecNorm &a, float *xs, double *red) {
  const int tid = threadIdx.x;
  const int dim = a.dim;
  if (a.y != nullptr) {
    double rms = 1.0;
    if (a.w_post != nullptr) {
      double ss = 0.0;
      for (int i = tid; i < dim; i += kNT) {
        const double v = a.y[i];
        ss += v * v;
      }
      rms = rms_of(block_sum(ss, red), dim, a.eps);
    }
    for (int i = tid; i < dim; i += kNT) {
      const float t = a.w_post != nullptr ? norm_one(a.y[i], rms, a.w_post[i]) : a.y[i];
      xs[i] = clamp_f32(t + a.x_res[i]);
    }
  } else {
    for (int i = tid; i < dim; i += kNT) xs[i] = a.x_res[i];
  }
  if (blockIdx.x == 0 && a.x_out != nullptr)
    for (int i = tid; i < dim; i += kNT) a.x_out[i] = xs[i];
  double ss = 0.0;
  for (int i = tid; i < dim; i += kNT) ss += (double)xs[i] * (double)xs[i];
  const double rms = rms_of(block_sum(ss, red), dim, a.eps);
  for (int i = tid; i < dim; i += kNT) xs[i] = norm_one(xs[i], rms, a.w_pre[i]);
  if (blockIdx.x == 0 && a.h_out != nullptr)
    for (int i = tid; i < dim; i += kNT) a.h_out[i] = xs[i];
  __syncthreads();
}

// Quantizes xs[0..k) into xq (LDS) exactly as quantize_act does
// (gemma.c:2590-2650); returns the activation scale.
__device__ float quantize_lds(const float *xs, int8_t *xq, int k, float *red) {
  const int tid = threadIdx.x;
  float amax = 0.0f;
  for (int i = tid; i < k; i += kNT) amax = fmaxf(amax, abs_daz(xs[i]));
  amax = block_max(amax, red);
  const QuantParams qp = quant_params(amax);
  for (int c = tid; c < k / 4; c += kNT)
    reinterpret_cast<uint32_t *>(xq)[c] =
        pack4(quant_one(xs[4 * c], qp.inv), quant_one(xs[4 * c + 1], qp.inv),
              quant_one(xs[4 * c + 2], qp.inv), quant_one(xs[4 * c + 3], qp.inv));
  __syncthreads();
  return qp.scale;
}

__device__ __forceinline__ int32_t dot16(v4i w, v4i x, int32_t acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}

// The int8 GEMV behind the norm prologue.  L lanes per row, CPL 16-byte
// chunks per lane; each lane issues the loads of its first row before the
// prologue so HBM latency overlaps it.
//  GELU == false: rows are the flat row range of `jobs` (q, k, v).
//  GELU == true:  virtual row 2r is gate row r (jobs.w[0]), 2r+1 is up row r
//                 (jobs.w[1]); both sit in one wave (L <= 32), and the lanes
//                 of the gate row store gelu(gate) * up to jobs.dst[0][r].
// Requires k % 16 == 0, 16-byte aligned weight rows, k <= L * CPL * 16.
template <int L, int CPL, bool GELU>
__global__ __launch_bounds__(kNT) void dec_norm_gemv_kernel(DecNorm na, GemvJobs jobs,
                                                            int total, int k) {
  extern __shared__ v4i lds4[];
  __shared__ double red[kWaves];
  __shared__ float redf[kWaves];
  float *xs = reinterpret_cast<float *>(lds4);
  v4i *xq4 = lds4 + (k * 4 + 15) / 16;
  static_assert(!GELU || L <= 32, "gate and up rows must share a wave");
  constexpr int kRowsPerWave = 64 / L;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % L;
  const int rloc = lane / L;
  const int kc = k >> 4;
  const int stride = gridDim.x * kWaves * kRowsPerWave;

  auto locate = [&](int row, int *r) -> int {
    if (GELU) {
      *r = row >> 1;
      return row & 1;
    }
    int j = 0, start = 0;
#pragma unroll
    for (int t = 0; t < kMaxJobs - 1; ++t)
      if (t + 1 < jobs.njobs && row >= jobs.end[t]) {
        j = t + 1;
        start = jobs.end[t];
      }
    *r = row - start;
    return j;
  };
  auto pick_w = [&](int j) {
    const void *v = jobs.w[0];
#pragma unroll
    for (int t = 1; t < kMaxJobs; ++t)
      if (j == t) v = jobs.w[t];
    return static_cast<const v4i *>(v);
  };
  auto pick_sc = [&](int j) {
    const float *v = jobs.sc[0];
#pragma unroll
    for (int t = 1; t < kMaxJobs; ++t)
      if (j == t) v = jobs.sc[t];
    return v;
  };
  auto pick_dst = [&](int j) {
    float *v = jobs.dst[0];
#pragma unroll
    for (int t = 1; t < kMaxJobs; ++t)
      if (j == t) v = jobs.dst[t];
    return v;
  };
  auto load_row = [&](int row, v4i (&buf)[CPL]) {
    if (row < total) {
      int r;
      const int j = locate(row, &r);
      const v4i *w4 = pick_w(j) + (size_t)r * kc;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = sub + i * L;
        buf[i] = c < kc ? __builtin_nontemporal_load(w4 + c) : v4i{0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int i = 0; i < CPL; ++i) buf[i] = v4i{0, 0, 0, 0};
    }
  };

  int base = (blockIdx.x * kWaves + wave) * kRowsPerWave;
  v4i cur[CPL];
  load_row(base + rloc, cur);
  norm_prologue(na, xs, red);
  const float act_scale = quantize_lds(xs, reinterpret_cast<int8_t *>(xq4), k, redf);

  for (; base < total; base += stride) {
    const int row = base + rloc;
    v4i nxt[CPL];
    load_row(row + stride, nxt);
    int32_t acc = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;
      if (c < kc) acc = dot16(cur[i], xq4[c], acc);
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    int r = 0;
    const int j = locate(row < total ? row : 0, &r);
    const float val = row < total ? rescale(acc, act_scale, pick_sc(j)[r]) : 0.0f;
    if (GELU) {
      const float up = __shfl_xor(val, L, 64);
      if (sub == 0 && (rloc & 1) == 0 && row < total)
        jobs.dst[0][r] = (float)(gelu_tanh((double)val) * (double)up);
    } else if (sub == 0 && row < total) {
      pick_dst(j)[r] = val;
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) cur[i] = nxt[i];
  }
}

// x = dequantized embedding row of the step's token (gemma.c:5468-5493)
__global__ __launch_bounds__(kNT) void dec_embed_kernel(DecEmbed a) {
  int token, pos;
  if (!step_ok(a.step, a.nvocab, a.clen, &token, &pos)) return;
  const float esc = a.esc * a.emb_s[token];
  const int8_t *row = a.emb_q + (size_t)token * a.dim;
  for (int i = threadIdx.x; i < a.dim; i += kNT) a.x[i] = (float)row[i] * esc;
}

// Final residual add + final norm (gemma.c:4950-4955): one workgroup writes h.
__global__ __launch_bounds__(kNT) void dec_final_norm_kernel(DecNorm na) {
  extern __shared__ v4i lds4[];
  __shared__ double red[kWaves];
  norm_prologue(na, reinterpret_cast<float *>(lds4), red);
}

// Attention of one kv head over one block of keys (gemma.c:4776-4851):
// grid (max blocks, nkv).  The workgroup prepares the q heads of its group
// (q norm, RoPE) and the new k (k norm, RoPE) and v rows in LDS; block 0
// appends k and v to the cache.  Keys before the step's position are read
// from the cache, the key at the position from LDS, so no workgroup waits
// for another.  Output per (q head, block), in fp64: the block's max score
// m, l = sum exp(s - m) and acc[d] = sum exp(s - m) v[d]; the combine kernel
// merges the blocks.
__global__ __launch_bounds__(kNT) void dec_attn_kernel(DecAttn a) {
  extern __shared__ double smem_d[];
  __shared__ double red[kWaves];
  int token, pos;
  if (!step_ok(a.step, a.nvocab, a.clen, &token, &pos)) return;
  const int hd = a.hdim;
  const int hk = blockIdx.y;
  const int hn = a.n_heads / a.nkv;
  const int h0 = hk * hn;
  const int spos = (a.slide > 0 && pos >= a.slide) ? pos + 1 - a.slide : 0;
  const int t0 = spos + blockIdx.x * a.block;
  if (t0 > pos) return;
  const int t1 = min(t0 + a.block, pos + 1);
  const int nt = t1 - t0;
  const int tid = threadIdx.x;

  double *s = smem_d;                                  // [hn][block]
  float *q = reinterpret_cast<float *>(s + hn * a.block);  // [hn][hd]
  float *kn = q + hn * hd;                             // [hd]
  float *vn = kn + hd;                                 // [hd]
  const float *cs = a.rope + (size_t)pos * hd;         // cos, sin interleaved

  // q heads: optional rmsnorm with nq, then RoPE (gemma.c:4778-4800)
  for (int g = 0; g < hn; ++g) {
    const float *src = a.xq + (size_t)(h0 + g) * hd;
    double rms = 1.0;
    if (a.nq != nullptr) {
      double ss = 0.0;
      for (int d = tid; d < hd; d += kNT) ss += (double)src[d] * (double)src[d];
      rms = rms_of(block_sum(ss, red), hd, a.eps);
    }
    for (int d = tid; d < hd; d += kNT)
      q[g * hd + d] = a.nq != nullptr ? norm_one(src[d], rms, a.nq[d]) : src[d];
    __syncthreads();
    for (int d = tid; d < hd / 2; d += kNT) {
      const double c = cs[2 * d], sn = cs[2 * d + 1];
      const double x0 = q[g * hd + d], x1 = q[g * hd + d + hd / 2];
      q[g * hd + d] = (float)(x0 * c - x1 * sn);
      q[g * hd + d + hd / 2] = (float)(x0 * sn + x1 * c);
    }
    __syncthreads();
  }
  // the new key (k norm, RoPE) and value rows
  {
    const float *src = a.xk + (size_t)hk * hd;
    double rms = 1.0;
    if (a.nk != nullptr) {
      double ss = 0.0;
      for (int d = tid; d < hd; d += kNT) ss += (double)src[d] * (double)src[d];
      rms = rms_of(block_sum(ss, red), hd, a.eps);
    }
    for (int d = tid; d < hd; d += kNT) {
      kn[d] = a.nk != nullptr ? norm_one(src[d], rms, a.nk[d]) : src[d];
      vn[d] = a.xv[(size_t)hk * hd + d];
    }
    __syncthreads();
    for (int d = tid; d < hd / 2; d += kNT) {
      const double c = cs[2 * d], sn = cs[2 * d + 1];
      const double x0 = kn[d], x1 = kn[d + hd / 2];
      kn[d] = (float)(x0 * c - x1 * sn);
      kn[d + hd / 2] = (float)(x0 * sn + x1 * c);
    }
    __syncthreads();
  }
  float *kc = a.kc + (size_t)hk * a.clen * hd;
  float *vc = a.vc + (size_t)hk * a.clen * hd;
  if (blockIdx.x == 0)
    for (int d = tid; d < hd; d += kNT) {
      kc[(size_t)pos * hd + d] = kn[d];
      vc[(size_t)pos * hd + d] = vn[d];
    }

  // scores: one key per wave at a time, lanes split the head dimension
  const int lane = tid & 63, wave = tid >> 6;
  for (int t = wave; t < nt; t += kWaves) {
    const int key = t0 + t;
    const float *kr = key == pos ? kn : kc + (size_t)key * hd;
    for (int g = 0; g < hn; ++g) {
      double part = 0.0;
      for (int d = lane; d < hd; d += 64) part += (double)q[g * hd + d] * (double)kr[d];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
      if (lane == 0) {
        double sc = part * (double)a.asc;
        if (a.sc_att != 0.0f) sc = tanh(sc / (double)a.sc_att) * (double)a.sc_att;
        s[g * a.block + t] = sc;
      }
    }
  }
  __syncthreads();
  // per head: max, exp, sum, and the value sum
  for (int g = 0; g < hn; ++g) {
    double m = -DBL_MAX;
    for (int t = tid; t < nt; t += kNT) m = fmax(m, s[g * a.block + t]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmax(m, __shfl_xor(m, off, 64));
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m = fmax(m, red[w]);
    double l = 0.0;
    for (int t = tid; t < nt; t += kNT) {
      const double e = exp(s[g * a.block + t] - m);
      s[g * a.block + t] = e;
      l += e;
    }
    l = block_sum(l, red);
    double *out = a.part + ((size_t)(h0 + g) * a.max_blocks + blockIdx.x) * (hd + 2);
    for (int d = tid; d < hd; d += kNT) {
      double acc = 0.0;
      for (int t = 0; t < nt; ++t) {
        const int key = t0 + t;
        const double v = key == pos ? vn[d] : vc[(size_t)key * hd + d];
        acc += s[g * a.block + t] * v;
      }
      out[d] = acc;
    }
    if (tid == 0) {
      out[hd] = m;
      out[hd + 1] = l;
    }
    __syncthreads();
  }
}

// xo[h] = sum_b exp(m_b - M) acc_b / sum_b exp(m_b - M) l_b: grid n_heads
__global__ __launch_bounds__(kNT) void dec_attn_combine_kernel(DecAttn a) {
  int token, pos;
  if (!step_ok(a.step, a.nvocab, a.clen, &token, &pos)) return;
  const int hd = a.hdim, h = blockIdx.x;
  const int spos = (a.slide > 0 && pos >= a.slide) ? pos + 1 - a.slide : 0;
  const int nb = (pos + 1 - spos + a.block - 1) / a.block;
  const double *p = a.part + (size_t)h * a.max_blocks * (hd + 2);
  double m = -DBL_MAX;
  for (int b = 0; b < nb; ++b) m = fmax(m, p[(size_t)b * (hd + 2) + hd]);
  double den = 0.0;
  for (int b = 0; b < nb; ++b) {
    const double *pb = p + (size_t)b * (hd + 2);
    den += exp(pb[hd] - m) * pb[hd + 1];
  }
  for (int d = threadIdx.x; d < hd; d += kNT) {
    double num = 0.0;
    for (int b = 0; b < nb; ++b) {
      const double *pb = p + (size_t)b * (hd + 2);
      num += exp(pb[hd] - m) * pb[d];
    }
    a.xo[(size_t)h * hd + d] = (float)(num / den);
  }
}

// Logit softcap (gemma.c:4970-4977)
__global__ __launch_bounds__(kNT) void dec_softcap_kernel(float *logits, int n, float cap) {
  const int i = blockIdx.x * kNT + threadIdx.x;
  if (i < n) logits[i] = (float)(tanh((double)logits[i] / (double)cap) * (double)cap);
}

// argmax, lowest index on ties (gemma.c:5600-5630): stage 1 per workgroup
__global__ __launch_bounds__(kNT) void dec_argmax_partial_kernel(const float *logits, int n,
                                                                 float *pval, int *pidx) {
  float best = -FLT_MAX;
  int bi = -1;
  for (int i = blockIdx.x * kNT + threadIdx.x; i < n; i += gridDim.x * kNT) {
    const float v = logits[i];
    if (v > best) {
      best = v;
      bi = i;
    }
  }
  __shared__ float sv[kNT];
  __shared__ int si[kNT];
  sv[threadIdx.x] = best;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int w = kNT / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      const float ov = sv[threadIdx.x + w];
      const int oi = si[threadIdx.x + w];
      if (oi >= 0 && (si[threadIdx.x] < 0 || ov > sv[threadIdx.x] ||
                      (ov == sv[threadIdx.x] && oi < si[threadIdx.x]))) {
        sv[threadIdx.x] = ov;
        si[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    pval[blockIdx.x] = sv[0];
    pidx[blockIdx.x] = si[0];
  }
}

// stage 2: one workgroup; writes the token, advances the step for the next
// launch and appends the token to the output list
__global__ __launch_bounds__(kNT) void dec_argmax_final_kernel(const float *pval, const int *pidx,
                                                               int nparts, int *step, int *tokens,
                                                               int max_tokens) {
  __shared__ float sv[kNT];
  __shared__ int si[kNT];
  float best = -FLT_MAX;
  int bi = -1;
  for (int i = threadIdx.x; i < nparts; i += kNT) {
    const float v = pval[i];
    const int ix = pidx[i];
    if (ix >= 0 && (bi < 0 || v > best || (v == best && ix < bi))) {
      best = v;
      bi = ix;
    }
  }
  sv[threadIdx.x] = best;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int w = kNT / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      const float ov = sv[threadIdx.x + w];
      const int oi = si[threadIdx.x + w];
      if (oi >= 0 && (si[threadIdx.x] < 0 || ov > sv[threadIdx.x] ||
                      (ov == sv[threadIdx.x] && oi < si[threadIdx.x]))) {
        sv[threadIdx.x] = ov;
        si[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int count = step[2];
    if (count >= 0 && count < max_tokens) tokens[count] = si[0];
    step[0] = si[0];
    step[1] = step[1] + 1;
    step[2] = count + 1;
  }
}

template <int L, int CPL, bool GELU>
hipError_t launch_norm_gemv_t(const DecNorm &na, const GemvJobs &jobs, int total, int k,
                              const DeviceInfo &dev, hipStream_t stream) {
  constexpr int rows_per_block = kWaves * (64 / L);
  long blocks = (total + rows_per_block - 1) / rows_per_block;
  const long cap = (long)dev.cus * 8;
  const size_t lds = (size_t)(k * 4 + 15) / 16 * 16 + (size_t)k;
  dec_norm_gemv_kernel<L, CPL, GELU>
      <<<dim3((unsigned)(blocks < cap ? blocks : cap)), kNT, lds, stream>>>(na, jobs, total, k);
  return hipGetLastError();
}

template <int L, bool GELU>
hipError_t norm_gemv_cpl(int cpl, const DecNorm &na, const GemvJobs &jobs, int total, int k,
                         const DeviceInfo &dev, hipStream_t stream) {
  switch (cpl) {
    case 1: return launch_norm_gemv_t<L, 1, GELU>(na, jobs, total, k, dev, stream);
    case 2: return launch_norm_gemv_t<L, 2, GELU>(na, jobs, total, k, dev, stream);
    case 3: return launch_norm_gemv_t<L, 3, GELU>(na, jobs, total, k, dev, stream);
    case 4: return launch_norm_gemv_t<L, 4, GELU>(na, jobs, total, k, dev, stream);
    case 5: return launch_norm_gemv_t<L, 5, GELU>(na, jobs, total, k, dev, stream);
    case 6: return launch_norm_gemv_t<L, 6, GELU>(na, jobs, total, k, dev, stream);
    case 7: return launch_norm_gemv_t<L, 7, GELU>(na, jobs, total, k, dev, stream);
    case 8: return launch_norm_gemv_t<L, 8, GELU>(na, jobs, total, k, dev, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_dec_norm_gemv(const DecNorm &na, const GemvJobs &jobs, int total, int k,
                                bool gelu, const DeviceInfo &dev, hipStream_t stream) {
  const int kc = k / 16;
  // 32 lanes per row (two rows per wave, as the gate/up pairing needs) up to
  // 256 chunks (k = 4096); 64 lanes beyond that for plain rows
  if (kc <= 32 * 8 || gelu) {
    const int cpl = (kc + 31) / 32;
    return gelu ? norm_gemv_cpl<32, true>(cpl, na, jobs, total, k, dev, stream)
                : norm_gemv_cpl<32, false>(cpl, na, jobs, total, k, dev, stream);
  }
  return norm_gemv_cpl<64, false>((kc + 63) / 64, na, jobs, total, k, dev, stream);
}

hipError_t launch_dec_embed(const DecEmbed &a, hipStream_t stream) {
  dec_embed_kernel<<<1, kNT, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_dec_final_norm(const DecNorm &na, hipStream_t stream) {
  dec_final_norm_kernel<<<1, kNT, (size_t)na.dim * 4, stream>>>(na);
  return hipGetLastError();
}

hipError_t launch_dec_attention(const DecAttn &a, hipStream_t stream) {
  const int hn = a.n_heads / a.nkv;
  const size_t lds = (size_t)hn * a.block * 8 + ((size_t)hn * a.hdim + 2 * (size_t)a.hdim) * 4;
  dec_attn_kernel<<<dim3(a.max_blocks, a.nkv), kNT, lds, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dec_attn_combine_kernel<<<a.n_heads, kNT, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_dec_softcap(float *logits, int n, float cap, hipStream_t stream) {
  dec_softcap_kernel<<<(n + kNT - 1) / kNT, kNT, 0, stream>>>(logits, n, cap);
  return hipGetLastError();
}

hipError_t launch_dec_argmax(const float *logits, int n, float *pval, int *pidx, int nparts,
                             int *step, int *tokens, int max_tokens, hipStream_t stream) {
  dec_argmax_partial_kernel<<<nparts, kNT, 0, stream>>>(logits, n, pval, pidx);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dec_argmax_final_kernel<<<1, kNT, 0, stream>>>(pval, pidx, nparts, step, tokens, max_tokens);
  return hipGetLastError();
}

}  // namespace gh
