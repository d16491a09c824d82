// prefill.hip -- the batched prompt pass of the device-resident decoder
// (forward_text_chunk, gemma.c:4985-5453): the n prompt tokens go through
// every layer together, their int8 projections as GEMMs (gemm_i8.hip,
// bit-exact like the GEMVs) and the fp32 glue row by row on the GPU.
//
// Per layer:
//   norm rows        residual add of the previous MLP output (post-FFN norm
//                    n4), pre-attention norm n1, quantize each row
//   GEMM q, k, v     into one row-major [n][q_sz + 2 kv_sz] buffer
//   q/k rows         q/k norm, RoPE at each row's position, k and v rows
//                    appended to the KV cache
//   attention        causal (and sliding-window) attention of every row over
//                    the cache, query rows in tiles that share K/V tiles
//   quantize + GEMM o
//   norm rows        residual add of the attention output (post-attention
//                    norm n2), pre-FFN norm n3, quantize
//   GEMM gate, up    into one [n][2 mlp] buffer (gate first)
//   GELU rows        gelu(gate) * up, quantized per row
//   GEMM down
// The last row then takes the decode step's tail: final residual and norm,
// the LM head, softcap and argmax.
//
// Arithmetic is that of the decode step (decode.hip): the glue is evaluated
// in fp64 and rounded once where the reference stores fp32, so a prefill of
// n tokens computes, row for row, what n decode steps compute; the oracle of
// both is the fp64 decode oracle.  The reference's own prefill evaluates its
// attention in fp32 with a different order (blockwise gemm_fpx, softmax,
// gemm_fpx_nn), which no fp32 bit pattern here could follow anyway.
#include <type_traits>

#include "dec_common.h"

namespace gh {
namespace {

// x[r] = emb_q[tokens[r]] * (esc * emb_s[tokens[r]]) (gemma.c:5468-5493,
// per token); the host range-checks every token
__global__ __launch_bounds__(kNT) void pf_embed_kernel(const int *tokens, const int8_t *emb_q,
                                                       const float *emb_s, float *x, int dim,
                                                       float esc) {
  const int token = tokens[blockIdx.x];
  const float s = esc * emb_s[token];
  const int8_t *row = emb_q + (size_t)token * dim;
  float *xr = x + (size_t)blockIdx.x * dim;
  for (int i = threadIdx.x; i < dim; i += kNT) xr[i] = (float)row[i] * s;
}

// One workgroup per row: x[r] = clamp(x[r] + post(y[r])), h = rmsnorm(x[r],
// w_pre), h quantized into xq[r] / xs[r] (quantize_acts, gemma.c:2652-2674).
template <int NPT>
__global__ __launch_bounds__(kNT) void pf_norm_rows_kernel(PfNorm a) {
  __shared__ double red[kWaves];
  __shared__ float redf[kWaves];
  const size_t r = blockIdx.x;
  float *xr = a.x + r * a.dim;
  const DecNorm na{xr, a.y != nullptr ? a.y + r * a.dim : nullptr, a.w_post, a.w_pre, xr,
                   nullptr, a.dim, a.eps};
  NormIn<NPT> in;
  norm_load<NPT, kNT>(na, in);
  const float s = norm_quant<NPT, kNT, true>(na, in, a.xq + r * a.dim, red, redf);
  if (threadIdx.x == 0) a.xs[r] = s;
}

// One wave per (row, head): q heads are normalized (nq) and rotated in place;
// the kv heads' k rows are normalized (nk), rotated and stored to the cache at
// the row's position together with their v rows (gemma.c:5093-5150).  Lane l
// holds d = l + 64 j, so the RoPE pair (d, d + HD/2) is (j, j + HD/128) in
// the same lane -- the decode step's arithmetic, row by row.
template <int HD>
__global__ __launch_bounds__(64) void pf_qk_rope_kernel(PfRope a) {
  constexpr int NJ = HD / 64, NH = NJ / 2;
  const int r = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int pos = a.pos0 + r;
  const bool is_q = h < a.n_heads;
  const int hk = h - a.n_heads;
  float *row = a.qkv + (size_t)r * a.stride + (is_q ? h * HD : a.q_sz + hk * HD);
  const float *w = is_q ? a.nq : a.nk;
  const float *cs = a.rope + (size_t)pos * HD;
  float v[NJ], c[NH], s[NH];
#pragma unroll
  for (int jj = 0; jj < NJ; ++jj) v[jj] = row[lane + 64 * jj];
#pragma unroll
  for (int jj = 0; jj < NH; ++jj) {
    c[jj] = cs[2 * (lane + 64 * jj)];
    s[jj] = cs[2 * (lane + 64 * jj) + 1];
  }
  if (w != nullptr) {
    double ss = 0.0;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) ss += (double)v[jj] * (double)v[jj];
    const double rms = rms_of(wave_sum_f64(ss), HD, a.eps);
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) v[jj] = norm_one(v[jj], rms, w[lane + 64 * jj]);
  }
#pragma unroll
  for (int jj = 0; jj < NH; ++jj) {
    const double cd = c[jj], sd = s[jj];
    const double x0 = v[jj], x1 = v[jj + NH];
    v[jj] = (float)(x0 * cd - x1 * sd);
    v[jj + NH] = (float)(x0 * sd + x1 * cd);
  }
  if (is_q) {
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) row[lane + 64 * jj] = v[jj];
    return;
  }
  const size_t at = ((size_t)hk * a.clen + pos) * HD;
  const float *vrow = a.qkv + (size_t)r * a.stride + a.q_sz + (size_t)(a.nkv + hk) * HD;
#pragma unroll
  for (int jj = 0; jj < NJ; ++jj) {
    a.kc[at + lane + 64 * jj] = v[jj];
    a.vc[at + lane + 64 * jj] = vrow[lane + 64 * jj];
  }
}

// Causal attention of the prompt rows (gemma.c:5152-5293).  A workgroup takes
// one kv head and QB = 32 / hn consecutive rows, i.e. the 32 query vectors of
// its hn q heads at those rows, and walks the cached keys from the first
// row's window start to the last row's position in tiles of kPfKeys; each
// K/V tile is loaded once into LDS for all 32 queries.  Scores, masks, the
// running max and sum and the value sums are fp64 (an online softmax: on a
// new max the partial sums are rescaled by exp(m_old - m_new)); each output
// element is rounded to fp32 once at the end.
//
// Scores: thread (c, qg, kg) = (tid & 3, (tid >> 2) & 7, tid >> 5) sums
// quarter c of the head dimension for queries 4qg..4qg+3 and keys 2kg,
// 2kg+1 (8 products per 6 LDS vector reads), then the four quarters are
// added across lanes.  LDS rows are padded so that the 32 (qg, c) and 8
// (kg, c) addresses of one read fall in distinct 16-byte bank groups as far
// as 64 banks allow.
constexpr int kPfQ = 32;     // query vectors per workgroup
constexpr int kPfKeys = 16;  // keys per tile

template <int HD>
__global__ __launch_bounds__(kNT) void pf_attn_kernel(PfAttn a) {
  constexpr int QQ = HD / 4 + 4;       // one padded quarter of a row
  constexpr int KS = 4 * QQ;           // K row
  constexpr int QS = 4 * QQ + 4;       // q row
  constexpr int PS = kPfQ + 2;         // probabilities row (one key)
  constexpr int QPT = kPfQ * HD / kNT; // query vectors per thread in the value sums
  __shared__ __attribute__((aligned(16))) float qs[kPfQ * QS];
  __shared__ __attribute__((aligned(16))) float kt[kPfKeys * KS];
  __shared__ float vt[kPfKeys][HD];
  __shared__ __attribute__((aligned(16))) double pp[kPfKeys * PS];
  __shared__ double alpha[kPfQ], run_m[kPfQ], run_l[kPfQ];

  const int tid = threadIdx.x;
  const int hn = a.n_heads / a.nkv;
  const int qb = kPfQ / hn;                 // rows per workgroup
  const int hk = blockIdx.y;
  // the longest rows (most keys) first
  const int r0 = (gridDim.x - 1 - blockIdx.x) * qb;
  const int rows = min(qb, a.n - r0);
  // query vector v: head h0 + v / qb, row r0 + v % qb
  auto q_row = [&](int v) { return r0 + v % qb; };
  auto q_head = [&](int v) { return hk * hn + v / qb; };
  auto window_start = [&](int p_abs) {
    return (a.slide > 0 && p_abs >= a.slide) ? p_abs + 1 - a.slide : 0;
  };

  for (int i = tid; i < kPfQ * HD / 4; i += kNT) {
    const int v = i / (HD / 4), c4 = i - v * (HD / 4);  // 4 floats at d = 4 c4
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    const v4f x = v % qb < rows ? reinterpret_cast<const v4f *>(
                                      a.qkv + (size_t)q_row(v) * a.stride + q_head(v) * HD)[c4]
                                : zero;
    const int d = 4 * c4;
    *reinterpret_cast<v4f *>(&qs[v * QS + (d / (HD / 4)) * QQ + d % (HD / 4)]) = x;
  }
  if (tid < kPfQ) {
    run_m[tid] = -DBL_MAX;
    run_l[tid] = 0.0;
  }
  const int p_first = a.pos0 + r0, p_last = a.pos0 + r0 + rows - 1;
  const int k_lo = window_start(p_first) / kPfKeys * kPfKeys;
  const float *kc = a.kc + (size_t)hk * a.clen * HD;
  const float *vc = a.vc + (size_t)hk * a.clen * HD;

  double acc[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) acc[u] = 0.0;
  const int d_own = tid % HD;           // this thread's dimension in the value sums
  const int v_own = (tid / HD) * QPT;   // and its first query vector
  const int sc_c = tid & 3, sc_qg = (tid >> 2) & 7, sc_kg = tid >> 5;

  for (int t0 = k_lo; t0 <= p_last; t0 += kPfKeys) {
    lds_barrier();  // the previous tile's K, V and p are no longer read
    for (int i = tid; i < kPfKeys * HD / 4; i += kNT) {
      const int t = i / (HD / 4), c4 = i - t * (HD / 4);
      const int kp = t0 + t;
      const v4f zero = {0.f, 0.f, 0.f, 0.f};
      const v4f kv4 = kp <= p_last ? reinterpret_cast<const v4f *>(kc + (size_t)kp * HD)[c4]
                                   : zero;
      const v4f vv4 = kp <= p_last ? reinterpret_cast<const v4f *>(vc + (size_t)kp * HD)[c4]
                                   : zero;
      const int d = 4 * c4;
      *reinterpret_cast<v4f *>(&kt[t * KS + (d / (HD / 4)) * QQ + d % (HD / 4)]) = kv4;
      *reinterpret_cast<v4f *>(&vt[t][d]) = vv4;
    }
    lds_barrier();
    {
      const float *qb4 = &qs[(4 * sc_qg) * QS + sc_c * QQ];
      const float *kb2 = &kt[(2 * sc_kg) * KS + sc_c * QQ];
      double s[4][2];
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j][0] = s[j][1] = 0.0;
#pragma unroll 4
      for (int i = 0; i < HD / 4; i += 4) {
        const v4f k0 = *reinterpret_cast<const v4f *>(kb2 + i);
        const v4f k1 = *reinterpret_cast<const v4f *>(kb2 + KS + i);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v4f q = *reinterpret_cast<const v4f *>(qb4 + j * QS + i);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s[j][0] = fma((double)q[e], (double)k0[e], s[j][0]);
            s[j][1] = fma((double)q[e], (double)k1[e], s[j][1]);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          double part = s[j][kk];
          part += dpp_f64<kDppXor1>(part);
          part += dpp_f64<kDppXor2>(part);
          const int v = 4 * sc_qg + j, t = 2 * sc_kg + kk;
          if (sc_c == 0) {
            const int p_abs = a.pos0 + q_row(v);
            const int kp = t0 + t;
            const bool live = v % qb < rows && kp <= p_abs && kp >= window_start(p_abs);
            double sc = part * (double)a.asc;
            if (a.sc_att != 0.0f) sc = tanh(sc / (double)a.sc_att) * (double)a.sc_att;
            pp[t * PS + v] = live ? sc : -DBL_MAX;
          }
        }
    }
    lds_barrier();
    // online softmax: 16 lanes (one DPP row) per query vector, lane t = key t
    for (int v = tid / kPfKeys; v < kPfQ; v += kNT / kPfKeys) {
      const int t = tid % kPfKeys;
      const double sv = pp[t * PS + v];
      double m = sv;
      m = fmax(m, dpp_f64<kDppXor1>(m));
      m = fmax(m, dpp_f64<kDppXor2>(m));
      m = fmax(m, dpp_f64<kDppHalfMirror>(m));
      m = fmax(m, dpp_f64<kDppMirror>(m));
      const double m_old = run_m[v];
      const double m_new = fmax(m_old, m);
      const double e = sv == -DBL_MAX ? 0.0 : exp(sv - m_new);
      double l = e;
      l += dpp_f64<kDppXor1>(l);
      l += dpp_f64<kDppXor2>(l);
      l += dpp_f64<kDppHalfMirror>(l);
      l += dpp_f64<kDppMirror>(l);
      pp[t * PS + v] = e;
      if (t == 0) {
        const double al = exp(m_old - m_new);
        alpha[v] = al;
        run_l[v] = run_l[v] * al + l;
        run_m[v] = m_new;
      }
    }
    lds_barrier();
    // value sums: thread (d, queries v_own .. v_own + QPT - 1); the key's
    // probabilities of two queries are one 16-byte broadcast read
#pragma unroll
    for (int u = 0; u < QPT; ++u) acc[u] *= alpha[v_own + u];
#pragma unroll 4
    for (int t = 0; t < kPfKeys; ++t) {
      const double vv = (double)vt[t][d_own];
      const double *pt = &pp[t * PS + v_own];
#pragma unroll
      for (int u = 0; u < QPT; u += 2) {
        const double2 pr = *reinterpret_cast<const double2 *>(pt + u);
        acc[u] = fma(pr.x, vv, acc[u]);
        acc[u + 1] = fma(pr.y, vv, acc[u + 1]);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int v = v_own + u;
    if (v % qb < rows)
      a.xo[(size_t)q_row(v) * a.q_sz + q_head(v) * HD + d_own] = (float)(acc[u] / run_l[v]);
  }
}

// One workgroup per row: out = gelu(gate) * up (gemma.c:4139-4172, the GELU
// gate fused with the up projection) rounded once, then quantized into
// xq[r] / xs[r] as quantize_act does.  g is [n][2 mlp], gate columns first.
template <int NPT, int NT>
__global__ __launch_bounds__(NT) void pf_gelu_quant_kernel(const float *g, int mlp, int8_t *xq,
                                                           float *xs) {
  __shared__ float redf[NT / 64];
  const int tid = threadIdx.x;
  const int n4 = mlp >> 2;
  const float *gate = g + (size_t)blockIdx.x * 2 * mlp;
  const float *up = gate + mlp;
  v4f out[NPT];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    const v4f gv = c < n4 ? reinterpret_cast<const v4f *>(gate)[c] : zero;
    const v4f uv = c < n4 ? reinterpret_cast<const v4f *>(up)[c] : zero;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[j][e] = (float)(gelu_tanh((double)gv[e]) * (double)uv[e]);
      amax = fmaxf(amax, abs_daz(out[j][e]));
    }
  }
  amax = block_max<NT>(amax, redf);
  const QuantParams qp = quant_params(amax);
  int8_t *row = xq + (size_t)blockIdx.x * mlp;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
    if (c < n4)
      reinterpret_cast<uint32_t *>(row)[c] =
          pack4(quant_one(out[j].x, qp.inv), quant_one(out[j].y, qp.inv),
                quant_one(out[j].z, qp.inv), quant_one(out[j].w, qp.inv));
  }
  if (tid == 0) xs[blockIdx.x] = qp.scale;
}

template <int C, int CMAX, class F>
hipError_t by_npt(int npt, F &&launch) {
  if (npt == C) return launch(std::integral_constant<int, C>{});
  if constexpr (C < CMAX) return by_npt<C + 1, CMAX>(npt, launch);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_pf_embed(const int *tokens, int n, const int8_t *emb_q, const float *emb_s,
                           float *x, int dim, float esc, hipStream_t stream) {
  pf_embed_kernel<<<n, kNT, 0, stream>>>(tokens, emb_q, emb_s, x, dim, esc);
  return hipGetLastError();
}

hipError_t launch_pf_norm_rows(const PfNorm &a, int n, hipStream_t stream) {
  const int npt = (a.dim / 4 + kNT - 1) / kNT;
  return by_npt<1, kPfMaxNpt>(npt, [&](auto c) {
    pf_norm_rows_kernel<decltype(c)::value><<<n, kNT, 0, stream>>>(a);
    return hipGetLastError();
  });
}

hipError_t launch_pf_qk_rope(const PfRope &a, int n, int hdim, hipStream_t stream) {
  const dim3 grid(n, a.n_heads + a.nkv);
  switch (hdim) {
    case 128: pf_qk_rope_kernel<128><<<grid, 64, 0, stream>>>(a); break;
    case 256: pf_qk_rope_kernel<256><<<grid, 64, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_pf_attention(const PfAttn &a, int hdim, hipStream_t stream) {
  const int qb = kPfQ / (a.n_heads / a.nkv);
  const dim3 grid((a.n + qb - 1) / qb, a.nkv);
  switch (hdim) {
    case 128: pf_attn_kernel<128><<<grid, kNT, 0, stream>>>(a); break;
    case 256: pf_attn_kernel<256><<<grid, kNT, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_pf_gelu_quant(const float *g, int n, int mlp, int8_t *xq, float *xs,
                                hipStream_t stream) {
  constexpr int NT = 1024;
  const int npt = (mlp / 4 + NT - 1) / NT;
  return by_npt<1, kPfMaxNpt>(npt, [&](auto c) {
    pf_gelu_quant_kernel<decltype(c)::value, NT><<<n, NT, 0, stream>>>(g, mlp, xq, xs);
    return hipGetLastError();
  });
}

}  // namespace gh
