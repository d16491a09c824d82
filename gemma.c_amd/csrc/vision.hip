// vision.hip -- the SigLIP vision tower of forward_vision (gemma.c:4394-4725)
// on the GPU: patch embedding, position embedding, the encoder layers
// (layer norm, q/k/v with biases, full attention over the patches, o, layer
// norm, fc1 with bias and GELU, fc2), the post layer norm, average pooling
// down to the image tokens, the soft-embedding RMSNorm and the projection
// into the text model's width.  The int8 projections are the library's
// GEMMs (gemm_i8.hip, bit-exact); these kernels are the fp32 glue between
// them, evaluated as the decode step's glue is (decode.hip): in fp64 from
// the reference's formulas, rounded to fp32 once where the reference stores
// an fp32 tensor, with single fp32 additions (biases, residuals, the
// dequantized position embedding) kept as the single fp32 operations they
// are.
#include <type_traits>

#include "dec_common.h"

namespace gh {
namespace {

// Patch embedding as a GEMM over im2col patches (gemma.c:4411-4448), in fp64:
// x[p][oc] = clamp((float)(sum_k a[p][k] * pe[oc][k] + pe_b[oc])), then the
// position embedding row p dequantized in fp32 and added (4452-4468):
// x = clamp(x + (float)q * scale).  A workgroup computes a 32 x 64 tile,
// each thread 2 x 4 outputs, over K in LDS chunks of 32.
constexpr int kVpM = 32, kVpN = 64, kVpK = 32;

__global__ __launch_bounds__(kNT) void vis_patch_kernel(VisPatch a) {
  __shared__ float as[kVpM][kVpK + 1];
  __shared__ float bs[kVpN][kVpK + 1];
  const int tid = threadIdx.x;
  const int m0 = blockIdx.x * kVpM, n0 = blockIdx.y * kVpN;
  const int tm = tid / 16, tn = tid % 16;  // outputs (m0 + 2 tm + i, n0 + tn + 16 j)
  double acc[2][4] = {};
  for (int k0 = 0; k0 < a.k; k0 += kVpK) {
    for (int i = tid; i < kVpM * kVpK; i += kNT) {
      const int r = i / kVpK, c = i % kVpK;
      as[r][c] = (m0 + r < a.m && k0 + c < a.k) ? a.patches[(size_t)(m0 + r) * a.k + k0 + c]
                                                 : 0.0f;
    }
    for (int i = tid; i < kVpN * kVpK; i += kNT) {
      const int r = i / kVpK, c = i % kVpK;
      bs[r][c] = (n0 + r < a.dim && k0 + c < a.k) ? a.pe[(size_t)(n0 + r) * a.k + k0 + c]
                                                   : 0.0f;
    }
    lds_barrier();
#pragma unroll 4
    for (int c = 0; c < kVpK; ++c) {
      const double x0 = as[2 * tm][c], x1 = as[2 * tm + 1][c];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double w = bs[tn + 16 * j][c];
        acc[0][j] = fma(x0, w, acc[0][j]);
        acc[1][j] = fma(x1, w, acc[1][j]);
      }
    }
    lds_barrier();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = m0 + 2 * tm + i;
    if (p >= a.m) continue;
    const float scale = a.pos_s[p];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int oc = n0 + tn + 16 * j;
      if (oc >= a.dim) continue;
      const float e = clamp_f32((float)(acc[i][j] + (double)a.pe_b[oc]));
      const float pos = (float)a.pos_q[(size_t)p * a.dim + oc] * scale;
      a.x[(size_t)p * a.dim + oc] = clamp_f32(e + pos);
    }
  }
}

// One workgroup per row.  With y: x[r] = clamp((y[r] + bias) + x[r]) (the
// output bias and the residual, gemma.c:4575-4590, 4641-4656), stored back
// as the new residual.  Then LayerNorm (layernorm, gemma.c:2526-2549) in
// fp64: mean, variance about it, (x - mean) / sqrt(var + eps) * w + b,
// rounded once; the row is quantized into xq[r] / xs[r] (quantize_acts)
// when xq is given, else stored to h[r].
template <int NPT>
__global__ __launch_bounds__(kNT) void vis_ln_rows_kernel(VisLn a) {
  __shared__ double red[kWaves];
  __shared__ float redf[kWaves];
  const int tid = threadIdx.x, n4 = a.dim >> 2;
  const size_t r = blockIdx.x;
  float *xr = a.x + r * a.dim;
  v4f xv[NPT];
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * kNT;
    xv[j] = c < n4 ? reinterpret_cast<const v4f *>(xr)[c] : zero;
    if (a.y != nullptr && c < n4) {
      const v4f yv = reinterpret_cast<const v4f *>(a.y + r * a.dim)[c];
      const v4f bv = reinterpret_cast<const v4f *>(a.bias)[c];
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[j][e] = clamp_f32((yv[e] + bv[e]) + xv[j][e]);
      reinterpret_cast<v4f *>(xr)[c] = xv[j];
    }
  }
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) s += (double)xv[j][e];
  const double mean = block_sum<kNT>(s, red) / (double)a.dim;
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
    if (tid + j * kNT < n4)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double d = (double)xv[j][e] - mean;
        ss += d * d;
      }
  const double inv = 1.0 / sqrt(block_sum<kNT>(ss, red) / (double)a.dim + (double)a.eps);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * kNT;
    if (c >= n4) {
      xv[j] = zero;
      continue;
    }
    const v4f wv = reinterpret_cast<const v4f *>(a.w)[c];
    const v4f bv = reinterpret_cast<const v4f *>(a.b)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xv[j][e] = (float)(((double)xv[j][e] - mean) * inv * (double)wv[e] + (double)bv[e]);
      amax = fmaxf(amax, abs_daz(xv[j][e]));
    }
  }
  if (a.xq == nullptr) {
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      if (tid + j * kNT < n4) reinterpret_cast<v4f *>(a.h + r * a.dim)[tid + j * kNT] = xv[j];
    return;
  }
  amax = block_max<kNT>(amax, redf);
  const QuantParams qp = quant_params(amax);
  int8_t *row = a.xq + r * a.dim;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * kNT;
    if (c < n4)
      reinterpret_cast<uint32_t *>(row)[c] =
          pack4(quant_one(xv[j].x, qp.inv), quant_one(xv[j].y, qp.inv),
                quant_one(xv[j].z, qp.inv), quant_one(xv[j].w, qp.inv));
  }
  if (tid == 0) a.xs[r] = qp.scale;
}

// Full (non-causal) attention of every patch over every patch, per head
// (gemma.c:4533-4561): q, k and v are the GEMM outputs plus their biases
// (single fp32 additions, 4517-4526), scores q.k * scale with scale =
// 1 / sqrtf(hdim) in fp32, softmax over all patches, value sums -- on the
// fp64 matrix cores.  v_mfma_f64_16x16x4f64 takes A[16][4] as lane l ->
// A[l%16][l/16], B[4][16] as lane l -> B[l/16][l%16], and leaves D[16][16]
// as lane l, element r -> D[4r + l/16][l%16] (checked on this GPU).
//
// A workgroup is 4 waves x 16 patches of one head; each wave holds its 16
// query rows as fp64 A operands in registers for the whole kernel.  Per tile
// of 32 keys (K and V staged in LDS as fp32, biases added): two 16x16 score
// blocks (HD/4 MFMA steps each); an online softmax in fp64 on the score
// registers -- the 16 lanes of a DPP row hold one query row, so row maxima
// and sums are DPP reductions; the probabilities go through LDS (16 x 32 per
// wave) to become A operands; the output block O[16][16 * NB] is rescaled by
// exp(m_old - m_new) and accumulates P . V (8 MFMA steps per 16 dims).  Every
// sum is fp64; each output is rounded to fp32 once at the end.
constexpr int kVaKeys = 32;  // keys per tile

template <int HD>
__global__ __launch_bounds__(kNT) void vis_attn_kernel(VisAttn a) {
  static_assert(HD % 4 == 0 && HD <= 128, "head dim");
  constexpr int KS = HD / 4;              // MFMA steps of the scores
  constexpr int NB = (HD + 15) / 16;      // 16-wide output blocks
  constexpr int RK = HD + 1;              // K row in LDS (odd: the B reads spread)
  constexpr int RP = kVaKeys + 4;         // P row (doubles)
  __shared__ float kt[kVaKeys * RK];
  __shared__ float vt[kVaKeys * (16 * NB + 16)];
  __shared__ double pw[4][16 * RP];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.y;
  const int q0 = blockIdx.x * 64 + wave * 16;  // this wave's first query row
  const int col = lane & 15, grp = lane >> 4;  // A/B: row/col col, k grp; D: col, rows 4r+grp
  constexpr int VS = 16 * NB + 16;             // V row stride in LDS (floats)

  // q rows as A operands: qa[s] = Q[q0 + col][4 s + grp] + bq
  double qa[KS];
  {
    const int qr = q0 + col;
    const float *qrow = a.qkv + (size_t)qr * a.stride + h * HD;
    const float *bq = a.bias + h * HD;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qa[s] = qr < a.n ? (double)(qrow[4 * s + grp] + bq[4 * s + grp]) : 0.0;
  }
  typedef double v4d __attribute__((ext_vector_type(4)));
  v4d o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = v4d{0.0, 0.0, 0.0, 0.0};
  double run_m[4], run_l[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    run_m[r] = -DBL_MAX;
    run_l[r] = 0.0;
  }
  const float *bk = a.bias + a.dim + h * HD;
  const float *bv = a.bias + 2 * a.dim + h * HD;

  for (int t0 = 0; t0 < a.n; t0 += kVaKeys) {
    lds_barrier();  // the previous tile's K, V and P are no longer read
    for (int i = tid; i < kVaKeys * (HD / 4); i += kNT) {
      const int t = i / (HD / 4), c4 = i - t * (HD / 4);
      v4f kx = {0.f, 0.f, 0.f, 0.f}, vx = kx;
      if (t0 + t < a.n) {
        const v4f *row = reinterpret_cast<const v4f *>(a.qkv + (size_t)(t0 + t) * a.stride);
        kx = row[(a.dim + h * HD) / 4 + c4] + reinterpret_cast<const v4f *>(bk)[c4];
        vx = row[(2 * a.dim + h * HD) / 4 + c4] + reinterpret_cast<const v4f *>(bv)[c4];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) kt[t * RK + 4 * c4 + e] = kx[e];
      *reinterpret_cast<v4f *>(&vt[t * VS + 4 * c4]) = vx;
    }
    if (16 * NB > HD)  // zero the padding columns of V (read by the last output block)
      for (int i = tid; i < kVaKeys * (16 * NB - HD); i += kNT) {
        const int t = i / (16 * NB - HD), c = i - t * (16 * NB - HD);
        vt[t * VS + HD + c] = 0.0f;
      }
    lds_barrier();
    // scores: block b covers keys t0 + 16 b + col
    v4d sc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      sc[b] = v4d{0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sc[b] = __builtin_amdgcn_mfma_f64_16x16x4f64(
            qa[s], (double)kt[(16 * b + col) * RK + 4 * s + grp], sc[b], 0, 0, 0);
    }
    // online softmax on rows 4r + grp (the 16 lanes of this DPP row)
    double alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      double s0 = t0 + col < a.n ? sc[0][r] * (double)a.scale : -DBL_MAX;
      double s1 = t0 + 16 + col < a.n ? sc[1][r] * (double)a.scale : -DBL_MAX;
      double m = fmax(s0, s1);
      m = fmax(m, dpp_f64<kDppXor1>(m));
      m = fmax(m, dpp_f64<kDppXor2>(m));
      m = fmax(m, dpp_f64<kDppHalfMirror>(m));
      m = fmax(m, dpp_f64<kDppMirror>(m));
      const double m_new = fmax(run_m[r], m);
      const double p0 = s0 == -DBL_MAX ? 0.0 : exp(s0 - m_new);
      const double p1 = s1 == -DBL_MAX ? 0.0 : exp(s1 - m_new);
      double l = p0 + p1;
      l += dpp_f64<kDppXor1>(l);
      l += dpp_f64<kDppXor2>(l);
      l += dpp_f64<kDppHalfMirror>(l);
      l += dpp_f64<kDppMirror>(l);
      alpha[r] = exp(run_m[r] - m_new);
      run_l[r] = run_l[r] * alpha[r] + l;
      run_m[r] = m_new;
      pw[wave][(4 * r + grp) * RP + col] = p0;
      pw[wave][(4 * r + grp) * RP + 16 + col] = p1;
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[nb][r] *= alpha[r];
    lds_barrier();  // P is read back in the A layout
#pragma unroll
    for (int s = 0; s < kVaKeys / 4; ++s) {
      const double pa = pw[wave][col * RP + 4 * s + grp];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        o[nb] = __builtin_amdgcn_mfma_f64_16x16x4f64(
            pa, (double)vt[(4 * s + grp) * VS + 16 * nb + col], o[nb], 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int qr = q0 + 4 * r + grp;
    if (qr >= a.n) continue;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int d = 16 * nb + col;
      if (d < HD) a.out[(size_t)qr * a.dim + h * HD + d] = (float)(o[nb][r] / run_l[r]);
    }
  }
}

// One workgroup per row: (float)gelu_tanh(h + b1) (gemma.c:4600-4604 with
// gelu 4150-4172: the bias added in fp32, the GELU in fp64 rounded once),
// quantized into xq[r] / xs[r].
template <int NPT, int NT>
__global__ __launch_bounds__(NT) void vis_gelu_quant_kernel(const float *hbuf, const float *bias,
                                                            int mlp, int8_t *xq, float *xs) {
  __shared__ float redf[NT / 64];
  const int tid = threadIdx.x, n4 = mlp >> 2;
  const float *row = hbuf + (size_t)blockIdx.x * mlp;
  v4f out[NPT];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    const v4f hv = c < n4 ? reinterpret_cast<const v4f *>(row)[c] : zero;
    const v4f bv = c < n4 ? reinterpret_cast<const v4f *>(bias)[c] : zero;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[j][e] = (float)gelu_tanh((double)(hv[e] + bv[e]));
      amax = fmaxf(amax, abs_daz(out[j][e]));
    }
  }
  amax = block_max<NT>(amax, redf);
  const QuantParams qp = quant_params(amax);
  int8_t *dst = xq + (size_t)blockIdx.x * mlp;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
    if (c < n4)
      reinterpret_cast<uint32_t *>(dst)[c] =
          pack4(quant_one(out[j].x, qp.inv), quant_one(out[j].y, qp.inv),
                quant_one(out[j].z, qp.inv), quant_one(out[j].w, qp.inv));
  }
  if (tid == 0) xs[blockIdx.x] = qp.scale;
}

// One workgroup per image token: the mean of its ksize x ksize patches
// (AvgPool2d, gemma.c:4673-4694) in fp64 rounded once, the soft-embedding
// RMSNorm (4698-4704) and the row quantized for the projection.
template <int NPT>
__global__ __launch_bounds__(kNT) void vis_pool_kernel(VisPool a) {
  __shared__ double red[kWaves];
  __shared__ float redf[kWaves];
  const int tid = threadIdx.x, n4 = a.dim >> 2;
  const int side = a.ppi / a.ksize;
  const int oy = blockIdx.x / side, ox = blockIdx.x % side;
  v4f pv[NPT];
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * kNT;
    double sum[4] = {0.0, 0.0, 0.0, 0.0};
    if (c < n4)
      for (int ky = 0; ky < a.ksize; ++ky)
        for (int kx = 0; kx < a.ksize; ++kx) {
          const int p = (oy * a.ksize + ky) * a.ppi + ox * a.ksize + kx;
          const v4f x = reinterpret_cast<const v4f *>(a.h + (size_t)p * a.dim)[c];
#pragma unroll
          for (int e = 0; e < 4; ++e) sum[e] += (double)x[e];
        }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pv[j][e] = (float)(sum[e] / (double)(a.ksize * a.ksize));
      ss += (double)pv[j][e] * (double)pv[j][e];
    }
  }
  const double rms = rms_of(block_sum<kNT>(ss, red), a.dim, a.eps);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * kNT;
    if (c >= n4) continue;
    const v4f wv = reinterpret_cast<const v4f *>(a.w)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pv[j][e] = norm_one(pv[j][e], rms, wv[e]);
      amax = fmaxf(amax, abs_daz(pv[j][e]));
    }
  }
  amax = block_max<kNT>(amax, redf);
  const QuantParams qp = quant_params(amax);
  int8_t *row = a.xq + (size_t)blockIdx.x * a.dim;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * kNT;
    if (c < n4)
      reinterpret_cast<uint32_t *>(row)[c] =
          pack4(quant_one(pv[j].x, qp.inv), quant_one(pv[j].y, qp.inv),
                quant_one(pv[j].z, qp.inv), quant_one(pv[j].w, qp.inv));
  }
  if (tid == 0) a.xs[blockIdx.x] = qp.scale;
}

template <int C, int CMAX, class F>
hipError_t by_npt(int npt, F &&launch) {
  if (npt == C) return launch(std::integral_constant<int, C>{});
  if constexpr (C < CMAX) return by_npt<C + 1, CMAX>(npt, launch);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_vis_patch(const VisPatch &a, hipStream_t stream) {
  const dim3 grid((a.m + kVpM - 1) / kVpM, (a.dim + kVpN - 1) / kVpN);
  vis_patch_kernel<<<grid, kNT, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_vis_ln_rows(const VisLn &a, int n, hipStream_t stream) {
  return by_npt<1, kPfMaxNpt>((a.dim / 4 + kNT - 1) / kNT, [&](auto c) {
    vis_ln_rows_kernel<decltype(c)::value><<<n, kNT, 0, stream>>>(a);
    return hipGetLastError();
  });
}

hipError_t launch_vis_attention(const VisAttn &a, int hdim, hipStream_t stream) {
  const dim3 grid((a.n + 63) / 64, a.n_heads);
  switch (hdim) {
    case 16: vis_attn_kernel<16><<<grid, kNT, 0, stream>>>(a); break;
    case 32: vis_attn_kernel<32><<<grid, kNT, 0, stream>>>(a); break;
    case 64: vis_attn_kernel<64><<<grid, kNT, 0, stream>>>(a); break;
    case 72: vis_attn_kernel<72><<<grid, kNT, 0, stream>>>(a); break;
    case 128: vis_attn_kernel<128><<<grid, kNT, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_vis_gelu_quant(const float *h, const float *bias, int n, int mlp, int8_t *xq,
                                 float *xs, hipStream_t stream) {
  constexpr int NT = 1024;
  return by_npt<1, kPfMaxNpt>((mlp / 4 + NT - 1) / NT, [&](auto c) {
    vis_gelu_quant_kernel<decltype(c)::value, NT><<<n, NT, 0, stream>>>(h, bias, mlp, xq, xs);
    return hipGetLastError();
  });
}

hipError_t launch_vis_pool(const VisPool &a, int ntok, hipStream_t stream) {
  return by_npt<1, kPfMaxNpt>((a.dim / 4 + kNT - 1) / kNT, [&](auto c) {
    vis_pool_kernel<decltype(c)::value><<<ntok, kNT, 0, stream>>>(a);
    return hipGetLastError();
  });
}

}  // namespace gh
