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

#include <cstdlib>
#include <cstring>

#include "dec_common.h"

namespace gh {
namespace {

// One workgroup per row.  With y: x[r] = clamp((y[r] + bias) + x[r]) (the
// output bias and the residual, gemma.c:4575-4590, 4641-4656), stored back
// as the new residual.  Then LayerNorm (layernorm, gemma.c:2526-2549) in
// fp64: mean, variance about it, (x - mean) / sqrt(var + eps) * w + b,
// rounded once; the row is quantized into xq[r] / xs[r] (quantize_acts)
// when xq is given, else stored to h[r].
template <int NPT, int NT>
__global__ __launch_bounds__(NT) void vis_ln_rows_kernel(VisLn a) {
  __shared__ double red[NT / 64];
  __shared__ float redf[NT / 64];
  const int tid = threadIdx.x, n4 = a.dim >> 2;
  const size_t r = blockIdx.x;
  float *xr = a.x + r * a.dim;
  v4f xv[NPT];
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
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
  const double mean = block_sum<NT>(s, red) / (double)a.dim;
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
    if (tid + j * NT < n4)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double d = (double)xv[j][e] - mean;
        ss += d * d;
      }
  const double inv = 1.0 / sqrt(block_sum<NT>(ss, red) / (double)a.dim + (double)a.eps);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
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
      if (tid + j * NT < n4) reinterpret_cast<v4f *>(a.h + r * a.dim)[tid + j * NT] = xv[j];
    return;
  }
  amax = block_max<NT>(amax, redf);
  const QuantParams qp = quant_params(amax);
  int8_t *row = a.xq + r * a.dim;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
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
// The products are taken transposed, S^T = K . Q^T and O^T = V^T . P^T, so
// that a lane (query j = l%16, g = l/16) holds the scores of query j for the
// keys 4r + g of a 16-key block, which are exactly the P^T operand the value
// product wants: the probabilities never leave registers.  A workgroup is
// 4 waves x 16 queries of one head; the queries stay in registers as fp64
// operands (lane g holds dims [g HD/4, (g+1) HD/4) of its query).  Per tile of
// 32 keys: K and V (biases added, fp32) are staged in LDS -- V transposed,
// its keys permuted so that the 4 a lane needs for one MFMA step are
// adjacent -- then two 16-key score blocks, the softmax weights, and P . V
// into the fp64 output block O^T[16 NB][16].  K and V are held in LDS as
// fp64, converted once when staged.
//
// Softmax: p = exp(s - m) with m a running reference maximum per query.
// Shifting by any m gives the same softmax; m is moved up (to the exact row
// maximum seen so far, rescaling O and the sums by exp(m_old - m_new)) only
// when some score of the wave exceeds it by more than kVaSlack, which keeps
// every p <= e^kVaSlack and lets most tiles skip the row reductions.  The
// row sums are per-lane partials, added across the 4 lanes of a query at
// the end.  Every sum is fp64; each output is rounded to fp32 once.
constexpr int kVaKeys = 32;          // keys per tile
constexpr int kVaWaves = 8;          // waves (16 queries each) per workgroup
constexpr int kVbWaves = 16;         // ... of the split-bf16 kernel (head dims <= 72)
constexpr double kVaSlack = 64.0;    // e^64 * 3.4e38 * n keys stays far below DBL_MAX

template <int HD, int NW>
__global__ __launch_bounds__(NW * 64, 8 / NW) void vis_attn_kernel(VisAttn a) {
  constexpr int NT = NW * 64, QB = NW * 16;  // threads, queries per workgroup
  static_assert(HD % 8 == 0 && HD <= 128, "head dim");
  constexpr int KS = HD / 4;            // MFMA steps of a score block (dims per lane)
  constexpr int NB = (HD + 15) / 16;    // 16-dim output blocks
  constexpr int RK = HD + 2;            // K row in LDS (doubles)
  constexpr int VS = kVaKeys + 2;       // V^T row in LDS (doubles)
  constexpr int C4 = HD / 4;            // float4 per key row
  constexpr int PF = (kVaKeys * C4 + NT - 1) / NT;  // float4 of K (and of V) per thread
  __shared__ double kt[kVaKeys * RK];
  __shared__ double vt[16 * NB * VS];
  __shared__ double etab[128];
  __shared__ v4f kvb[2][C4];  // the k and v biases of this head
  typedef double v2d __attribute__((ext_vector_type(2)));
  typedef double v4d __attribute__((ext_vector_type(4)));

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // blocks of one head share K and V: give each XCD (blocks b, b+8, ...) a
  // contiguous run of (head, query block) pairs so they meet in its L2
  const int nqb = (a.n + QB - 1) / QB, nblk = nqb * a.n_heads;
  int blk = blockIdx.x;
  if (nblk % 8 == 0) blk = (blk % 8) * (nblk / 8) + blk / 8;
  const int h = blk / nqb;
  const int q0 = (blk - h * nqb) * QB + wave * 16;
  const int col = lane & 15, grp = lane >> 4;

  double qa[KS];
  {
    const int qr = min(q0 + col, a.n - 1);
    const float *qrow = a.qkv + (size_t)qr * a.stride + h * HD + grp * KS;
    const float *bq = a.bias + h * HD + grp * KS;
#pragma unroll
    for (int s = 0; s < KS; ++s) qa[s] = (double)(qrow[s] + bq[s]);
  }
  v4d o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = v4d{0.0, 0.0, 0.0, 0.0};
  double m_ref = -DBL_MAX, l_part = 0.0;
  const double scale = (double)a.scale;
  const float *bk = a.bias + a.dim + h * HD;
  const float *bv = a.bias + 2 * a.dim + h * HD;
  const float *kbase = a.qkv + a.dim + h * HD;
  const float *vbase = a.qkv + 2 * a.dim + h * HD;

  // padding dims of V^T (never overwritten by the staging below)
  for (int i = HD * VS + tid; i < 16 * NB * VS; i += NT) vt[i] = 0.0;
  exp_tab_load(etab);
  for (int i = tid; i < 2 * C4; i += NT)
    kvb[i / C4][i % C4] = reinterpret_cast<const v4f *>(i < C4 ? bk : bv)[i % C4];
  const ExpConsts ec = exp_consts();

  v4f kx[PF], vx[PF];
  auto fetch = [&](int t0) {  // rows clamped into range: every load is unconditional
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = min(tid + j * NT, kVaKeys * C4 - 1);
      const int t = i / C4, c4 = i - t * C4;
      const size_t row = (size_t)min(t0 + t, a.n - 1) * a.stride;
      kx[j] = *reinterpret_cast<const v4f *>(kbase + row + 4 * c4);
      vx[j] = *reinterpret_cast<const v4f *>(vbase + row + 4 * c4);
    }
  };
  fetch(0);
  for (int t0 = 0; t0 < a.n; t0 += kVaKeys) {
    lds_barrier();  // every wave is done with the previous tile
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = tid + j * NT;
      if (i >= kVaKeys * C4) break;
      const int t = i / C4, c4 = i - t * C4;
      const bool ok = t0 + t < a.n;
      const v4f zero = {0.f, 0.f, 0.f, 0.f};
      const v4f kv = ok ? kx[j] + kvb[0][c4] : zero;
      const v4f vv = ok ? vx[j] + kvb[1][c4] : zero;
      *reinterpret_cast<v2d *>(&kt[t * RK + 4 * c4]) = v2d{(double)kv[0], (double)kv[1]};
      *reinterpret_cast<v2d *>(&kt[t * RK + 4 * c4 + 2]) = v2d{(double)kv[2], (double)kv[3]};
      const int tp = (t & 16) | ((t & 3) << 2) | ((t >> 2) & 3);  // key 16b+4s+g -> 16b+4g+s
#pragma unroll
      for (int e = 0; e < 4; ++e) vt[(4 * c4 + e) * VS + tp] = (double)vv[e];
    }
    lds_barrier();
    if (t0 + kVaKeys < a.n) fetch(t0 + kVaKeys);

    // scores: sc[b][r] = q(col) . k(t0 + 16 b + 4 r + grp)
    v4d sc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      sc[b] = v4d{0.0, 0.0, 0.0, 0.0};
      const double *kr = &kt[(16 * b + col) * RK + grp * KS];
#pragma unroll
      for (int s = 0; s < KS; s += 2) {
        const v2d k2 = *reinterpret_cast<const v2d *>(kr + s);
        sc[b] = __builtin_amdgcn_mfma_f64_16x16x4f64(k2[0], qa[s], sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f64_16x16x4f64(k2[1], qa[s + 1], sc[b], 0, 0, 0);
      }
    }
    double tmax = -DBL_MAX;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = t0 + 16 * b + 4 * r + grp < a.n;
        sc[b][r] = ok ? sc[b][r] * scale : -DBL_MAX;
        tmax = fmax(tmax, sc[b][r]);
      }
    if (__any(tmax > m_ref + kVaSlack)) {
      double rmax = fmax(tmax, __shfl_xor(tmax, 16, 64));
      rmax = fmax(rmax, __shfl_xor(rmax, 32, 64));
      const double m_new = fmax(m_ref, rmax);
      const double alpha = exp_tab(m_ref - m_new, etab, ec);
      m_ref = m_new;
      l_part *= alpha;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) o[nb] *= alpha;
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // a masked key (-DBL_MAX) lands on exp_tab's clamp and gives 0
        const double pr = exp_tab(sc[b][r] - m_ref, etab, ec);
        l_part += pr;
        sc[b][r] = pr;
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const double *vr = &vt[(16 * nb + col) * VS + 16 * b + 4 * grp];
        const v2d v01 = *reinterpret_cast<const v2d *>(vr);
        const v2d v23 = *reinterpret_cast<const v2d *>(vr + 2);
        o[nb] = __builtin_amdgcn_mfma_f64_16x16x4f64(v01[0], sc[b][0], o[nb], 0, 0, 0);
        o[nb] = __builtin_amdgcn_mfma_f64_16x16x4f64(v01[1], sc[b][1], o[nb], 0, 0, 0);
        o[nb] = __builtin_amdgcn_mfma_f64_16x16x4f64(v23[0], sc[b][2], o[nb], 0, 0, 0);
        o[nb] = __builtin_amdgcn_mfma_f64_16x16x4f64(v23[1], sc[b][3], o[nb], 0, 0, 0);
      }
    }
  }
  double l = l_part + __shfl_xor(l_part, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  const int qr = q0 + col;
  if (qr < a.n) {
    float *orow = a.out + (size_t)qr * a.dim + h * HD;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * nb + 4 * r + grp;
        if (d < HD) orow[d] = (float)(o[nb][r] / l);
      }
  }
}

// The same attention on the fp32 matrix cores (v_mfma_f32_16x16x4f32, twice
// the fp64 rate): q, k, v, scores, weights and value sums in fp32, as the
// reference computes them (gemm_fpx, softmax, gemm_fpx_nn), in a different
// order, so the result agrees with the fp64 form to fp32 rounding rather
// than bit for bit.  The fp32 MFMA takes A and B as the fp64 one does but
// leaves D as lane l, element r -> D[4 (l/16) + r][l%16] (checked on this
// GPU), so a lane (query col, g = l/16) holds the scores of keys 4g + r of a
// 16-key block, and the value product's MFMA step r takes keys 4g + r from
// lane group g: V^T stays in natural key order and a lane reads its four
// keys as one float4.  The reference maximum moves when a score exceeds it
// by more than 16 (e^16 * n keys * |v| stays far below FLT_MAX).  The
// exponential is __expf (v_exp_f32 on x log2 e: a relative error near
// |x| 2^-24 for the arguments here, |x| <= 16 past the masked keys), and two
// workgroups share a CU (113 registers at head dim 72): 880 -> 785 us per
// SigLIP layer against expf at one workgroup per CU.
constexpr float kVaSlackF = 16.0f;
constexpr int kVaKeysF = 32;  // keys per tile (fp32 kernel; 64 measured 2% slower)

template <int HD, int NW, int TK>
__global__ __launch_bounds__(NW * 64, 16 / NW) void vis_attn_f32_kernel(VisAttn a) {
  constexpr int NS = TK / 16;         // 16-key score blocks per tile
  constexpr int NT = NW * 64, QB = NW * 16;
  static_assert(HD % 8 == 0 && HD <= 128, "head dim");
  constexpr int KS = HD / 4;          // MFMA steps of a score block (dims per lane)
  constexpr int NB = (HD + 15) / 16;  // 16-dim output blocks
  constexpr int RK = HD + 2;          // K row in LDS (floats)
  constexpr int VS = TK + 4;     // V^T row in LDS (floats)
  constexpr int C4 = HD / 4;
  constexpr int PF = (TK * C4 + NT - 1) / NT;
  __shared__ float kt[TK * RK];
  __shared__ float vt[16 * NB * VS];
  __shared__ v4f kvb[2][C4];
  typedef float v2f __attribute__((ext_vector_type(2)));

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nqb = (a.n + QB - 1) / QB, nblk = nqb * a.n_heads;
  int blk = blockIdx.x;
  if (nblk % 8 == 0) blk = (blk % 8) * (nblk / 8) + blk / 8;
  const int h = blk / nqb;
  const int q0 = (blk - h * nqb) * QB + wave * 16;
  const int col = lane & 15, grp = lane >> 4;

  float qa[KS];
  {
    const int qr = min(q0 + col, a.n - 1);
    const float *qrow = a.qkv + (size_t)qr * a.stride + h * HD + grp * KS;
    const float *bq = a.bias + h * HD + grp * KS;
#pragma unroll
    for (int s = 0; s < KS; ++s) qa[s] = qrow[s] + bq[s];
  }
  v4f o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_ref = -FLT_MAX, l_part = 0.0f;
  const float *bk = a.bias + a.dim + h * HD;
  const float *bv = a.bias + 2 * a.dim + h * HD;
  const float *kbase = a.qkv + a.dim + h * HD;
  const float *vbase = a.qkv + 2 * a.dim + h * HD;

  for (int i = HD * VS + tid; i < 16 * NB * VS; i += NT) vt[i] = 0.0f;  // padding dims
  for (int i = tid; i < 2 * C4; i += NT)
    kvb[i / C4][i % C4] = reinterpret_cast<const v4f *>(i < C4 ? bk : bv)[i % C4];

  // K: float4 i of the tile is key i / C4, dims 4 (i % C4) .. +3.  V goes
  // to LDS transposed in blocks of 4 keys x 4 dims: block b = (tq, c4) =
  // (b % 8, b / 8) holds keys 4 tq .. 4 tq + 3 of dims 4 c4 .. 4 c4 + 3 and
  // is written as 4 float4 of V^T; eight consecutive lanes differ in tq, so
  // with the row pitch VS = TK + 4 their 16-byte writes fall in eight
  // different bank groups (scattering single floats instead put a
  // half-wave's writes on two banks).
  static_assert(TK % 4 == 0 && TK / 4 == 8, "V blocks: 8 key quads per tile");
  constexpr int VB = 8 * C4;               // V blocks per tile
  constexpr int PV = (VB + NT - 1) / NT;   // V blocks per thread
  v4f kx[PF], vx[PV][4];
  auto fetch = [&](int t0) {  // rows clamped into range: every load is unconditional
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = min(tid + j * NT, TK * C4 - 1);
      const int t = i / C4, c4 = i - t * C4;
      kx[j] = *reinterpret_cast<const v4f *>(kbase + (size_t)min(t0 + t, a.n - 1) * a.stride +
                                             4 * c4);
    }
#pragma unroll
    for (int j = 0; j < PV; ++j) {
      const int b = min(tid + j * NT, VB - 1);
      const int tq = b % 8, c4 = b / 8;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        vx[j][u] = *reinterpret_cast<const v4f *>(
            vbase + (size_t)min(t0 + 4 * tq + u, a.n - 1) * a.stride + 4 * c4);
    }
  };
  fetch(0);
  for (int t0 = 0; t0 < a.n; t0 += TK) {
    lds_barrier();  // every wave is done with the previous tile
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = tid + j * NT;
      if (i >= TK * C4) break;
      const int t = i / C4, c4 = i - t * C4;
      const v4f kv = t0 + t < a.n ? kx[j] + kvb[0][c4] : zero;
      *reinterpret_cast<v2f *>(&kt[t * RK + 4 * c4]) = v2f{kv[0], kv[1]};
      *reinterpret_cast<v2f *>(&kt[t * RK + 4 * c4 + 2]) = v2f{kv[2], kv[3]};
    }
#pragma unroll
    for (int j = 0; j < PV; ++j) {
      const int b = tid + j * NT;
      if (b >= VB) break;
      const int tq = b % 8, c4 = b / 8;
      v4f r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = t0 + 4 * tq + u < a.n ? vx[j][u] + kvb[1][c4] : zero;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<v4f *>(&vt[(4 * c4 + e) * VS + 4 * tq]) =
            v4f{r[0][e], r[1][e], r[2][e], r[3][e]};
    }
    lds_barrier();
    if (t0 + TK < a.n) fetch(t0 + TK);

    // scores: sc[b][r] = q(col) . k(t0 + 16 b + 4 grp + r)
    v4f sc[NS];
#pragma unroll
    for (int b = 0; b < NS; ++b) {
      sc[b] = v4f{0.f, 0.f, 0.f, 0.f};
      const float *kr = &kt[(16 * b + col) * RK + grp * KS];
#pragma unroll
      for (int s = 0; s < KS; s += 2) {
        const v2f k2 = *reinterpret_cast<const v2f *>(kr + s);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(k2[0], qa[s], sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(k2[1], qa[s + 1], sc[b], 0, 0, 0);
      }
    }
    float tmax = -FLT_MAX;
#pragma unroll
    for (int b = 0; b < NS; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = t0 + 16 * b + 4 * grp + r < a.n;
        sc[b][r] = ok ? sc[b][r] * a.scale : -FLT_MAX;
        tmax = fmaxf(tmax, sc[b][r]);
      }
    if (__any(tmax > m_ref + kVaSlackF)) {
      float rmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
      const float m_new = fmaxf(m_ref, rmax);
      const float alpha = __expf(m_ref - m_new);
      m_ref = m_new;
      l_part *= alpha;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) o[nb] *= alpha;
    }
#pragma unroll
    for (int b = 0; b < NS; ++b) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = sc[b][r] > -FLT_MAX ? __expf(sc[b][r] - m_ref) : 0.0f;
        l_part += pr;
        sc[b][r] = pr;
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const v4f v4 = *reinterpret_cast<const v4f *>(&vt[(16 * nb + col) * VS + 16 * b + 4 * grp]);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[r], sc[b][r], o[nb], 0, 0, 0);
      }
    }
  }
  float l = l_part + __shfl_xor(l_part, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  const int qr = q0 + col;
  if (qr < a.n) {
    float *orow = a.out + (size_t)qr * a.dim + h * HD;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * nb + 4 * grp + r;
        if (d < HD) orow[d] = o[nb][r] / l;
      }
  }
}

// One workgroup per row: (float)gelu_tanh(h + b1) (gemma.c:4600-4604 with
// gelu 4150-4172: the bias added in fp32, the GELU in fp64 rounded once),
// quantized into xq[r] / xs[r].
template <int NPT, int NT>
__global__ __launch_bounds__(NT) void vis_gelu_quant_kernel(const float *hbuf, const float *bias,
                                                            int mlp, int8_t *xq, float *xs,
                                                            WarmRegions warm) {
  __shared__ float redf[NT / 64];
  __shared__ double etab[128];
  exp_tab_load(etab);
  const ExpConsts ec = exp_consts();
  const int tid = threadIdx.x, n4 = mlp >> 2;
  const float *row = hbuf + (size_t)blockIdx.x * mlp;
  v4f hv[NPT], bv[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    hv[j] = c < n4 ? reinterpret_cast<const v4f *>(row)[c] : zero;
    bv[j] = c < n4 ? reinterpret_cast<const v4f *>(bias)[c] : zero;
  }
  lds_barrier();  // the exp table
  v4f out[NPT];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[j][e] = (float)gelu((double)(hv[j][e] + bv[j][e]), etab, ec);
      amax = fmaxf(amax, abs_daz(out[j][e]));
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
  warm_share(warm, blockIdx.x, gridDim.x, tid, NT);
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
  if (a.xq == nullptr) {  // fp32 rows for an fp32 projection
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int c = tid + j * kNT;
      if (c < n4) reinterpret_cast<v4f *>(a.out + (size_t)blockIdx.x * a.dim)[c] = pv[j];
    }
    return;
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

// h = gelu(h + bias) in place, grid (ceil(mlp / 4 / kNT), rows): the fp32
// tower's fc1 epilogue (gemma.c:4620-4622), each value as the quantizing
// kernel computes it.
__global__ __launch_bounds__(kNT) void vis_bias_gelu_kernel(float *h, const float *bias, int mlp) {
  __shared__ double etab[128];
  exp_tab_load(etab);
  const ExpConsts ec = exp_consts();
  const int c = blockIdx.x * kNT + threadIdx.x;
  float *row = h + (size_t)blockIdx.y * mlp;
  const bool ok = c < mlp / 4;
  v4f hv = {0.f, 0.f, 0.f, 0.f}, bv = hv;
  if (ok) {
    hv = reinterpret_cast<const v4f *>(row)[c];
    bv = reinterpret_cast<const v4f *>(bias)[c];
  }
  lds_barrier();  // the exp table
  if (!ok) return;
  v4f out;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = (float)gelu((double)(hv[e] + bv[e]), etab, ec);
  reinterpret_cast<v4f *>(row)[c] = out;
}

template <int C, int CMAX, class F>
hipError_t by_npt(int npt, F &&launch) {
  if (npt == C) return launch(std::integral_constant<int, C>{});
  if constexpr (C < CMAX) return by_npt<C + 1, CMAX>(npt, launch);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_vis_ln_rows(const VisLn &a, int n, hipStream_t stream) {
  // the fewest threads per row that cover it in kPfMaxNpt chunks: more rows
  // in flight per CU (SigLIP's 1152 columns: one wave, 5 chunks)
  const int n4 = a.dim / 4;
  auto go = [&](auto nt) {
    constexpr int NT = decltype(nt)::value;
    return by_npt<1, kPfMaxNpt>((n4 + NT - 1) / NT, [&](auto c) {
      vis_ln_rows_kernel<decltype(c)::value, NT><<<n, NT, 0, stream>>>(a);
      return hipGetLastError();
    });
  };
  if ((n4 + 63) / 64 <= kPfMaxNpt) return go(std::integral_constant<int, 64>{});
  if ((n4 + 127) / 128 <= kPfMaxNpt) return go(std::integral_constant<int, 128>{});
  return go(std::integral_constant<int, 256>{});
}

// The fp32 mode's attention on the bf16 matrix cores: every fp32 operand x
// of the two products (q, k, the probabilities p and v) is split into three
// bf16 pieces x = x0 + x1 + x2 (each rounded to nearest from the remainder,
// so together they hold x's 24 significant bits), and each product a.b is
// summed from the six piece products whose orders add up to at most 2
// (a0 b0, a0 b1, a1 b0, a0 b2, a1 b1, a2 b0): the dropped ones are below
// 3 * 2^-24 |a b|, fp32 rounding.  bf16 x bf16 products are exact in the
// fp32 accumulators.  v_mfma_f32_16x16x32_bf16 (lane l: A[l%16][8(l/16) ..
// +7], B[8(l/16) .. +7][l%16], D[4(l/16) + r][l%16], checked on the GPU)
// runs 14x the fp32 MFMA's rate here, so the six cost ~0.4 of one fp32 MFMA
// step.  Geometry as vis_attn_f32_kernel: NW waves x 16 queries of one head,
// 32-key tiles.  The next tile's fp32 K and V rows go by LDS DMA into a
// staging buffer while the current tile's planes are in use; at a tile's
// start the staged rows get their bias and are split into the planes (once
// per workgroup, not per wave; with no prefetch registers the kernel fits
// two workgroups per CU at head dim 72).  Scores per 16-key
// block b: S[key 16b + 4g + r][query col] over 32-dim chunks of the head dim
// (padded with zeros to CH * 32); K in LDS as three bf16 planes [key][dim].
// Values: the PV product's k index is 8g + 4b + r, the key 16b + 4g + r,
// so a lane's own eight probabilities are its B operand as they stand; V^T
// is staged in LDS as three bf16 planes [dim][k] in that key order.
// One LDS DMA load: every lane's 16 bytes at g land at lds + 16 * lane (lds
// wave-uniform); from inline asm so that the compiler does not wait for the
// pending load before later LDS reads (the kernel waits itself).  m0 has no
// other user in the kernel that calls this.
__device__ __forceinline__ void vis_dma16(const float *g, void *lds) {
  const uint32_t m = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m), "v"(g)
               : "memory", "m0");
#pragma clang diagnostic pop
}

template <int HD, int NW>
__global__ __launch_bounds__(NW * 64, 16 / NW) void vis_attn_bf3_kernel(VisAttn a) {
  constexpr int TK = 32;              // keys per tile
  constexpr int CH = (HD + 31) / 32;  // 32-dim chunks of the score product
  constexpr int DP = CH * 32;         // padded head dim of the K planes
  // A last chunk of 8 dims (head dim 72) takes two MFMAs instead of six: its
  // k index carries four piece products over the 8 dims, k = 8 g + e for
  // dim 32 CF + e of piece pair g (first MFMA: k2 q0, k1 q1, k0 q2, k1 q0;
  // second: k0 q1, k0 q0 and two zero pairs)
  constexpr bool kTail8 = HD % 32 == 8;
  constexpr int CF = kTail8 ? CH - 1 : CH;  // chunks summed piece by piece
  constexpr int NB = (HD + 15) / 16;  // 16-dim output blocks
  constexpr int RK = DP + 8;          // K plane row (bf16): 16 rows in distinct banks
  constexpr int RV = TK + 8;          // V^T plane row (bf16)
  constexpr int NT = NW * 64, QB = NW * 16;
  constexpr int C4 = HD / 4;
  constexpr int PF = (TK * C4 + NT - 1) / NT;  // K float4 per thread
  static_assert(HD % 8 == 0 && HD <= 128, "head dim");
  // planes 16 bytes apart in the banks: the first tail MFMA reads three of
  // them at one offset
  __shared__ __attribute__((aligned(16))) __bf16 kt[3][TK * RK + 8];
  __shared__ __attribute__((aligned(16))) __bf16 vt[3][NB * 16 * RV];
  __shared__ v4f kvb[2][C4];
  // the next tile's fp32 K and V rows land here by LDS DMA, key-major [key][C4]
  constexpr int SG = TK * C4;
  __shared__ v4f stg[2][SG];
  static_assert(SG % 64 == 0, "whole DMA instructions per tile");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nqb = (a.n + QB - 1) / QB, nblk = nqb * a.n_heads;
  int blk = blockIdx.x;
  if (nblk % 8 == 0) blk = (blk % 8) * (nblk / 8) + blk / 8;
  const int h = blk / nqb;
  const int q0 = (blk - h * nqb) * QB + wave * 16;
  const int col = lane & 15, grp = lane >> 4;

  // the query's pieces: lane (col, g) holds dims 32 c + 8 g .. + 7
  bf8 qa[3][CH];
  {
    const int qr = min(q0 + col, a.n - 1);
    const float *qrow = a.qkv + (size_t)qr * a.stride + h * HD;
    const float *bq = a.bias + h * HD;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      u4 w0, w1, w2;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int d = 32 * c + 8 * grp + e;  // HD is even: d and d + 1 are both in or out
        const float x0 = d < HD ? qrow[d] + bq[d] : 0.0f;
        const float x1 = d < HD ? qrow[d + 1] + bq[d + 1] : 0.0f;
        const Bf3x2 sp = split3x2(x0, x1);
        w0[e / 2] = sp.q0;
        w1[e / 2] = sp.q1;
        w2[e / 2] = sp.q2;
      }
      qa[0][c] = as_bf8(w0);
      qa[1][c] = as_bf8(w1);
      qa[2][c] = as_bf8(w2);
    }
  }
  // the tail chunk's operands: lane (col, 0) holds dims 32 CF .. + 7 of
  // every piece in qa[p][CF]; lane (col, g) takes the piece of pair g
  bf8 qt1 = {}, qt2 = {};
  int tsel = 0;  // the K plane lane (col, g) reads in the first tail MFMA
  if constexpr (kTail8) {
    u4 t[3];
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const u4 v = __builtin_bit_cast(u4, qa[p][CF]);
#pragma unroll
      for (int d = 0; d < 4; ++d) t[p][d] = (uint32_t)__shfl((int)v[d], col, 64);
    }
    qt1 = as_bf8(grp == 1 ? t[1] : grp == 2 ? t[2] : t[0]);          // q0 q1 q2 q0
    qt2 = as_bf8(grp == 0 ? t[1] : grp == 1 ? t[0] : u4{0, 0, 0, 0});  // q1 q0 0 0
    tsel = grp == 0 ? 2 : grp == 2 ? 0 : 1;                            // k2 k1 k0 k1
  }
  v4f o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_ref = -FLT_MAX, l_part = 0.0f;
  const float *bk = a.bias + a.dim + h * HD;
  const float *bv = a.bias + 2 * a.dim + h * HD;
  const float *kbase = a.qkv + a.dim + h * HD;
  const float *vbase = a.qkv + 2 * a.dim + h * HD;

  // zero padding: K dims HD .. DP-1 and V^T rows HD .. 16 NB - 1, never staged
  const __bf16 bz = (__bf16)0.0f;
  for (int i = tid; i < 3 * TK * (DP - HD); i += NT) {
    const int p = i / (TK * (DP - HD)), j = i % (TK * (DP - HD));
    kt[p][(j / (DP - HD)) * RK + HD + j % (DP - HD)] = bz;
  }
  for (int i = tid; i < 3 * (16 * NB - HD) * RV; i += NT) {
    const int p = i / ((16 * NB - HD) * RV), j = i % ((16 * NB - HD) * RV);
    vt[p][HD * RV + j] = bz;
  }
  for (int i = tid; i < 2 * C4; i += NT)
    kvb[i / C4][i % C4] = reinterpret_cast<const v4f *>(i < C4 ? bk : bv)[i % C4];

  static_assert(TK / 4 == 8, "V blocks: 8 key quads per tile");
  constexpr int VB = 8 * C4;              // V blocks (4 keys x 4 dims) per tile
  constexpr int PV = (VB + NT - 1) / NT;  // V blocks per thread
  constexpr int NI = 2 * SG / 64;  // DMA instructions per tile (K, then V)
  auto fetch = [&](int t0) {  // rows clamped into range: every load is unconditional
    for (int i = wave; i < NI; i += NW) {  // wave-uniform
      const int kv = i / (SG / 64), ch = (i % (SG / 64)) * 64 + lane;
      const int t = ch / C4, c4 = ch - t * C4;
      vis_dma16((kv == 0 ? kbase : vbase) + (size_t)min(t0 + t, a.n - 1) * a.stride + 4 * c4,
                &stg[kv][(i % (SG / 64)) * 64]);
    }
  };
  fetch(0);
  for (int t0 = 0; t0 < a.n; t0 += TK) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's DMAs landed
    lds_barrier();  // every wave is done with the previous tile (and every DMA landed)
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = tid + j * NT;
      if (i >= TK * C4) break;
      const int t = i / C4, c4 = i - t * C4;
      const v4f kv = t0 + t < a.n ? stg[0][i] + kvb[0][c4] : zero;
      const Bf3x2 lo = split3x2(kv[0], kv[1]), hi = split3x2(kv[2], kv[3]);
      *reinterpret_cast<u2 *>(&kt[0][t * RK + 4 * c4]) = u2{lo.q0, hi.q0};
      *reinterpret_cast<u2 *>(&kt[1][t * RK + 4 * c4]) = u2{lo.q1, hi.q1};
      *reinterpret_cast<u2 *>(&kt[2][t * RK + 4 * c4]) = u2{lo.q2, hi.q2};
    }
#pragma unroll
    for (int j = 0; j < PV; ++j) {
      const int b = tid + j * NT;
      if (b >= VB) break;
      const int tq = b % 8, c4 = b / 8;
      const int k0i = 8 * (tq % 4) + 4 * (tq / 4);  // PV index of key 4 tq
      v4f r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        r[u] = t0 + 4 * tq + u < a.n ? stg[1][(4 * tq + u) * C4 + c4] + kvb[1][c4] : zero;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const Bf3x2 lo = split3x2(r[0][e], r[1][e]), hi = split3x2(r[2][e], r[3][e]);
        const int at = (4 * c4 + e) * RV + k0i;
        *reinterpret_cast<u2 *>(&vt[0][at]) = u2{lo.q0, hi.q0};
        *reinterpret_cast<u2 *>(&vt[1][at]) = u2{lo.q1, hi.q1};
        *reinterpret_cast<u2 *>(&vt[2][at]) = u2{lo.q2, hi.q2};
      }
    }
    lds_barrier();
    if (t0 + TK < a.n) fetch(t0 + TK);

    // scores: sc[b][r] = q(col) . k(t0 + 16 b + 4 grp + r), the small piece
    // products first
    v4f sc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      sc[b] = v4f{0.f, 0.f, 0.f, 0.f};
      if constexpr (kTail8) {
        const int at = (16 * b + col) * RK + 32 * CF;
        const bf8 a1 = *reinterpret_cast<const bf8 *>(&kt[tsel][at]);
        const bf8 a2 = *reinterpret_cast<const bf8 *>(&kt[0][at]);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qt1, sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, qt2, sc[b], 0, 0, 0);
      }
#pragma unroll
      for (int c = 0; c < CF; ++c) {
        const int at = (16 * b + col) * RK + 32 * c + 8 * grp;
        const bf8 k0 = *reinterpret_cast<const bf8 *>(&kt[0][at]);
        const bf8 k1 = *reinterpret_cast<const bf8 *>(&kt[1][at]);
        const bf8 k2 = *reinterpret_cast<const bf8 *>(&kt[2][at]);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k2, qa[0][c], sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qa[1][c], sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qa[2][c], sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qa[0][c], sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qa[1][c], sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qa[0][c], sc[b], 0, 0, 0);
      }
    }
    float tmax = -FLT_MAX;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = t0 + 16 * b + 4 * grp + r < a.n;
        sc[b][r] = ok ? sc[b][r] * a.scale : -FLT_MAX;
        tmax = fmaxf(tmax, sc[b][r]);
      }
    if (__any(tmax > m_ref + kVaSlackF)) {
      float rmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
      const float m_new = fmaxf(m_ref, rmax);
      const float alpha = __expf(m_ref - m_new);
      m_ref = m_new;
      l_part *= alpha;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) o[nb] *= alpha;
    }
    // probabilities, their pieces (k = 4 b + r of this lane's eight)
    u4 w0, w1, w2;  // weight k = 4 b + r of the lane's eight is dword 2 b + r / 2
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const float pa = sc[b][r] > -FLT_MAX ? __expf(sc[b][r] - m_ref) : 0.0f;
        const float pb = sc[b][r + 1] > -FLT_MAX ? __expf(sc[b][r + 1] - m_ref) : 0.0f;
        l_part += pa;
        l_part += pb;
        const Bf3x2 sp = split3x2(pa, pb);
        w0[2 * b + r / 2] = sp.q0;
        w1[2 * b + r / 2] = sp.q1;
        w2[2 * b + r / 2] = sp.q2;
      }
    const bf8 p0 = as_bf8(w0), p1 = as_bf8(w1), p2 = as_bf8(w2);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int at = (16 * nb + col) * RV + 8 * grp;
      const bf8 v0 = *reinterpret_cast<const bf8 *>(&vt[0][at]);
      const bf8 v1 = *reinterpret_cast<const bf8 *>(&vt[1][at]);
      const bf8 v2 = *reinterpret_cast<const bf8 *>(&vt[2][at]);
      o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v2, p0, o[nb], 0, 0, 0);
      o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v1, p1, o[nb], 0, 0, 0);
      o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, p2, o[nb], 0, 0, 0);
      o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v1, p0, o[nb], 0, 0, 0);
      o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, p1, o[nb], 0, 0, 0);
      o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, p0, o[nb], 0, 0, 0);
    }
  }
  float l = l_part + __shfl_xor(l_part, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  const int qr = q0 + col;
  if (qr < a.n) {
    float *orow = a.out + (size_t)qr * a.dim + h * HD;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * nb + 4 * grp + r;
        if (d < HD) orow[d] = o[nb][r] / l;
      }
  }
}

// The fp32 mode's kernel: the split bf16 one by default, the fp32-MFMA one
// with GEMMA_HIP_VIS_ATTN=f32.  Read at every launch (one getenv per layer),
// so that one process can time or check both.
bool vis_attn_split() {
  const char *e = getenv("GEMMA_HIP_VIS_ATTN");
  return e == nullptr || strcmp(e, "f32") != 0;
}

hipError_t launch_vis_attention(const VisAttn &a, int hdim, bool f32, hipStream_t stream) {
  constexpr int NW = kVaWaves;
  const dim3 grid((a.n + NW * 16 - 1) / (NW * 16) * a.n_heads);
  if (f32 && vis_attn_split()) {
    // 16-wave workgroups (256 queries share each staged and split tile):
    // SigLIP 896 px 19.24-19.39 -> 17.86-17.95 ms per image against 8 waves
    // (4 waves: 25.5); head dim 128 keeps 8, its registers exceed the 128 of
    // four waves per SIMD
    constexpr int W = kVbWaves;
    const dim3 gw((a.n + W * 16 - 1) / (W * 16) * a.n_heads);
    switch (hdim) {
      case 16: vis_attn_bf3_kernel<16, W><<<gw, W * 64, 0, stream>>>(a); break;
      case 32: vis_attn_bf3_kernel<32, W><<<gw, W * 64, 0, stream>>>(a); break;
      case 64: vis_attn_bf3_kernel<64, W><<<gw, W * 64, 0, stream>>>(a); break;
      case 72: vis_attn_bf3_kernel<72, W><<<gw, W * 64, 0, stream>>>(a); break;
      case 128: vis_attn_bf3_kernel<128, NW><<<grid, NW * 64, 0, stream>>>(a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (f32) {
    switch (hdim) {
      case 16: vis_attn_f32_kernel<16, NW, kVaKeysF><<<grid, NW * 64, 0, stream>>>(a); break;
      case 32: vis_attn_f32_kernel<32, NW, kVaKeysF><<<grid, NW * 64, 0, stream>>>(a); break;
      case 64: vis_attn_f32_kernel<64, NW, kVaKeysF><<<grid, NW * 64, 0, stream>>>(a); break;
      case 72: vis_attn_f32_kernel<72, NW, kVaKeysF><<<grid, NW * 64, 0, stream>>>(a); break;
      case 128: vis_attn_f32_kernel<128, NW, kVaKeysF><<<grid, NW * 64, 0, stream>>>(a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (hdim) {
    case 16: vis_attn_kernel<16, NW><<<grid, NW * 64, 0, stream>>>(a); break;
    case 32: vis_attn_kernel<32, NW><<<grid, NW * 64, 0, stream>>>(a); break;
    case 64: vis_attn_kernel<64, NW><<<grid, NW * 64, 0, stream>>>(a); break;
    case 72: vis_attn_kernel<72, NW><<<grid, NW * 64, 0, stream>>>(a); break;
    case 128: vis_attn_kernel<128, NW><<<grid, NW * 64, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_vis_gelu_quant(const float *h, const float *bias, int n, int mlp, int8_t *xq,
                                 float *xs, const WarmRegions &warm, hipStream_t stream) {
  // the fewest threads per row that cover it in kPfMaxNpt chunks: at SigLIP's
  // 4304 columns, 256 threads leave 16% of the slots empty, 1024 threads 47%
  // (54.7 -> 36.7 us per layer measured)
  const int n4 = mlp / 4;
  auto go = [&](auto nt) {
    constexpr int NT = decltype(nt)::value;
    return by_npt<1, kPfMaxNpt>((n4 + NT - 1) / NT, [&](auto c) {
      vis_gelu_quant_kernel<decltype(c)::value, NT><<<n, NT, 0, stream>>>(h, bias, mlp, xq, xs,
                                                                             warm);
      return hipGetLastError();
    });
  };
  if ((n4 + 255) / 256 <= kPfMaxNpt) return go(std::integral_constant<int, 256>{});
  if ((n4 + 511) / 512 <= kPfMaxNpt) return go(std::integral_constant<int, 512>{});
  return go(std::integral_constant<int, 1024>{});
}

hipError_t launch_vis_bias_gelu(float *h, const float *bias, int n, int mlp, hipStream_t stream) {
  if (n <= 0 || mlp <= 0 || mlp % 4 != 0) return hipErrorInvalidValue;
  vis_bias_gelu_kernel<<<dim3((mlp / 4 + kNT - 1) / kNT, n), kNT, 0, stream>>>(h, bias, mlp);
  return hipGetLastError();
}

hipError_t launch_vis_pool(const VisPool &a, int ntok, hipStream_t stream) {
  return by_npt<1, kPfMaxNpt>((a.dim / 4 + kNT - 1) / kNT, [&](auto c) {
    vis_pool_kernel<decltype(c)::value><<<ntok, kNT, 0, stream>>>(a);
    return hipGetLastError();
  });
}

}  // namespace gh
