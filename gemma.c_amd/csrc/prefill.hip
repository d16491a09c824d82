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
//                    the cache, query rows in tiles that share K/V tiles; or
//                    dense: every row over the whole cache up to the last row
//                    (the image tokens' bidirectional attention)
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
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <vector>

#include "dec_common.h"

namespace gh {
namespace {

// x[r] = emb_q[tokens[r]] * (esc * emb_s[tokens[r]]) (gemma.c:5468-5493,
// per token); the host range-checks every token
__global__ __launch_bounds__(kNT) void pf_embed_kernel(const int *tokens, const int8_t *emb_q,
                                                       const float *emb_s, const float *emb_f,
                                                       float *x, int dim, float esc) {
  const int token = tokens[blockIdx.x];
  float *xr = x + (size_t)blockIdx.x * dim;
  if (emb_f != nullptr) {
    const float *row = emb_f + (size_t)token * dim;
    for (int i = threadIdx.x; i < dim; i += kNT) xr[i] = row[i] * esc;
    return;
  }
  const float s = esc * emb_s[token];
  const int8_t *row = emb_q + (size_t)token * dim;
  for (int i = threadIdx.x; i < dim; i += kNT) xr[i] = (float)row[i] * s;
}

// One workgroup per row: x[r] = clamp(x[r] + post(y[r])), h = rmsnorm(x[r],
// w_pre), h quantized into xq[r] / xs[r] (quantize_acts, gemma.c:2652-2674),
// or stored to h[r] when xq is null.
template <int NPT>
__global__ __launch_bounds__(kNT) void pf_norm_rows_kernel(PfNorm a) {
  __shared__ double red[kWaves];
  __shared__ float redf[kWaves];
  const size_t r = blockIdx.x;
  float *xr = a.x + r * a.dim;
  const bool quant = a.xq != nullptr;
  const DecNorm na{xr, a.y != nullptr ? a.y + r * a.dim : nullptr, a.w_post, a.w_pre, xr,
                   quant ? nullptr : a.h + r * a.dim, a.dim, a.eps};
  NormIn<NPT> in;
  norm_load<NPT, kNT>(na, in);
  const float s = norm_quant<NPT, kNT, true>(na, in, quant ? a.xq + r * a.dim : nullptr, red,
                                             redf);
  if (quant && threadIdx.x == 0) a.xs[r] = s;
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

// Causal attention of the prompt rows (gemma.c:5152-5293) on the fp64
// matrix cores, in the form of the vision tower's attention (vision.hip):
// v_mfma_f64_16x16x4f64 (lane l: A[l%16][l/16], B[l/16][l%16], result r ->
// D[4r + l/16][l%16]) on the transposed products S^T = K . Q^T and
// O^T = V^T . P^T, so the probabilities a lane computes (query l%16, keys
// 4r + l/16 of a 16-key block) are the operand of the value product as they
// stand.
//
// A workgroup is one kv head and 64 query vectors -- its hn q heads at
// qb = 64 / hn consecutive rows -- as 4 waves x 16; each wave holds its
// queries as fp64 operands (lane l/16 holds dims [l/16 HD/4, (l/16+1) HD/4)).
// It walks the cached keys from the first row's window start to the last
// row's position in tiles of 32, staged in LDS (fp32; V transposed with each
// 16-key block's keys permuted so that one MFMA step's 4 values are
// adjacent) with the next tile's loads in flight during the current one.  A
// wave skips the tiles that lie wholly outside its own rows' windows;
// per key the mask is the reference's: key <= position and, on sliding
// layers, key > position - window.  Scores are scaled (and soft-capped) in
// fp64; the softmax shifts by a per-query reference maximum that only moves,
// rescaling O and the partial sums by exp(m_old - m_new), when a score
// exceeds it by more than kPaSlack (the softmax is shift-invariant).  The
// reference maximum starts at kPaFloor, far below any score and far above
// -DBL_MAX, so a masked score (-DBL_MAX) gives exp = 0 even before a query
// has seen its first key.  Every sum is fp64; each output is rounded to
// fp32 once.
constexpr int kPaQ = 64;              // query vectors per workgroup (head dim 128)
constexpr int kPaPairWaves = 8;       // waves per workgroup (head dim 256): 4 pairs
constexpr int kPaQPair = kPaPairWaves * 8;  // query vectors per workgroup (16 per pair)
constexpr int kPaKeys = 32;           // keys per tile (register-staged kernel)
constexpr double kPaSlack = 64.0;     // p <= e^64: sums stay far below DBL_MAX
constexpr double kPaFloor = -1e300;   // |score| <= 256 * FLT_MAX^2 << 1e300
typedef double v4d __attribute__((ext_vector_type(4)));

// What a lane of a prefill attention workgroup works on: the block's
// (kv head, row block, key chunk) and the lane's query vector.
struct PaLane {
  int hk, r0, rows, chunk_id, nchunks, k_lo, k_end;  // block
  int row, head, p_abs, ws, p_top;                    // lane
  bool valid;
  int w_lo, w_hi;  // the keys any query of the wave can see
  bool empty;      // no chunk for this block
};

__host__ __device__ __forceinline__ int pa_window_start(const PfAttn &a, int p_abs) {
  return (!a.dense && a.slide > 0 && p_abs >= a.slide) ? p_abs + 1 - a.slide : 0;
}

// The keys rows r0 .. r0+rows-1 read: from the first row's window start,
// rounded down to a key tile, to the last row's position -- or, dense, every
// key 0 .. pos0+n-1 for every row.
struct PaRange {
  int k_base, p_last;
};
__host__ __device__ __forceinline__ PaRange pa_range(const PfAttn &a, int r0, int rows) {
  const int p_last = a.dense ? a.pos0 + a.n - 1 : a.pos0 + r0 + rows - 1;
  return {pa_window_start(a, a.pos0 + r0) / kPaKeys * kPaKeys, p_last};
}

// block = ((row block from the last) * nsplit + c) * nkv + kv head: the
// longest rows first, and with nkv dividing 8 each XCD (blocks b, b+8, ...)
// sees one kv head.  When nkv * nsplit is a multiple of 8, the chunk is c
// rotated by the row block's index: an XCD would otherwise see one chunk
// parity for every row block, and in causal layers the low chunks carry most
// of the work (measured, gemma-3-4b global layers at 2048 tokens: 683 ->
// 437 us).  A chunk is chunk_id's run of a.chunk keys of the row block's key
// range (its first row's window start, rounded down to 32, to its last row's
// position).
__device__ __forceinline__ PaLane pa_lane(const PfAttn &a, int wave, int col) {
  PaLane L;
  const int hn = a.n_heads / a.nkv, qb = a.qpb / hn;
  const int nrb = (a.n + qb - 1) / qb;
  L.hk = blockIdx.x % a.nkv;
  const int rot = (a.nkv * a.nsplit) % 8 == 0 ? blockIdx.x / a.nkv / a.nsplit : 0;
  L.chunk_id = ((blockIdx.x / a.nkv) % a.nsplit + rot) % a.nsplit;
  L.r0 = (nrb - 1 - blockIdx.x / a.nkv / a.nsplit) * qb;
  L.rows = min(qb, a.n - L.r0);
  const auto [k_base, p_last] = pa_range(a, L.r0, L.rows);
  L.nchunks = (p_last - k_base + a.chunk) / a.chunk;
  L.empty = L.chunk_id >= L.nchunks;
  L.k_lo = k_base + L.chunk_id * a.chunk;
  L.k_end = min(L.k_lo + a.chunk - 1, p_last);
  const int v = 16 * wave + col;
  L.valid = v % qb < L.rows;
  L.row = L.r0 + min(v % qb, L.rows - 1);
  L.head = L.hk * hn + v / qb;
  // the last key the query sees; -1: every key masked
  L.p_abs = !L.valid ? -1 : a.dense ? p_last : a.pos0 + L.row;
  L.ws = pa_window_start(a, max(L.p_abs, 0));
  L.p_top = min(L.p_abs, L.k_end);  // the last key of this chunk the query sees
  int hi = L.p_top, lo = L.valid ? L.ws : INT_MAX;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    hi = max(hi, __shfl_xor(hi, off, 64));
    lo = min(lo, __shfl_xor(lo, off, 64));
  }
  L.w_hi = __builtin_amdgcn_readfirstlane(hi);
  L.w_lo = __builtin_amdgcn_readfirstlane(lo);
  return L;
}

// Scale, soft-cap and mask the scores of keys key0 + 4r + l/16 (r = 0..3),
// move the reference maximum when the wave needs it, and turn the scores
// into weights: p = e^(s - m).
template <int NB, int NS>
__device__ __forceinline__ void pa_softmax(const PfAttn &a, const PaLane &L, v4d (&sc)[NS],
                                           int key0, int grp, double &m_ref, double &l_part,
                                           v4d (&o)[NB], const double *etab,
                                           const ExpConsts &ec) {
  const double asc = (double)a.asc, cap = (double)a.sc_att;
  double tmax = -DBL_MAX;
#pragma unroll
  for (int b = 0; b < NS; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = key0 + 16 * b + 4 * r + grp;
      double x = sc[b][r] * asc;
      if (a.sc_att != 0.0f) x = tanh(x / cap) * cap;
      sc[b][r] = (key <= L.p_top && key >= L.ws) ? x : -DBL_MAX;
      tmax = fmax(tmax, sc[b][r]);
    }
  if (__any(tmax > m_ref + kPaSlack)) {
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
  for (int b = 0; b < NS; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sc[b][r] = exp_tab(sc[b][r] - m_ref, etab, ec);
      l_part += sc[b][r];
    }
}

// The lane's outputs O^T[16 nb + 4 r + l/16][query]: normalized into xo when
// the row block took one chunk, else the chunk's partial for
// pf_attn_merge_kernel.
template <int HD, int NB>
__device__ __forceinline__ void pa_store(const PfAttn &a, const PaLane &L, const v4d (&o)[NB],
                                         double m_ref, double l_part, int grp) {
  double l = l_part + __shfl_xor(l_part, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  if (!L.valid) return;
  if (L.nchunks == 1) {
    float *orow = a.xo + (size_t)L.row * a.q_sz + L.head * HD;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) orow[16 * nb + 4 * r + grp] = (float)(o[nb][r] / l);
    return;
  }
  const size_t at = (size_t)L.chunk_id * a.n + L.row;
  double *prow = a.part + at * a.q_sz + L.head * HD;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int r = 0; r < 4; ++r) prow[16 * nb + 4 * r + grp] = o[nb][r];
  if (grp == 0) {
    double *ml = a.part + (size_t)kPfMaxSplit * a.n * a.q_sz + (at * a.n_heads + L.head) * 2;
    ml[0] = m_ref;
    ml[1] = l;
  }
}

// HD 128.  K/V tiles of 32 keys staged through registers (the next tile's
// loads in flight during the current one), V transposed with each 16-key
// block's keys permuted so that one MFMA step's 4 values are adjacent; the
// queries are fp64 registers.
template <int HD>
__global__ __launch_bounds__(kNT, 2) void pf_attn_kernel(PfAttn a) {
  constexpr int KS = HD / 4;              // score MFMA steps (dims per lane)
  constexpr int NB = HD / 16;             // 16-dim output blocks
  constexpr int RK = HD + 4;              // K row in LDS (floats)
  constexpr int VS = kPaKeys + 4;         // V^T row in LDS (floats)
  constexpr int C4 = HD / 4;              // float4 per key row
  constexpr int PF = kPaKeys * C4 / kNT;  // float4 of K (and of V) per thread
  static_assert(PF * kNT == kPaKeys * C4, "tile staging");
  __shared__ float kt[kPaKeys * RK];
  __shared__ float vt[HD * VS];
  __shared__ double etab[128];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const PaLane L = pa_lane(a, wave, col);
  if (L.empty) return;  // the whole block: before any barrier
  double qa[KS];
  {
    const float *qrow = a.qkv + (size_t)L.row * a.stride + L.head * HD + grp * KS;
#pragma unroll
    for (int s = 0; s < KS; ++s) qa[s] = (double)qrow[s];
  }
  v4d o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = v4d{0.0, 0.0, 0.0, 0.0};
  double m_ref = kPaFloor, l_part = 0.0;
  const float *kc = a.kc + (size_t)L.hk * a.clen * HD;
  const float *vc = a.vc + (size_t)L.hk * a.clen * HD;
  exp_tab_load(etab);
  const ExpConsts ec = exp_consts();

  v4f kx[PF], vx[PF];
  auto fetch = [&](int t0) {  // rows clamped to the chunk's last key: loads are unconditional
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = tid + j * kNT;
      const int t = i / C4, c4 = i - t * C4;
      const size_t at = (size_t)min(t0 + t, L.k_end) * HD + 4 * c4;
      kx[j] = *reinterpret_cast<const v4f *>(kc + at);
      vx[j] = *reinterpret_cast<const v4f *>(vc + at);
    }
  };
  fetch(L.k_lo);
  for (int t0 = L.k_lo; t0 <= L.k_end; t0 += kPaKeys) {
    lds_barrier();  // every wave is done with the previous tile
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = tid + j * kNT;
      const int t = i / C4, c4 = i - t * C4;
      const bool ok = t0 + t <= L.k_end;  // later keys: another chunk's, or not in the cache yet
      const v4f zero = {0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<v4f *>(&kt[t * RK + 4 * c4]) = ok ? kx[j] : zero;
      const v4f vv = ok ? vx[j] : zero;
      const int tp = (t & 16) | ((t & 3) << 2) | ((t >> 2) & 3);  // key 16b+4s+g -> 16b+4g+s
#pragma unroll
      for (int e = 0; e < 4; ++e) vt[(4 * c4 + e) * VS + tp] = vv[e];
    }
    lds_barrier();
    if (t0 + kPaKeys <= L.k_end) fetch(t0 + kPaKeys);

    if (t0 > L.w_hi || t0 + kPaKeys - 1 < L.w_lo) continue;  // wave-uniform
    // scores of both 16-key blocks, two independent MFMA chains
    v4d sc[2] = {v4d{0.0, 0.0, 0.0, 0.0}, v4d{0.0, 0.0, 0.0, 0.0}};
#pragma unroll
    for (int s = 0; s < KS; s += 4) {
      const v4f k0 = *reinterpret_cast<const v4f *>(&kt[col * RK + grp * KS + s]);
      const v4f k1 = *reinterpret_cast<const v4f *>(&kt[(16 + col) * RK + grp * KS + s]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sc[0] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)k0[e], qa[s + e], sc[0], 0, 0, 0);
        sc[1] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)k1[e], qa[s + e], sc[1], 0, 0, 0);
      }
    }
    pa_softmax<NB, 2>(a, L, sc, t0, grp, m_ref, l_part, o, etab, ec);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const v4f v0 = *reinterpret_cast<const v4f *>(&vt[(16 * nb + col) * VS + 4 * grp]);
      const v4f v1 = *reinterpret_cast<const v4f *>(&vt[(16 * nb + col) * VS + 16 + 4 * grp]);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        o[nb] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)v0[r], sc[0][r], o[nb], 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        o[nb] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)v1[r], sc[1][r], o[nb], 0, 0, 0);
    }
  }
  pa_store<HD, NB>(a, L, o, m_ref, l_part, grp);
}

// The same attention on the fp32 matrix cores (v_mfma_f32_16x16x4f32, twice
// the fp64 rate), head dims 128 and 256: queries, scores, weights and value
// sums in fp32, as the reference computes them (gemm_fpx, softmax,
// gemm_fpx_nn, gemma.c:5198-5255), in a different order, so the result
// agrees with the fp64 form to fp32 rounding rather than bit for bit.  One
// wave per 16 query vectors holds a whole head dim (64 + 64 registers at
// 256); K/V tiles of 32 keys are staged through registers as in
// pf_attn_kernel.  The fp32 MFMA leaves D as lane l, element r ->
// D[4 (l/16) + r][l%16], so a lane (query col, g) holds keys 4g + r of a
// 16-key block and V^T stays in natural key order.  Partials of a key-split
// row block go to the fp64 merge as for the fp64 kernels.
constexpr float kPaSlackF = 16.0f;    // p <= e^16
constexpr float kPaFloorF = -1e30f;   // far below any score, far above -FLT_MAX

// e^x for the softmax (x <= kPaSlackF) in seven instructions: 2^(x log2 e)
// by v_exp_f32 at h = fl(x * L), times 2^l ~ 1 + l ln 2 for the remainder
// l = x log2 e - h (the product's rounding error, exact by fma, plus x times
// the error of L = fl(log2 e)); |l| <= ~|x| 2^-24, so the neglected
// (l ln 2)^2 / 2 is below 2^-40 and the result is within about one ulp of
// v_exp_f32's own.  Below e^-87 the result may be 0 (the weight is then
// negligible beside the row's largest, which is at least e^-16).
__device__ __forceinline__ float exp_pa(float x) {
  constexpr float L = 1.44269502162933349609375f;       // fl(log2 e)
  constexpr float L_lo = 1.92596298909109e-8f;  // log2 e - L
  const float h = x * L;
  const float l = fmaf(x, L, -h) + x * L_lo;
  const float r = __builtin_amdgcn_exp2f(h);
  return fmaf(r, l * 0.693147182464599609375f, r);
}

template <int NB, int NS>
__device__ __forceinline__ void pa_softmax_f32(const PfAttn &a, const PaLane &L, v4f (&sc)[NS],
                                               int key0, int grp, float &m_ref, float &l_part,
                                               v4f (&o)[NB]) {
  float tmax = -FLT_MAX;
#pragma unroll
  for (int b = 0; b < NS; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = key0 + 16 * b + 4 * grp + r;
      float x = sc[b][r] * a.asc;
      if (a.sc_att != 0.0f) x = tanhf(x / a.sc_att) * a.sc_att;
      sc[b][r] = (key <= L.p_top && key >= L.ws) ? x : -FLT_MAX;
      tmax = fmaxf(tmax, sc[b][r]);
    }
  if (__any(tmax > m_ref + kPaSlackF)) {
    float rmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
    const float m_new = fmaxf(m_ref, rmax);
    const float alpha = exp_pa(m_ref - m_new);
    m_ref = m_new;
    l_part *= alpha;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) o[nb] *= alpha;
  }
#pragma unroll
  for (int b = 0; b < NS; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sc[b][r] = sc[b][r] > -FLT_MAX ? exp_pa(sc[b][r] - m_ref) : 0.0f;
      l_part += sc[b][r];
    }
}

// One LDS DMA load: every lane's 16 bytes at g land at lds + 16 * lane (lds
// wave-uniform).  Issued from inline asm so that the compiler does not treat
// every later LDS read as a possible alias of the pending load (it would
// wait for the load before each of them); the kernel waits itself (vmcnt(0)
// and a barrier) before it reads the buffer.  m0 has no other user in the
// kernel that calls this.
__device__ __forceinline__ void lds_dma16(const float *g, float *lds) {
  const uint32_t m = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float *)lds;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m), "v"(g)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// K and V tiles of 16 keys go from the cache straight into a two-slot LDS
// ring by DMA (no registers held, one barrier per tile), each row of HD
// floats as HD/4 16-byte chunks with chunk c of tile row t at position
// c ^ (t & 7): the K reads (16 lanes = 16 rows, one chunk) then hit 8
// different bank groups per 8 lanes.  Scores: lane (key col, group g)
// feeds K[col][g KS + s + e] against qa[s + e], two MFMA chains over
// alternate dims.  Values: V stays in key-major order; one 16-byte read of
// V[4 g + r][64 q + 4 col .. + 3] feeds four MFMAs, one for each of the
// output blocks 4 q + e, whose row col is dim 64 q + 4 col + e.  The lane
// (query col, g) then holds dims 64 q + 16 g + 4 r + e in o[4 q + e][r].
template <int HD>
__global__ __launch_bounds__(kNT, 2) void pf_attn_f32_kernel(PfAttn a) {
  constexpr int TK = 16;                   // keys per tile
  constexpr int KS = HD / 4;               // score MFMA steps (dims per lane)
  constexpr int NB = HD / 16;              // 16-dim output blocks
  constexpr int CR = HD / 4;               // 16-byte chunks per key row
  constexpr int TC = TK * CR;              // chunks per K (or V) tile
  constexpr int NI = 2 * TC / 64;          // DMA instructions per tile (K, then V)
  constexpr int NIW = NI / kWaves;         // per wave
  constexpr int RPI = 64 / CR;             // tile rows per DMA instruction
  static_assert(HD % 64 == 0 && CR >= 8 && NIW * kWaves == NI && kPaKeys % TK == 0,
                "tile staging");
  __shared__ v4f ring[2][2][TC];           // [slot][K, V][chunk]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const PaLane L = pa_lane(a, wave, col);
  if (L.empty) return;  // the whole block: before any barrier
  float qa[KS];
  {
    const float *qrow = a.qkv + (size_t)L.row * a.stride + L.head * HD + grp * KS;
#pragma unroll
    for (int s = 0; s < KS; s += 4) {
      const v4f q4 = *reinterpret_cast<const v4f *>(qrow + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) qa[s + e] = q4[e];
    }
  }
  v4f o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_ref = kPaFloorF, l_part = 0.0f;
  const float *kc = a.kc + (size_t)L.hk * a.clen * HD;
  const float *vc = a.vc + (size_t)L.hk * a.clen * HD;

  // this lane's share of each of the wave's DMA instructions: tile row and
  // the source chunk that lands at the lane's position (rows past the
  // chunk's last key repeat it: their weights are exactly 0)
  int trow[NIW], tsrc[NIW];
#pragma unroll
  for (int j = 0; j < NIW; ++j) {
    const int ri = (wave * NIW + j) % (NI / 2);
    const int t = ri * RPI + lane / CR, pos = lane % CR;
    trow[j] = t;
    tsrc[j] = 4 * (pos ^ (t & 7));
  }
  auto issue = [&](int t0, int slot) {
#pragma unroll
    for (int j = 0; j < NIW; ++j) {
      const int i = wave * NIW + j;  // wave-uniform
      const int kv = i / (NI / 2), ri = i % (NI / 2);
      const size_t at = (size_t)min(t0 + trow[j], L.k_end) * HD + tsrc[j];
      lds_dma16((kv == 0 ? kc : vc) + at,
                reinterpret_cast<float *>(&ring[slot][kv][ri * 64]));
    }
  };
  issue(L.k_lo, 0);
  int slot = 0;
  for (int t0 = L.k_lo; t0 <= L.k_end; t0 += TK, slot ^= 1) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's part of the tile has landed
    lds_barrier();  // every wave's part has landed, and every wave is done with the other slot
    if (t0 + TK <= L.k_end) issue(t0 + TK, slot ^ 1);

    if (t0 > L.w_hi || t0 + TK - 1 < L.w_lo) continue;  // wave-uniform
    const v4f *kt = ring[slot][0];
    const v4f *vt = ring[slot][1];
    v4f s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; s += 4) {
      const v4f k4 = kt[col * CR + (((grp * KS + s) >> 2) ^ (col & 7))];
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[0], qa[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[1], qa[s + 1], s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[2], qa[s + 2], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[3], qa[s + 3], s1, 0, 0, 0);
    }
    v4f sc[1] = {s0 + s1};
    pa_softmax_f32<NB, 1>(a, L, sc, t0, grp, m_ref, l_part, o);
#pragma unroll
    for (int q = 0; q < NB / 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 4 * grp + r;
        const v4f v4 = vt[t * CR + ((16 * q + col) ^ (t & 7))];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[4 * q + e] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[e], sc[0][r], o[4 * q + e], 0, 0, 0);
      }
  }
  float l = l_part + __shfl_xor(l_part, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  if (!L.valid) return;
  // dims 64 q + 16 grp + 4 r .. + 3 are o[4 q .. 4 q + 3][r]
  auto out4 = [&](int q, int r) {
    return v4f{o[4 * q][r], o[4 * q + 1][r], o[4 * q + 2][r], o[4 * q + 3][r]};
  };
  if (L.nchunks == 1) {
    float *orow = a.xo + (size_t)L.row * a.q_sz + L.head * HD;
#pragma unroll
    for (int q = 0; q < NB / 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<v4f *>(orow + 64 * q + 16 * grp + 4 * r) = out4(q, r) / l;
    return;
  }
  // fp32 partials (the fp64 kernels' layout in floats: half the bytes; the
  // merge still combines them in fp64)
  float *pf = reinterpret_cast<float *>(a.part);
  const size_t at = (size_t)L.chunk_id * a.n + L.row;
  float *prow = pf + at * a.q_sz + L.head * HD;
#pragma unroll
  for (int q = 0; q < NB / 4; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<v4f *>(prow + 64 * q + 16 * grp + 4 * r) = out4(q, r);
  if (grp == 0) {
    float *ml = pf + (size_t)kPfMaxSplit * a.n * a.q_sz + (at * a.n_heads + L.head) * 2;
    ml[0] = m_ref;
    ml[1] = l;
  }
}

// The same attention on the bf16 matrix cores in split precision: q, k, the
// weights p and v each as three bf16 pieces (split3x2), every product summed
// from its six leading piece products (v_mfma_f32_16x16x32_bf16, the small
// ones first) with fp32 accumulation, so the error per product is of the
// size of an fp32 rounding and the result agrees with the fp64 form to fp32
// rounding, as pf_attn_f32_kernel's does, at ~2.5x its matrix-core rate.
// A workgroup is kPbWaves waves x 16 query vectors (one workgroup per CU:
// the planes below take most of the LDS).  Key tiles of 32, whose K rows go
// by LDS DMA into an fp32 staging buffer and whose V rows (4 keys x 4 dims
// per thread) into registers while the tile before is in use; at a tile's
// start the workgroup splits both, once for all its waves, into three bf16
// planes each: K [key][dim] and V^T [dim][k], where k = 8 g + 4 b + r is the
// value product's index of key 16 b + 4 g + r -- the key whose score lane
// (query, g) holds in element r of block b, so a lane's eight weights are
// its operand of that product as they stand.  Lane (query col, g) holds the
// query's dims 32 c + 8 g .. + 7 of every piece and the outputs' dims
// 16 nb + 4 g .. + 3.  Masks, softmax and partials as pf_attn_f32_kernel.
constexpr int kPbWaves = 8;
constexpr int kPbQ = kPbWaves * 16;  // query vectors per workgroup

template <int HD>
__global__ __launch_bounds__(kPbWaves * 64) void pf_attn_bf3_kernel(PfAttn a) {
  constexpr int NT = kPbWaves * 64;
  constexpr int TK = 32;          // keys per tile
  constexpr int CH = HD / 32;     // 32-dim chunks of the score product
  constexpr int NB = HD / 16;     // 16-dim output blocks
  constexpr int C4 = HD / 4;      // float4 per key row
  constexpr int RK = HD + 8;      // K plane row (bf16): 8 rows in distinct banks
  constexpr int RV = TK + 8;      // V^T plane row (bf16)
  constexpr int SG = TK * C4;     // float4 of a K tile
  constexpr int NIW = SG / 64 / kPbWaves;  // K DMA instructions per wave and tile
  constexpr int PF = (SG + NT - 1) / NT;   // K float4 split per thread
  constexpr int VB = 8 * C4;               // V blocks (4 keys x 4 dims) per tile
  static_assert(HD % 64 == 0 && TK == kPaKeys && NIW * 64 * kPbWaves == SG && VB <= NT,
                "tile staging");
  __shared__ __attribute__((aligned(16))) __bf16 kt[3][TK * RK];
  __shared__ __attribute__((aligned(16))) __bf16 vt[3][HD * RV];
  __shared__ v4f stg[SG];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const PaLane L = pa_lane(a, wave, col);
  if (L.empty) return;  // the whole block: before any barrier
  bf8 qa[3][CH];
  {
    const float *qrow = a.qkv + (size_t)L.row * a.stride + L.head * HD + 8 * grp;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      u4 w0, w1, w2;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const v4f q4 = *reinterpret_cast<const v4f *>(qrow + 32 * c + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          const Bf3x2 sp = split3x2(q4[e], q4[e + 1]);
          w0[2 * h + e / 2] = sp.q0;
          w1[2 * h + e / 2] = sp.q1;
          w2[2 * h + e / 2] = sp.q2;
        }
      }
      qa[0][c] = as_bf8(w0);
      qa[1][c] = as_bf8(w1);
      qa[2][c] = as_bf8(w2);
    }
  }
  v4f o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_ref = kPaFloorF, l_part = 0.0f;
  const float *kc = a.kc + (size_t)L.hk * a.clen * HD;
  const float *vc = a.vc + (size_t)L.hk * a.clen * HD;

  // rows past the chunk's last key repeat it: their weights are exactly 0
  const int vtq = tid % 8, vc4 = tid / 8;  // this thread's V block (tid < VB)
  v4f vr[4];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int j = 0; j < NIW; ++j) {
      const int i = wave * NIW + j;  // wave-uniform
      const int ch = 64 * i + lane, t = ch / C4;
      lds_dma16(kc + (size_t)min(t0 + t, L.k_end) * HD + 4 * (ch - t * C4),
                reinterpret_cast<float *>(&stg[64 * i]));
    }
    if (tid < VB) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        vr[u] = *reinterpret_cast<const v4f *>(vc + (size_t)min(t0 + 4 * vtq + u, L.k_end) * HD +
                                               4 * vc4);
    }
  };
  fetch(L.k_lo);
  for (int t0 = L.k_lo; t0 <= L.k_end; t0 += TK) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's K DMAs and V rows are in
    lds_barrier();  // every wave's DMAs landed, every wave is done with the planes
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = tid + j * NT;
      if (i >= SG) break;
      const int t = i / C4, c4 = i - t * C4;
      const v4f kv = stg[i];
      const Bf3x2 lo = split3x2(kv[0], kv[1]), hi = split3x2(kv[2], kv[3]);
      *reinterpret_cast<u2 *>(&kt[0][t * RK + 4 * c4]) = u2{lo.q0, hi.q0};
      *reinterpret_cast<u2 *>(&kt[1][t * RK + 4 * c4]) = u2{lo.q1, hi.q1};
      *reinterpret_cast<u2 *>(&kt[2][t * RK + 4 * c4]) = u2{lo.q2, hi.q2};
    }
    if (tid < VB) {
      const int k0i = 8 * (vtq % 4) + 4 * (vtq / 4);  // the value product's k of key 4 vtq
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const Bf3x2 lo = split3x2(vr[0][e], vr[1][e]), hi = split3x2(vr[2][e], vr[3][e]);
        const int at = (4 * vc4 + e) * RV + k0i;
        *reinterpret_cast<u2 *>(&vt[0][at]) = u2{lo.q0, hi.q0};
        *reinterpret_cast<u2 *>(&vt[1][at]) = u2{lo.q1, hi.q1};
        *reinterpret_cast<u2 *>(&vt[2][at]) = u2{lo.q2, hi.q2};
      }
    }
    lds_barrier();  // the planes are complete; the staging buffer is free
    if (t0 + TK <= L.k_end) fetch(t0 + TK);

    if (t0 > L.w_hi || t0 + TK - 1 < L.w_lo) continue;  // wave-uniform
    v4f sc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      sc[b] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < CH; ++c) {
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
    pa_softmax_f32<NB, 2>(a, L, sc, t0, grp, m_ref, l_part, o);
    u4 w0, w1, w2;  // weight k = 4 b + r of the lane's eight is dword 2 b + r / 2
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const Bf3x2 sp = split3x2(sc[b][r], sc[b][r + 1]);
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
  if (!L.valid) return;
  // dims 16 nb + 4 grp .. + 3 are o[nb]
  if (L.nchunks == 1) {
    float *orow = a.xo + (size_t)L.row * a.q_sz + L.head * HD + 4 * grp;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) *reinterpret_cast<v4f *>(orow + 16 * nb) = o[nb] / l;
    return;
  }
  float *pf = reinterpret_cast<float *>(a.part);
  const size_t at = (size_t)L.chunk_id * a.n + L.row;
  float *prow = pf + at * a.q_sz + L.head * HD + 4 * grp;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) *reinterpret_cast<v4f *>(prow + 16 * nb) = o[nb];
  if (grp == 0) {
    float *ml = pf + (size_t)kPfMaxSplit * a.n * a.q_sz + (at * a.n_heads + L.head) * 2;
    ml[0] = m_ref;
    ml[1] = l;
  }
}

// HD 256 on wave pairs.  A whole head dim per wave needs 64 fp64 output
// accumulators and 64 fp64 query operands per lane, i.e. one wave per SIMD,
// and then nothing overlaps a wave's softmax, barriers and operand reads with
// MFMAs.  Here the two waves of a pair take the same 16 queries and one half
// of the head dim each: a wave computes the partial scores over its half,
// the pair exchanges them through LDS and both add them in the same order
// (half 0 + half 1), both run the (identical) softmax, and each accumulates
// the value sums of its half.  The MFMA count is that of one wave per query
// group; a lane holds 32 + 32 fp64 values, so two workgroups (4 waves = 2
// pairs = 32 query vectors each) share a CU and one's waits hide under the
// other's MFMAs.  K/V tiles of 16 keys go from the cache into LDS by LDS DMA
// loads (one 1 KB key row per wave instruction), double-buffered.
template <int HD, int NW>
__global__ __launch_bounds__(NW * 64, 8 / NW) void pf_attn_pair_kernel(PfAttn a) {
  static_assert(HD == 256, "one key row is one wave's 64 x 16-byte LDS load");
  constexpr int HH = HD / 2;   // dims per wave
  constexpr int KS = HH / 4;   // score MFMA steps (dims per lane)
  constexpr int NB = HH / 16;  // 16-dim output blocks per wave
  constexpr int TK = 16;       // keys per tile
  constexpr int RK = HD + 4;   // K row (floats): rows 16 bytes apart in the banks
  constexpr int RV = HD + 16;  // V row (floats): rows 16 banks apart
  constexpr int KB = 2 * TK * RK * 4, VB = 2 * TK * RV * 4;
  constexpr int RO = HH + 4;   // output staging row (doubles)
  constexpr int OB = NW * 16 * RO * 8;
  __shared__ __attribute__((aligned(16))) char smem[KB + VB > OB ? KB + VB : OB];
  float(*kt)[TK * RK] = reinterpret_cast<float(*)[TK * RK]>(smem);
  float(*vt)[TK * RV] = reinterpret_cast<float(*)[TK * RV]>(smem + KB);
  __shared__ double xch[NW][4][64];  // partial scores: [wave][r][lane]
  __shared__ double etab[128];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wave >> 1, dh = wave & 1;  // query group, dim half
  const int col = lane & 15, grp = lane >> 4;
  const PaLane L = pa_lane(a, qg, col);
  if (L.empty) return;  // the whole block: before any barrier
  double qa[KS];  // dims dh * HH + grp * KS + s
  {
    const float *qrow = a.qkv + (size_t)L.row * a.stride + L.head * HD + dh * HH + grp * KS;
#pragma unroll
    for (int s = 0; s < KS; s += 4) {
      const v4f q4 = *reinterpret_cast<const v4f *>(qrow + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) qa[s + e] = (double)q4[e];
    }
  }
  v4d o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = v4d{0.0, 0.0, 0.0, 0.0};
  double m_ref = kPaFloor, l_part = 0.0;
  const float *kc = a.kc + (size_t)L.hk * a.clen * HD;
  const float *vc = a.vc + (size_t)L.hk * a.clen * HD;
  exp_tab_load(etab);
  const ExpConsts ec = exp_consts();

  // wave w loads key rows w, w + NW, ... of the tile at t0 (rows past the
  // chunk's last key repeat it; their weights are 0)
  auto issue = [&](int t0, int bi) {
#pragma unroll
    for (int j = 0; j < TK / NW; ++j) {
      const int t = wave + NW * j;
      const size_t at = (size_t)min(t0 + t, L.k_end) * HD + 4 * lane;
      lds_dma16(kc + at, &kt[bi][t * RK]);
      lds_dma16(vc + at, &vt[bi][t * RV]);
    }
  };
  issue(L.k_lo, 0);
  int bi = 0;
  for (int t0 = L.k_lo; t0 <= L.k_end; t0 += TK, bi ^= 1) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's rows of the tile have landed
    lds_barrier();  // every wave's rows have landed, and the previous tile is done
    if (t0 + TK <= L.k_end) issue(t0 + TK, bi ^ 1);
    // both waves of a pair hold the same queries: the same decision
    const bool live = !(t0 > L.w_hi || t0 + TK - 1 < L.w_lo);
    const float *kb = &kt[bi][0];
    const float *vb = &vt[bi][0];
    v4d sc[1];
    if (live) {
      v4d s0 = v4d{0.0, 0.0, 0.0, 0.0}, s1 = s0;  // even and odd steps: two chains
#pragma unroll
      for (int s = 0; s < KS; s += 4) {
        const v4f k4 = *reinterpret_cast<const v4f *>(&kb[col * RK + dh * HH + grp * KS + s]);
        s0 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)k4[0], qa[s], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)k4[1], qa[s + 1], s1, 0, 0, 0);
        s0 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)k4[2], qa[s + 2], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)k4[3], qa[s + 3], s1, 0, 0, 0);
      }
      sc[0] = s0 + s1;
#pragma unroll
      for (int r = 0; r < 4; ++r) xch[wave][r][lane] = sc[0][r];
    }
    lds_barrier();  // the pair's partial scores
    if (!live) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const double other = xch[wave ^ 1][r][lane];
      sc[0][r] = dh == 0 ? sc[0][r] + other : other + sc[0][r];
    }
    pa_softmax<NB, 1>(a, L, sc, t0, grp, m_ref, l_part, o, etab, ec);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        o[nb] = __builtin_amdgcn_mfma_f64_16x16x4f64(
            (double)vb[(4 * r + grp) * RV + dh * HH + 16 * nb + col], sc[0][r], o[nb], 0, 0, 0);
  }
  // outputs through LDS, so that each query row's half leaves as one contiguous store
  double l = l_part + __shfl_xor(l_part, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  lds_barrier();  // every wave is done with the K/V buffers
  double *ow = reinterpret_cast<double *>(smem) + wave * 16 * RO;
  const bool whole = L.nchunks == 1;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      ow[col * RO + 16 * nb + 4 * r + grp] = whole ? o[nb][r] / l : o[nb][r];
  if (!whole && dh == 0 && grp == 0 && L.valid) {
    const size_t at = (size_t)L.chunk_id * a.n + L.row;
    double *ml = a.part + (size_t)kPfMaxSplit * a.n * a.q_sz + (at * a.n_heads + L.head) * 2;
    ml[0] = m_ref;
    ml[1] = l;
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's rows are in LDS
  __builtin_amdgcn_wave_barrier();
  const int hn = a.n_heads / a.nkv, qb = a.qpb / hn;
  for (int q = 0; q < 16; ++q) {
    const int v = 16 * qg + q;
    if (v % qb >= L.rows) continue;  // wave-uniform
    const int row = L.r0 + v % qb, head = L.hk * hn + v / qb;
    const double2 x = *reinterpret_cast<const double2 *>(ow + q * RO + 2 * lane);
    const size_t off = (size_t)head * HD + dh * HH + 2 * lane;
    if (whole) {
      *reinterpret_cast<float2 *>(a.xo + (size_t)row * a.q_sz + off) =
          float2{(float)x.x, (float)x.y};
    } else {
      *reinterpret_cast<double2 *>(a.part + ((size_t)L.chunk_id * a.n + row) * a.q_sz + off) = x;
    }
  }
}

// The chunks' partials of one row (a workgroup per row): with M the largest
// reference maximum, out = sum_c e^(m_c - M) O_c / sum_c e^(m_c - M) l_c in
// fp64, rounded once.  A chunk in which a query saw no key has l = 0, O = 0
// and m = kPaFloor (kPaFloorF), so it adds nothing.  Rows whose row block
// took a single chunk were written by the attention kernel.  P: the
// partials' type (double from the fp64 kernels, float from the fp32 one).
// With a.xq the row (merged, or as the attention kernel wrote it) is
// quantized as quantize_acts does (gemma.c:2652-2674) instead of stored:
// the o projection's quantize, fused.  NPT float4 of the row per thread.
template <class P, int NPT>
__global__ __launch_bounds__(kNT) void pf_attn_merge_kernel(PfAttn a, int hdim) {
  __shared__ double wt[kPfMaxMergeHeads][kPfMaxSplit + 1];  // weights, then the denominator
  __shared__ float redf[kWaves];
  const int row = blockIdx.x, tid = threadIdx.x;
  const int hn = a.n_heads / a.nkv, qb = a.qpb / hn;
  const int r0 = row / qb * qb;
  const auto [k_base, p_last] = pa_range(a, r0, min(qb, a.n - r0));
  const int nchunks = a.nsplit > 1 ? (p_last - k_base + a.chunk) / a.chunk : 1;
  if (nchunks == 1 && a.xq == nullptr) return;
  const int n4 = a.q_sz >> 2;
  v4f out[NPT];
  if (nchunks == 1) {
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int c = tid + j * kNT;
      out[j] = c < n4 ? reinterpret_cast<const v4f *>(a.xo + (size_t)row * a.q_sz)[c]
                      : v4f{0.f, 0.f, 0.f, 0.f};
    }
  } else {
    const P *part = reinterpret_cast<const P *>(a.part);
    const P *ml = part + (size_t)kPfMaxSplit * a.n * a.q_sz;
    for (int h = tid; h < a.n_heads; h += kNT) {
      double m = -DBL_MAX;
      for (int c = 0; c < nchunks; ++c)
        m = fmax(m, (double)ml[(((size_t)c * a.n + row) * a.n_heads + h) * 2]);
      double den = 0.0;
      for (int c = 0; c < nchunks; ++c) {
        const size_t at = ((size_t)c * a.n + row) * a.n_heads + h;
        const double w = exp((double)ml[at * 2] - m);
        wt[h][c] = w;
        den += w * (double)ml[at * 2 + 1];
      }
      wt[h][kPfMaxSplit] = den;
    }
    __syncthreads();
    // every chunk's 4 values of a float4 are loaded before any is summed (the
    // loads of a row are all in flight at once), then summed in chunk order
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int c4 = tid + j * kNT;
      out[j] = v4f{0.f, 0.f, 0.f, 0.f};
      if (c4 >= n4) continue;
      const int h = 4 * c4 / hdim;
      double v[kPfMaxSplit][4];
#pragma unroll
      for (int c = 0; c < kPfMaxSplit; ++c) {
        const P *src = part + ((size_t)min(c, nchunks - 1) * a.n + row) * a.q_sz + 4 * c4;
        if constexpr (sizeof(P) == 4) {
          const v4f x = *reinterpret_cast<const v4f *>(src);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[c][e] = (double)x[e];
        } else {
          const double2 x0 = reinterpret_cast<const double2 *>(src)[0];
          const double2 x1 = reinterpret_cast<const double2 *>(src)[1];
          v[c][0] = x0.x; v[c][1] = x0.y; v[c][2] = x1.x; v[c][3] = x1.y;
        }
      }
      double num[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int c = 0; c < kPfMaxSplit; ++c)
        if (c < nchunks)
#pragma unroll
          for (int e = 0; e < 4; ++e) num[e] += wt[h][c] * v[c][e];
#pragma unroll
      for (int e = 0; e < 4; ++e) out[j][e] = (float)(num[e] / wt[h][kPfMaxSplit]);
    }
  }
  if (a.xq == nullptr) {
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int c = tid + j * kNT;
      if (c < n4) reinterpret_cast<v4f *>(a.xo + (size_t)row * a.q_sz)[c] = out[j];
    }
    return;
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) amax = fmaxf(amax, abs_daz(out[j][e]));
  amax = block_max<kNT>(amax, redf);
  const QuantParams qp = quant_params(amax);
  int8_t *dst = a.xq + (size_t)row * a.q_sz;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * kNT;
    if (c < n4)
      reinterpret_cast<uint32_t *>(dst)[c] =
          pack4(quant_one(out[j].x, qp.inv), quant_one(out[j].y, qp.inv),
                quant_one(out[j].z, qp.inv), quant_one(out[j].w, qp.inv));
  }
  if (tid == 0) a.xs[row] = qp.scale;
}

// gate = gelu(gate) * up in place over rows [gate (mlp) | up (mlp)], grid
// (ceil(mlp / 4 / kNT), rows): the fp32-weight path's GELU (gemma.c:
// 4139-4172 with mul), each value evaluated in fp64 and rounded once as the
// quantizing kernels do.
__global__ __launch_bounds__(kNT) void gelu_mul_rows_kernel(float *g, int mlp) {
  __shared__ double etab[128];
  exp_tab_load(etab);
  const ExpConsts ec = exp_consts();
  const int c = blockIdx.x * kNT + threadIdx.x;
  float *gate = g + (size_t)blockIdx.y * 2 * mlp;
  const bool ok = c < mlp / 4;
  v4f gv = {0.f, 0.f, 0.f, 0.f}, uv = gv;
  if (ok) {
    gv = reinterpret_cast<const v4f *>(gate)[c];
    uv = reinterpret_cast<const v4f *>(gate + mlp)[c];
  }
  lds_barrier();  // the exp table
  if (!ok) return;
  v4f out;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = (float)(gelu((double)gv[e], etab, ec) * (double)uv[e]);
  reinterpret_cast<v4f *>(gate)[c] = out;
}

// One workgroup per row: out = gelu(gate) * up (gemma.c:4139-4172, the GELU
// gate fused with the up projection) rounded once, then quantized into
// xq[r] / xs[r] as quantize_act does.  g is [n][2 mlp], gate columns first.
template <int NPT, int NT>
__global__ __launch_bounds__(NT) void pf_gelu_quant_kernel(const float *g, int mlp, int8_t *xq,
                                                           float *xs, WarmRegions warm) {
  __shared__ float redf[NT / 64];
  __shared__ double etab[128];
  exp_tab_load(etab);
  const ExpConsts ec = exp_consts();
  const int tid = threadIdx.x;
  const int n4 = mlp >> 2;
  const float *gate = g + (size_t)blockIdx.x * 2 * mlp;
  const float *up = gate + mlp;
  v4f gv[NPT], uv[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = tid + j * NT;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    gv[j] = c < n4 ? reinterpret_cast<const v4f *>(gate)[c] : zero;
    uv[j] = c < n4 ? reinterpret_cast<const v4f *>(up)[c] : zero;
  }
  lds_barrier();  // the exp table
  v4f out[NPT];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[j][e] = (float)(gelu((double)gv[j][e], etab, ec) * (double)uv[j][e]);
      amax = fmaxf(amax, abs_daz(out[j][e]));
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
  warm_share(warm, blockIdx.x, gridDim.x, tid, NT);
}

template <int C, int CMAX, class F>
hipError_t by_npt(int npt, F &&launch) {
  if (npt == C) return launch(std::integral_constant<int, C>{});
  if constexpr (C < CMAX) return by_npt<C + 1, CMAX>(npt, launch);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_pf_embed(const int *tokens, int n, const int8_t *emb_q, const float *emb_s,
                           const float *emb_f, float *x, int dim, float esc, hipStream_t stream) {
  pf_embed_kernel<<<n, kNT, 0, stream>>>(tokens, emb_q, emb_s, emb_f, x, dim, esc);
  return hipGetLastError();
}

hipError_t launch_gelu_mul_rows(float *g, int n, int mlp, hipStream_t stream) {
  if (n <= 0 || mlp <= 0 || mlp % 4 != 0) return hipErrorInvalidValue;
  const int n4 = mlp / 4;
  gelu_mul_rows_kernel<<<dim3((n4 + kNT - 1) / kNT, n), kNT, 0, stream>>>(g, mlp);
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

// Keys per chunk when a row block's range of at most kmax keys is split in
// `split`: whole tiles.
int pf_chunk(int kmax, int split) {
  return ((kmax + split - 1) / split + kPaKeys - 1) / kPaKeys * kPaKeys;
}

// The key split for the split-bf16 kernel, which runs one workgroup per CU:
// each candidate split's blocks are dealt, in launch order (pa_lane's block
// order), to the CU that frees first, each costing its chunk's tiles plus a
// fixed prologue and epilogue of about two tiles (empty blocks next to
// nothing), and the merge pass reads and writes the partials once per chunk.
// Measured at the gemma-3-4b prefill (2048 rows, 8 q heads on 4 kv heads):
// sliding layers 147 -> 124 us with two chunks instead of seven, global
// layers 182 -> 146 us with three instead of eight (kernel + merge); this
// model ranks the splits as the measurements do.
// The plan is a host computation of a few thousand heap operations, and a
// decoder asks for the same few shapes at every layer: the last plans are
// kept (per thread).
int pf_bf3_split_plan(const PfAttn &b0, int hdim, int qb, int nrb, int kmax, int cus);
int pf_bf3_split(const PfAttn &b, int hdim, int qb, int nrb, int kmax, int cus) {
  struct Key {
    int n, pos0, n_heads, nkv, q_sz, slide, dense, hdim, cus;
    bool operator==(const Key &o) const {
      return n == o.n && pos0 == o.pos0 && n_heads == o.n_heads && nkv == o.nkv &&
             q_sz == o.q_sz && slide == o.slide && dense == o.dense && hdim == o.hdim &&
             cus == o.cus;
    }
  };
  constexpr int kKeep = 8;
  thread_local Key keys[kKeep];
  thread_local int plans[kKeep], used = 0, next = 0;
  const Key key{b.n, b.pos0, b.n_heads, b.nkv, b.q_sz, b.slide, b.dense, hdim, cus};
  for (int i = 0; i < used; ++i)
    if (keys[i] == key) return plans[i];
  const int split = pf_bf3_split_plan(b, hdim, qb, nrb, kmax, cus);
  keys[next] = key;
  plans[next] = split;
  next = (next + 1) % kKeep;
  used = std::min(used + 1, kKeep);
  return split;
}

int pf_bf3_split_plan(const PfAttn &b0, int hdim, int qb, int nrb, int kmax, int cus) {
  const double tile_us = 6.0 * hdim / 256.0, fixed_tiles = 2.0;
  const double merge_us = 0.143e-6 * 4.0 * (double)b0.n * b0.q_sz;  // per chunk
  const int max_split = std::min(kPfMaxSplit, (kmax + kPaKeys - 1) / kPaKeys);
  int best = 1, last_nsplit = 0;
  double best_cost = 0.0;
  // free_at: a min-heap of the CUs' busy-until times
  std::vector<double> free_at((size_t)std::max(cus, 1));
  const auto later = [](double x, double y) { return x > y; };
  for (int s = 1; s <= max_split; ++s) {
    PfAttn b = b0;
    b.chunk = pf_chunk(kmax, s);
    b.nsplit = (kmax + b.chunk - 1) / b.chunk;
    if (b.nsplit == last_nsplit) continue;
    last_nsplit = b.nsplit;
    std::fill(free_at.begin(), free_at.end(), 0.0);
    double makespan = 0.0;
    const int blocks = nrb * b.nsplit * b.nkv;
    for (int blk = 0; blk < blocks; ++blk) {
      // pa_lane's mapping of a block to its row block and chunk
      const int rot = (b.nkv * b.nsplit) % 8 == 0 ? blk / b.nkv / b.nsplit : 0;
      const int cid = ((blk / b.nkv) % b.nsplit + rot) % b.nsplit;
      const int r0 = (nrb - 1 - blk / b.nkv / b.nsplit) * qb;
      const PaRange r = pa_range(b, r0, std::min(qb, b.n - r0));
      const int nch = (r.p_last - r.k_base + b.chunk) / b.chunk;
      double cost = 0.05;
      if (cid < nch) {
        const int lo = r.k_base + cid * b.chunk, hi = std::min(lo + b.chunk - 1, r.p_last);
        cost = (hi - lo + kPaKeys) / kPaKeys + fixed_tiles;
      }
      std::pop_heap(free_at.begin(), free_at.end(), later);
      free_at.back() += cost;
      makespan = std::max(makespan, free_at.back());
      std::push_heap(free_at.begin(), free_at.end(), later);
    }
    const double us = makespan * tile_us + merge_us * b.nsplit;
    if (s == 1 || us < best_cost) {
      best = s;
      best_cost = us;
    }
  }
  return best;
}

// The fp32 mode's kernel, read at every launch so that one process can time
// or check both: GEMMA_HIP_PF_ATTN=f32 the fp32-MFMA one, =bf3 the split-bf16
// one; unset, the split-bf16 one unless the pass is so small that it would
// have fewer than kPbMinBlocks workgroups, where the fp32-MFMA kernel's
// smaller workgroups, two per CU, finish first (gemma-3-270m, 32 rows: one
// split-bf16 workgroup, 19.8 us per layer against 13.5).
constexpr int kPbMinBlocks = 32;
enum PfKind { kPfF32, kPfBf3, kPfAuto };
PfKind pf_attn_kind() {
  const char *e = getenv("GEMMA_HIP_PF_ATTN");
  if (e == nullptr) return kPfAuto;
  return strcmp(e, "f32") == 0 ? kPfF32 : strcmp(e, "bf3") == 0 ? kPfBf3 : kPfAuto;
}

// Row blocks of qpb query vectors and the longest key range among them.
struct PaGeo {
  int qb, nrb, kmax;
};
PaGeo pa_geo(const PfAttn &a, int qpb) {
  PaGeo g;
  g.qb = qpb / (a.n_heads / a.nkv);
  g.nrb = (a.n + g.qb - 1) / g.qb;
  g.kmax = 0;
  for (int rb = 0; rb < g.nrb; ++rb) {
    const PaRange r = pa_range(a, rb * g.qb, std::min(g.qb, a.n - rb * g.qb));
    g.kmax = std::max(g.kmax, r.p_last - r.k_base + 1);
  }
  return g;
}

hipError_t launch_pf_attention(const PfAttn &a, int hdim, bool f32, const DeviceInfo &dev,
                               hipStream_t stream) {
  const int hn = a.nkv > 0 ? a.n_heads / a.nkv : 0;
  if (hn <= 0 || kPbQ % hn != 0 || kPaQ % hn != 0 || kPaQPair % hn != 0 || a.n <= 0 ||
      a.part == nullptr || a.n_heads > kPfMaxMergeHeads)
    return hipErrorInvalidValue;
  bool bf3 = false;
  PaGeo geo{};
  if (f32) {
    const PfKind kind = pf_attn_kind();
    if (kind != kPfF32) {
      geo = pa_geo(a, kPbQ);
      const int most = geo.nrb * a.nkv *
                       std::min(kPfMaxSplit, (geo.kmax + kPaKeys - 1) / kPaKeys);
      bf3 = kind == kPfBf3 || most >= kPbMinBlocks;
    }
  }
  const int qpb = bf3 ? kPbQ : f32 ? kPaQ : hdim == 256 ? kPaQPair : kPaQ;
  if (!bf3) geo = pa_geo(a, qpb);
  const int qb = geo.qb, nrb = geo.nrb, kmax = geo.kmax;
  // GEMMA_HIP_PF_BLOCKS (a tuning knob, read once): split the key ranges
  // until there are about that many blocks.  Otherwise the fp32-MFMA and fp64
  // kernels (two workgroups per CU) take about 2048 blocks (half of them
  // empty for causal rows), and the split-bf16 kernel the split of
  // pf_bf3_split.
  static const int knob = [] {
    const char *e = getenv("GEMMA_HIP_PF_BLOCKS");
    const int v = e != nullptr ? atoi(e) : 0;
    return v >= 64 && v <= (1 << 16) ? v : 0;
  }();
  PfAttn b = a;
  b.qpb = qpb;
  int split;
  if (bf3 && knob == 0) {
    split = pf_bf3_split(b, hdim, qb, nrb, kmax, dev.cus);
  } else {
    const int target = knob > 0 ? knob : 2048;
    const int want = (target + nrb * a.nkv - 1) / (nrb * a.nkv);
    split = std::max(1, std::min({kPfMaxSplit, want, (kmax + kPaKeys - 1) / kPaKeys}));
  }
  b.chunk = pf_chunk(kmax, split);
  b.nsplit = (kmax + b.chunk - 1) / b.chunk;
  const dim3 grid(nrb * b.nsplit * a.nkv);
  if (bf3) {
    switch (hdim) {
      case 128: pf_attn_bf3_kernel<128><<<grid, kPbWaves * 64, 0, stream>>>(b); break;
      case 256: pf_attn_bf3_kernel<256><<<grid, kPbWaves * 64, 0, stream>>>(b); break;
      default: return hipErrorInvalidValue;
    }
  } else if (f32) {
    switch (hdim) {
      case 128: pf_attn_f32_kernel<128><<<grid, kNT, 0, stream>>>(b); break;
      case 256: pf_attn_f32_kernel<256><<<grid, kNT, 0, stream>>>(b); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (hdim) {
      case 128: pf_attn_kernel<128><<<grid, kNT, 0, stream>>>(b); break;
      case 256: pf_attn_pair_kernel<256, kPaPairWaves><<<grid, kPaPairWaves * 64, 0, stream>>>(b);
        break;
      default: return hipErrorInvalidValue;
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || (b.nsplit == 1 && b.xq == nullptr)) return e;
  if (a.q_sz % 4 != 0) return hipErrorInvalidValue;
  return by_npt<1, kPfMaxNpt>((a.q_sz / 4 + kNT - 1) / kNT, [&](auto c) {
    constexpr int NPT = decltype(c)::value;
    if (f32)
      pf_attn_merge_kernel<float, NPT><<<a.n, kNT, 0, stream>>>(b, hdim);
    else
      pf_attn_merge_kernel<double, NPT><<<a.n, kNT, 0, stream>>>(b, hdim);
    return hipGetLastError();
  });
}

hipError_t launch_pf_gelu_quant(const float *g, int n, int mlp, int8_t *xq, float *xs,
                                const WarmRegions &warm, hipStream_t stream) {
  // the fewest threads per row that cover it in kPfMaxNpt chunks (fewer idle
  // slots: gemma-3-4b's 10240 columns take 512 threads x 5 chunks exactly)
  const int n4 = mlp / 4;
  auto go = [&](auto nt) {
    constexpr int NT = decltype(nt)::value;
    return by_npt<1, kPfMaxNpt>((n4 + NT - 1) / NT, [&](auto c) {
      pf_gelu_quant_kernel<decltype(c)::value, NT><<<n, NT, 0, stream>>>(g, mlp, xq, xs, warm);
      return hipGetLastError();
    });
  };
  if ((n4 + 255) / 256 <= kPfMaxNpt) return go(std::integral_constant<int, 256>{});
  if ((n4 + 511) / 512 <= kPfMaxNpt) return go(std::integral_constant<int, 512>{});
  return go(std::integral_constant<int, 1024>{});
}

}  // namespace gh
