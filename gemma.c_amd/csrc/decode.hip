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

#include "dec_common.h"

namespace gh {
namespace {

// The int8 GEMV behind the norm prologue.  L lanes per row, CPL 16-byte
// chunks per lane, 64 / L rows per wave; a wave's rows sit `stride` apart,
// in groups g = 0, 1, ... (row base + g * stride + lane / L).
//  GELU == false: rows are the flat row range of `jobs` (q, k, v).
//  GELU == true:  virtual row 2r is gate row r (jobs.w[0]), 2r+1 is up row r
//                 (jobs.w[1]); both sit in one wave (L <= 32), and the lanes
//                 of the gate row store gelu(gate) * up to jobs.dst[0][r].
//  G >= 1: every wave has at most G groups, all loaded before the norm
//          prologue so the weight stream runs under it.
//  G == 0: any number of groups, loaded two ahead of their use.
// Every weight load is issued unconditionally (a row past the end reads a
// row of the wave's own first group, or the last row, and is not used):
// the compiler's wait counts merge the paths of a conditional load by the
// path without it, which would make the prologue wait for every weight load
// issued before its own inputs arrive.
// Requires k % 16 == 0, 16-byte aligned weight rows, k <= L * CPL * 16.
template <int L, int CPL, bool GELU, int G, int NT>
__global__ __launch_bounds__(NT) void dec_norm_gemv_kernel(DecNorm na, GemvJobs jobs,
                                                           int total, int k) {
  extern __shared__ v4i xq4[];
  constexpr int kW = NT / 64;
  __shared__ double red[kW];
  __shared__ float redf[kW];
  __shared__ double etab[GELU ? 128 : 1];
  hold_args(na);
  hold_args(jobs);
  if (GELU) exp_tab_load(etab);  // visible after the prologue's barriers
  const ExpConsts ec = exp_consts();
  constexpr int kNpt = (CPL * L * 16 + NT * 4 - 1) / (NT * 4);
  static_assert(!GELU || L <= 32, "gate and up rows must share a wave");
  constexpr int kRowsPerWave = 64 / L;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane % L;
  const int rloc = lane / L;
  const int kc = k >> 4;
  const int stride = gridDim.x * kW * kRowsPerWave;
  const int base = (blockIdx.x * kW + wave) * kRowsPerWave;  // wave-uniform
  const int own = base + rloc < total ? base + rloc : total - 1;

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
  struct Row {
    v4i w[CPL];
    float sc;  // loaded with the weights: loads complete in issue order
  };
  auto load_group = [&](int g, Row &buf) {
    const int row = base + g * stride + rloc;
    int r;
    const int j = locate(row < total ? row : own, &r);
    const gptr<const v4i> w4 =
        as_global(static_cast<const v4i *>(pick4(jobs.w, j))) + (size_t)r * kc;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;
      buf.w[i] = __builtin_nontemporal_load(w4 + (c < kc ? c : 0));
    }
    buf.sc = as_global(pick4(jobs.sc, j))[r];
  };

  NormIn<kNpt> in;
  norm_load<kNpt, NT>(na, in);
  constexpr int kDepth = G > 0 ? G : 2;
  Row rows[kDepth];
#pragma unroll
  for (int g = 0; g < kDepth; ++g) load_group(g, rows[g]);
  const float act_scale =
      norm_quant<kNpt, NT>(na, in, reinterpret_cast<int8_t *>(xq4), red, redf);

  auto process = [&](int g, const Row &w) {
    const int row = base + g * stride + rloc;
    int32_t acc = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;
      if (c < kc) acc = dot16(w.w[i], xq4[c], acc);
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    const float val = row < total ? rescale(acc, act_scale, w.sc) : 0.0f;
    int r = 0;
    const int j = locate(row < total ? row : 0, &r);
    if (GELU) {
      const float up = __shfl_xor(val, L, 64);
      if (sub == 0 && (rloc & 1) == 0 && row < total)
        as_global(pick4(jobs.dst, 0))[r] = (float)(gelu((double)val, etab, ec) * (double)up);
    } else if (sub == 0 && row < total) {
      as_global(pick4(jobs.dst, j))[r] = val;
    }
  };
  if (G > 0) {
    // groups past the wave's last are skipped whole (g * stride is uniform)
#pragma unroll
    for (int g = 0; g < kDepth; ++g)
      if (base + g * stride < total) process(g, rows[g]);
  } else {
    for (int g = 0; base + g * stride < total; g += 2) {
      process(g, rows[0]);
      load_group(g + 2, rows[0]);
      if (base + (g + 1) * stride < total) process(g + 1, rows[1]);
      load_group(g + 3, rows[1]);
    }
  }
}

// The norm prologue + int8 GEMV on the stream schedule of gemv.hip's
// stream kernel: an all-resident grid deals groups of R = 64 / L rows to its
// waves round robin, each wave reducing one group and then loading its next.
// Every workgroup computes the residual + norm + quantize prologue into LDS
// itself, with its first group's weight loads issued before it.
//  GELU == false: rows are the flat row range of `jobs` (q, k, v); a group
//                 lies within one job.
//  GELU == true:  group g covers outputs r = g R/2 .. g R/2 + R/2 - 1; row
//                 rloc of the group is gate row r (jobs.w[0]) for even rloc
//                 and up row r (jobs.w[1]) for odd, and the gate lanes store
//                 gelu(gate) * up to jobs.dst[0][r] (jobs.end[0] = 2 x outputs,
//                 the gate and up rows together; the launcher checks it).
// Loads are unconditional: a row past the end reads the job's last row and
// a chunk past k reads chunk 0; neither is used.
template <int L, int CPL, bool GELU, int NPT>
__global__ __launch_bounds__(kNT) void dec_norm_stream_kernel(DecNorm na, GemvJobs jobs,
                                                              int ngroups, int k) {
  extern __shared__ v4i xq4[];
  __shared__ double red[kWaves];
  __shared__ float redf[kWaves];
  __shared__ double etab[GELU ? 128 : 1];
  hold_args(na);
  hold_args(jobs);
  asm volatile("" ::"s"(ngroups), "s"(k));
  // the exp table is loaded first and stored to LDS after the other loads
  // are issued (visible after the prologue's barriers)
  const double etv = GELU ? kExp2Tab[threadIdx.x & 127] : 0.0;
  const ExpConsts ec = exp_consts();
  constexpr int R = 64 / L;
  static_assert(!GELU || R >= 2, "gate and up rows must share a wave");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane % L, rloc = lane / L;
  const int kc = k >> 4;
  const int nwaves = gridDim.x * kWaves;
  const int w0 = blockIdx.x * kWaves + wave;

  int gend[kMaxJobs];  // groups up to the end of each job
  {
    int prev = 0, g = 0;
#pragma unroll
    for (int t = 0; t < kMaxJobs; ++t) {
      if (t < jobs.njobs) g += (jobs.end[t] - prev + R - 1) / R;
      gend[t] = g;
      prev = jobs.end[t];
    }
  }
  struct At {
    int job, row, out;  // job, row read (clamped), row of the output
    bool ok;
  };
  auto where = [&](int g) {
    At a;
    if (GELU) {
      const int m = jobs.end[0] >> 1;  // outputs: end[0] counts gate and up rows
      a.out = g * (R / 2) + (rloc >> 1);
      a.job = rloc & 1;
      a.ok = g < ngroups && a.out < m;
      a.row = a.ok ? a.out : m - 1;
    } else {
      int j = 0, gs = 0, rs = 0;
#pragma unroll
      for (int t = 0; t < kMaxJobs - 1; ++t)
        if (t + 1 < jobs.njobs && g >= gend[t]) {
          j = t + 1;
          gs = gend[t];
          rs = jobs.end[t];
        }
      const int m = pick4(jobs.end, j) - rs;  // a register select, not a memory read
      a.out = (g - gs) * R + rloc;
      a.job = j;
      a.ok = g < ngroups && a.out < m;
      a.row = a.ok ? a.out : m - 1;
    }
    return a;
  };
  struct Slot {
    v4i w[CPL];
    float sc;  // loaded with the weights: loads complete in issue order
  };
  auto load = [&](int g, Slot &s) {
    const At a = where(g);
    const gptr<const v4i> w4 =
        as_global(static_cast<const v4i *>(pick4(jobs.w, a.job))) + (size_t)a.row * kc;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;
      s.w[i] = __builtin_nontemporal_load(w4 + (c < kc ? c : 0));
    }
    s.sc = as_global(pick4(jobs.sc, a.job))[a.row];
  };

  NormIn<NPT> in;
  norm_load<NPT, kNT>(na, in);
  Slot ring;
  load(w0, ring);
  if (GELU && threadIdx.x < 128) etab[threadIdx.x] = etv;
  const float act_scale =
      norm_quant<NPT, kNT>(na, in, reinterpret_cast<int8_t *>(xq4), red, redf);

  auto process = [&](int g, const Slot &s) {
    int32_t acc = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + i * L;
      if (c < kc) acc = dot16(s.w[i], xq4[c], acc);
    }
    acc = group_sum_i32<L>(acc);
    const At a = where(g);
    const float val = rescale(acc, act_scale, s.sc);
    if (GELU) {
      const float up = __shfl_xor(val, L, 64);  // the up row's lanes
      if (sub == 0 && (rloc & 1) == 0 && a.ok)
        as_global(pick4(jobs.dst, 0))[a.out] = (float)(gelu((double)val, etab, ec) * (double)up);
    } else if (sub == 0 && a.ok) {
      as_global(pick4(jobs.dst, a.job))[a.out] = val;
    }
  };
  const int mine = w0 < ngroups ? (ngroups - 1 - w0) / nwaves + 1 : 0;
  for (int i = 0; i < mine; ++i) {
    const int g = w0 + i * nwaves;
    process(g, ring);
    if (i + 1 < mine) load(g + nwaves, ring);
  }
}

// The norm prologue + fp32 GEMV of the unquantized ('U') decode step
// (forward_text_decode's !quant branches, gemma.c:4762-4768 and 4906-4915:
// rmsnorm, then gemv_fpx_multi of q, k, v or of gate and up, then GELU(gate)
// * up) in one launch, on gemv_f32_stream_kernel's schedule: an
// all-resident grid deals groups of R = 64 / L rows to its waves round
// robin; lane `sub` of a row takes 16-byte chunks sub, sub + L, ... in
// `passes` passes of CPL chunks, fp32 FMAs in two chains, then the fixed
// L-lane tree, the same sums as that kernel for the same L.  Every workgroup
// computes the residual and norm itself (dec_final_norm_kernel's arithmetic)
// into LDS as fp32, with its first weight loads issued before it; workgroup
// 0 stores the new residual.
//  GELU == false: rows are the flat row range of `jobs` (q, k, v).
//  GELU == true:  group g covers outputs r = g R/2 .. g R/2 + R/2 - 1; row
//                 rloc of the group is gate row r (jobs.w[0]) for even rloc
//                 and up row r (jobs.w[1]) for odd, and the gate lanes store
//                 gelu(gate) * up to jobs.dst[0][r] (jobs.end[0] = 2 x
//                 outputs), rounded once as gelu_mul_rows_kernel does.
// Loads are unconditional: a row past the end reads the job's last row and
// a chunk past k reads chunk 0; neither is summed or stored.
template <int L, int CPL, bool GELU, int NPT>
__global__ __launch_bounds__(kNT) void dec_norm_f32_kernel(DecNorm na, GemvJobs jobs, int ngroups,
                                                           int k, int passes) {
  extern __shared__ v4f hf4[];
  __shared__ double red[kWaves];
  __shared__ float redf[kWaves];
  __shared__ double etab[GELU ? 128 : 1];
  hold_args(na);
  hold_args(jobs);
  asm volatile("" ::"s"(ngroups), "s"(k), "s"(passes));
  const double etv = GELU ? kExp2Tab[threadIdx.x & 127] : 0.0;
  const ExpConsts ec = exp_consts();
  constexpr int R = 64 / L;
  static_assert(!GELU || R >= 2, "gate and up rows must share a wave");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane % L, rloc = lane / L;
  const int kc = k >> 2;
  const int nwaves = gridDim.x * kWaves;
  const int w0 = blockIdx.x * kWaves + wave;

  int gend[kMaxJobs];  // groups up to the end of each job
  {
    int prev = 0, g = 0;
#pragma unroll
    for (int t = 0; t < kMaxJobs; ++t) {
      if (t < jobs.njobs) g += (jobs.end[t] - prev + R - 1) / R;
      gend[t] = g;
      prev = jobs.end[t];
    }
  }
  struct At {
    int job, row, out;  // job, row read (clamped), row of the output
    bool ok;
  };
  auto where = [&](int g) {
    At a;
    if (GELU) {
      const int m = jobs.end[0] >> 1;
      a.out = g * (R / 2) + (rloc >> 1);
      a.job = rloc & 1;
      a.ok = g < ngroups && a.out < m;
      a.row = a.ok ? a.out : m - 1;
    } else {
      int j = 0, gs = 0, rs = 0;
#pragma unroll
      for (int t = 0; t < kMaxJobs - 1; ++t)
        if (t + 1 < jobs.njobs && g >= gend[t]) {
          j = t + 1;
          gs = gend[t];
          rs = jobs.end[t];
        }
      const int m = pick4(jobs.end, j) - rs;
      a.out = (g - gs) * R + rloc;
      a.job = j;
      a.ok = g < ngroups && a.out < m;
      a.row = a.ok ? a.out : m - 1;
    }
    return a;
  };
  struct Slot {
    v4f w[CPL];
  };
  auto load = [&](int g, int pass, Slot &s) {
    const At a = where(g);
    const gptr<const v4f> w4 =
        as_global(static_cast<const v4f *>(pick4(jobs.w, a.job))) + (size_t)a.row * kc;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = sub + (pass * CPL + i) * L;
      s.w[i] = __builtin_nontemporal_load(w4 + (c < kc ? c : 0));
    }
  };

  const int mine = w0 < ngroups ? (ngroups - 1 - w0) / nwaves + 1 : 0;
  const int items = mine * passes;
  auto item_load = [&](int t, Slot &s) { load(w0 + (t / passes) * nwaves, t % passes, s); };

  NormIn<NPT> in;
  norm_load<NPT, kNT>(na, in);
  Slot buf0, buf1;
  item_load(0, buf0);
  if (GELU && threadIdx.x < 128) etab[threadIdx.x] = etv;
  norm_quant<NPT, kNT>(na, in, nullptr, red, redf);
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int c = threadIdx.x + j * kNT;
    if (c < kc) hf4[c] = in.y[j];
  }
  lds_barrier();

  float a0 = 0.0f, a1 = 0.0f;
  auto item_sum = [&](int t, const Slot &s) {
    const int pass = t % passes;
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      const int c = sub + (pass * CPL + u) * L;
      if (c < kc) {
        const v4f xv = hf4[c];
        a0 = __builtin_fmaf(s.w[u].x, xv.x, a0);
        a1 = __builtin_fmaf(s.w[u].y, xv.y, a1);
        a0 = __builtin_fmaf(s.w[u].z, xv.z, a0);
        a1 = __builtin_fmaf(s.w[u].w, xv.w, a1);
      }
    }
    if (pass == passes - 1) {
      const float acc = group_sum_f32<L>(a0 + a1);
      const At a = where(w0 + (t / passes) * nwaves);
      if (GELU) {
        const float up = __shfl_xor(acc, L, 64);  // the up row's lanes
        if (sub == 0 && (rloc & 1) == 0 && a.ok)
          as_global(pick4(jobs.dst, 0))[a.out] =
              (float)(gelu((double)acc, etab, ec) * (double)up);
      } else if (sub == 0 && a.ok) {
        as_global(pick4(jobs.dst, a.job))[a.out] = acc;
      }
      a0 = 0.0f;
      a1 = 0.0f;
    }
  };
  for (int t = 0; t < items; t += 2) {
    item_load(t + 1, buf1);
    item_sum(t, buf0);
    if (t + 1 < items) {
      item_load(t + 2, buf0);
      item_sum(t + 1, buf1);
    }
  }
}

// x = dequantized embedding row of the step's token, or its fp32 row times
// the embedding scale (gemma.c:5468-5493)
__global__ __launch_bounds__(kNT) void dec_embed_kernel(DecEmbed a) {
  int token, pos;
  if (!step_ok(a.step, a.nvocab, a.clen, &token, &pos)) return;
  if (a.emb_f != nullptr) {
    const float *row = a.emb_f + (size_t)token * a.dim;
    for (int i = threadIdx.x; i < a.dim; i += kNT) a.x[i] = row[i] * a.esc;
    return;
  }
  const float esc = a.esc * a.emb_s[token];
  const int8_t *row = a.emb_q + (size_t)token * a.dim;
  for (int i = threadIdx.x; i < a.dim; i += kNT) a.x[i] = (float)row[i] * esc;
}

// Final residual add + final norm (gemma.c:4950-4955): one workgroup writes h.
template <int NPT>
__global__ __launch_bounds__(kNT) void dec_final_norm_kernel(DecNorm na) {
  __shared__ double red[kWaves];
  __shared__ float redf[kWaves];
  hold_args(na);
  NormIn<NPT> in;
  norm_load<NPT, kNT>(na, in);
  norm_quant<NPT, kNT>(na, in, nullptr, red, redf);
}

// Attention of one kv head over one block of keys (gemma.c:4776-4851):
// grid (max blocks, nkv), kAttB keys per block.  The workgroup prepares the
// q heads of its group (q norm, RoPE) and the new k (k norm, RoPE) and v
// rows, loads its block's K and V rows into LDS with all loads in flight at
// once (the key at the step's position comes from the new rows, so no
// workgroup waits for another; block 0 appends them to the cache), then
// computes scores, the block softmax and the value sums.  Output per (q head,
// block), in fp64: the block's max score m, l = sum exp(s - m) and
// acc[d] = sum exp(s - m) v[d]; the combine kernel merges the blocks.
template <int HD>
__global__ __launch_bounds__(kNT) void dec_attn_kernel(DecAttn a) {
  extern __shared__ double smem_d[];
  constexpr int hd = HD;
  const int hk = blockIdx.y;
  const int hn = a.n_heads / a.nkv;
  const int h0 = hk * hn;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: row selects stay scalar
  // every argument in one batch of scalar loads (the compiler otherwise
  // fetches each one where it is first used, a round trip at a time)
  asm volatile("" ::"s"(a.xq), "s"(a.xk), "s"(a.xv), "s"(a.nq), "s"(a.nk), "s"(a.rope),
               "s"(a.kc), "s"(a.vc), "s"(a.step), "s"(a.part));
  asm volatile("" ::"s"(a.n_heads), "s"(a.nkv), "s"(a.clen), "s"(a.slide), "s"(a.max_blocks),
               "s"(a.nvocab), "s"(a.asc), "s"(a.sc_att), "s"(a.eps));

  // Loads, in the order their data is needed (vector loads return in issue
  // order): this wave's prologue rows (q heads wave and wave + kWaves, or
  // the new key) and the new value row, which do not depend on the step;
  // then, once the step record is in, the rows' RoPE factors and the
  // block's cached K and V rows.  Every load is unconditional, with its
  // index clamped into range (a value loaded past the range is not used):
  // the compiler's wait counts merge the paths of a conditional load by the
  // path without it, which turned this prologue into a dozen dependent
  // memory round trips (5 us at gemma-3-1b, 17 us at 4b).
  constexpr int NJ = HD / 64, NH = NJ / 2;
  struct Row {
    float v[NJ], w[NJ], c[NH], s[NH];
  };
  auto load_in = [&](int r, Row &row) {  // r <= hn
    const float *src = r < hn ? a.xq + (size_t)(h0 + r) * hd : a.xk + (size_t)hk * hd;
    const float *w = r < hn ? a.nq : a.nk;
    const float *wl = w != nullptr ? w : src;  // any valid row when there are no weights
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      row.v[jj] = src[lane + 64 * jj];
      row.w[jj] = wl[lane + 64 * jj];
    }
  };
  auto load_cs = [&](const float *cs, Row &row) {
#pragma unroll
    for (int jj = 0; jj < NH; ++jj) {
      row.c[jj] = cs[2 * (lane + 64 * jj)];
      row.s[jj] = cs[2 * (lane + 64 * jj) + 1];
    }
  };
  Row r0, r1;
  load_in(min(wave, hn), r0);
  load_in(min(wave + kWaves, hn), r1);
  constexpr int kVn = (HD + kNT - 1) / kNT;
  float vnr[kVn];
#pragma unroll
  for (int u = 0; u < kVn; ++u) vnr[u] = a.xv[(size_t)hk * hd + min(tid + u * kNT, hd - 1)];
  // the step record last: it returns with the rows, in one round trip
  int token, pos;
  const bool step_in_range = step_ok(a.step, a.nvocab, a.clen, &token, &pos);
  asm volatile("" ::: "memory");  // keeps the loads above ahead of the step check
  if (!step_in_range) return;
  const int spos = (a.slide > 0 && pos >= a.slide) ? pos + 1 - a.slide : 0;
  const int t0 = spos + blockIdx.x * kAttB;
  if (t0 > pos) return;
  const int nt = min(kAttB, pos + 1 - t0);

  double *e = smem_d;                                       // [hn][kAttB]
  float *q = reinterpret_cast<float *>(e + hn * kAttB);     // [hn][hd]
  float *kn = q + hn * hd;                                  // [hd]
  float *vn = kn + hd;                                      // [hd]
  constexpr int KS = HD + 16;  // padded K rows: four rows of 16-byte score reads hit distinct banks
  float *kt = vn + hd;                                      // [kAttB][KS]
  float *vt = kt + kAttB * KS;                              // [kAttB][hd]
  const float *cs = a.rope + (size_t)pos * hd;              // cos, sin interleaved
  float *kc = a.kc + (size_t)hk * a.clen * hd;
  float *vc = a.vc + (size_t)hk * a.clen * hd;
  load_cs(cs, r0);
  load_cs(cs, r1);

  // the block's cached keys t0 .. t0+ncached-1 (the step's own key comes
  // from the new rows, so no workgroup waits for another)
  const int ncached = min(nt, pos - t0);
  const int vec = hd / 4;
  const int ntile = ncached * vec;
  constexpr int kTileV = kAttB * HD / 4 / kNT;  // 16-byte loads per thread per tile
  v4f kr[kTileV], vr[kTileV];
#pragma unroll
  for (int u = 0; u < kTileV; ++u) {
    const int i = tid + u * kNT;
    const int t = i / vec, c = i - t * vec;
    const size_t at = (size_t)min(t0 + t, a.clen - 1) * hd;
    kr[u] = reinterpret_cast<const v4f *>(kc + at)[c];
    vr[u] = reinterpret_cast<const v4f *>(vc + at)[c];
  }

  // q heads and the new key: optional rmsnorm (nq / nk), then RoPE
  // (gemma.c:4778-4800).  One wave per row; lane l holds d = l + 64 j, so
  // the RoPE pair (d, d + HD/2) is (j, j + HD/128) in the same lane.
  auto prep = [&](int r, Row &row) {
    const bool has_w = (r < hn ? a.nq : a.nk) != nullptr;
    if (has_w) {
      double ss = 0.0;
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) ss += (double)row.v[jj] * (double)row.v[jj];
      const double rms = rms_of(wave_sum_f64(ss), hd, a.eps);
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) row.v[jj] = norm_one(row.v[jj], rms, row.w[jj]);
    }
#pragma unroll
    for (int jj = 0; jj < NH; ++jj) {
      const double c = row.c[jj], sv = row.s[jj];
      const double x0 = row.v[jj], x1 = row.v[jj + NH];
      row.v[jj] = (float)(x0 * c - x1 * sv);
      row.v[jj + NH] = (float)(x0 * sv + x1 * c);
    }
    float *dst = r < hn ? q + (size_t)r * hd : kn;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) dst[lane + 64 * jj] = row.v[jj];
  };
  if (wave <= hn) prep(wave, r0);
  if (wave + kWaves <= hn) prep(wave + kWaves, r1);
  for (int r = wave + 2 * kWaves; r <= hn; r += kWaves) {  // more than 2 rows per wave
    Row row;
    load_in(r, row);
    load_cs(cs, row);
    prep(r, row);
  }
#pragma unroll
  for (int u = 0; u < kVn; ++u)
    if (tid + u * kNT < hd) vn[tid + u * kNT] = vnr[u];
#pragma unroll
  for (int u = 0; u < kTileV; ++u) {
    const int i = tid + u * kNT;
    if (i < ntile) {
      const int t = i / vec, c = i - t * vec;
      *reinterpret_cast<v4f *>(kt + t * KS + 4 * c) = kr[u];
      reinterpret_cast<v4f *>(vt)[i] = vr[u];
    }
  }
  lds_barrier();
  if (blockIdx.x == 0)
    for (int d = tid; d < hd; d += kNT) {
      kc[(size_t)pos * hd + d] = kn[d];
      vc[(size_t)pos * hd + d] = vn[d];
    }
  if (ncached < nt)  // the block holds the step's position: its rows from LDS
    for (int d = tid; d < hd; d += kNT) {
      kt[ncached * KS + d] = kn[d];
      vt[ncached * hd + d] = vn[d];
    }
  lds_barrier();

  // scores: four threads per (head, key) pair; thread c of the quad sums the
  // 16-byte chunks c, c + 4, c + 8, ... of the head dimension, then a quad
  // reduction
  const int npair = hn * nt;
  for (int p0 = 0; p0 < npair; p0 += kNT / 4) {
    const int pr = p0 + (tid >> 2), c = tid & 3;
    double a0 = 0.0, a1 = 0.0;
    if (pr < npair) {
      const int g = pr / nt, t = pr - g * nt;
      const v4f *qg = reinterpret_cast<const v4f *>(q + g * hd) + c;
      const v4f *kr = reinterpret_cast<const v4f *>(kt + t * KS) + c;
#pragma unroll 4
      for (int i = 0; i < HD / 16; ++i) {
        const v4f x = qg[4 * i], y = kr[4 * i];
        a0 += (double)x[0] * (double)y[0];
        a1 += (double)x[1] * (double)y[1];
        a0 += (double)x[2] * (double)y[2];
        a1 += (double)x[3] * (double)y[3];
      }
    }
    double part = a0 + a1;
    part += dpp_f64<kDppXor1>(part);
    part += dpp_f64<kDppXor2>(part);
    if (pr < npair && c == 0) {
      const int g = pr / nt, t = pr - g * nt;
      double sc = part * (double)a.asc;
      if (a.sc_att != 0.0f) sc = tanh(sc / (double)a.sc_att) * (double)a.sc_att;
      e[g * kAttB + t] = sc;
    }
  }
  lds_barrier();
  // block softmax: one wave per head, lane t holds key t (nt <= 16 lanes:
  // one DPP row)
  double *out_base = a.part + ((size_t)h0 * a.max_blocks + blockIdx.x) * (hd + 2);
  const size_t head_stride = (size_t)a.max_blocks * (hd + 2);
  for (int g = wave; g < hn; g += kWaves) {
    const bool live = lane < nt;
    double sv = live ? e[g * kAttB + lane] : -DBL_MAX;
    double m = sv;
    m = fmax(m, dpp_f64<kDppXor1>(m));
    m = fmax(m, dpp_f64<kDppXor2>(m));
    m = fmax(m, dpp_f64<kDppHalfMirror>(m));
    m = fmax(m, dpp_f64<kDppMirror>(m));
    m = readlane_f64(m, 0);
    const double x = live ? exp(sv - m) : 0.0;
    double l = x;
    l += dpp_f64<kDppXor1>(l);
    l += dpp_f64<kDppXor2>(l);
    l += dpp_f64<kDppHalfMirror>(l);
    l += dpp_f64<kDppMirror>(l);
    if (lane < kAttB) e[g * kAttB + lane] = x;  // zero past nt
    if (lane == 0) {
      out_base[g * head_stride + hd] = m;
      out_base[g * head_stride + hd + 1] = l;
    }
  }
  lds_barrier();
  // value sums: thread d holds the block's values of dimension d (zero past
  // nt, where the weights are zero too) and sums them for every head of the
  // group, four chains over the keys
  for (int d = tid; d < hd; d += kNT) {
    double v[kAttB];
#pragma unroll
    for (int t = 0; t < kAttB; ++t) v[t] = t < nt ? (double)vt[t * hd + d] : 0.0;
    for (int g = 0; g < hn; ++g) {
      const double2 *eg = reinterpret_cast<const double2 *>(e + g * kAttB);
      double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
#pragma unroll
      for (int t = 0; t < kAttB; t += 4) {
        const double2 e01 = eg[t / 2], e23 = eg[t / 2 + 1];
        a0 += e01.x * v[t];
        a1 += e01.y * v[t + 1];
        a2 += e23.x * v[t + 2];
        a3 += e23.y * v[t + 3];
      }
      out_base[g * head_stride + d] = (a0 + a1) + (a2 + a3);
    }
  }
}

// xo[h] = sum_b exp(m_b - M) acc_b / sum_b exp(m_b - M) l_b: grid (n_heads,
// hdim / 64).  The 256 threads of a workgroup split its 64 dimensions into
// 16 quads and the blocks into 16 strided groups.  At the start every thread
// issues the loads of block tid's (m, l) and of the acc values of up to
// kCombBatch of its group's blocks, so that (for up to 16 * kCombBatch
// blocks) the combine waits for memory once.  Then: M = the block-wide max
// of m; thread b computes the block weight exp(m_b - M) into LDS (the same
// bits in every workgroup of the head) and the denominator is summed; each
// thread sums its blocks' weighted acc values, and the 16 group sums are
// added in group order.
constexpr int kCombGroups = 16;
constexpr int kCombBatch = 12;

__global__ __launch_bounds__(kNT) void dec_attn_combine_kernel(DecAttn a) {
  extern __shared__ double wts[];
  __shared__ double red[kWaves];
  __shared__ double2 gsum[kCombGroups][32];
  hold_args(a);
  const int hd = a.hdim, h = blockIdx.x, tid = threadIdx.x;
  const int stride = hd + 2;
  const double *p = a.part + (size_t)h * a.max_blocks * stride;
  const int g = tid / 16, q = tid % 16;
  const int d = blockIdx.y * 64 + 4 * q;
  const bool dv = d < hd;
  // (m, l) of blocks tid and tid + 256, then this group's first kCombBatch
  // blocks' acc values.  They are issued before the step record is in, so
  // the two memory round trips overlap: the indices are clamped into the
  // partials buffer (max_blocks per head), and the values of blocks at or
  // past the step's block count nb, left from earlier steps or never
  // written, are selected away or not read once nb is known.
  const int top = a.max_blocks - 1;
  constexpr int kMl = 2;
  double mraw[kMl], lb[kMl];
#pragma unroll
  for (int u = 0; u < kMl; ++u) {
    const double *pb = p + (size_t)min(tid + u * kNT, top) * stride;
    mraw[u] = pb[hd];
    lb[u] = pb[hd + 1];
  }
  const int dc = dv ? d : 0;
  double2 x01[kCombBatch], x23[kCombBatch];
#pragma unroll
  for (int u = 0; u < kCombBatch; ++u) {
    const double *pb = p + (size_t)min(g + u * kCombGroups, top) * stride;
    x01[u] = *reinterpret_cast<const double2 *>(pb + dc);
    x23[u] = *reinterpret_cast<const double2 *>(pb + dc + 2);
  }
  // No early return on a rejected step (which stores nothing): a branch here
  // lets the compiler sink the loads above past it, one round trip later.
  int token, pos;
  const bool ok = step_ok(a.step, a.nvocab, a.clen, &token, &pos);
  if (!ok) pos = 0;
  const int spos = (a.slide > 0 && pos >= a.slide) ? pos + 1 - a.slide : 0;
  const int nb = (pos + 1 - spos + kAttB - 1) / kAttB;
  double mb[kMl];
#pragma unroll
  for (int u = 0; u < kMl; ++u) mb[u] = tid + u * kNT < nb ? mraw[u] : -DBL_MAX;
  double m = fmax(mb[0], mb[1]);
  for (int b = tid + kMl * kNT; b < nb; b += kNT) m = fmax(m, p[(size_t)b * stride + hd]);
  m = fmax(m, dpp_f64<kDppXor1>(m));
  m = fmax(m, dpp_f64<kDppXor2>(m));
  m = fmax(m, dpp_f64<kDppHalfMirror>(m));
  m = fmax(m, dpp_f64<kDppMirror>(m));
  m = fmax(fmax(readlane_f64(m, 0), readlane_f64(m, 16)),
           fmax(readlane_f64(m, 32), readlane_f64(m, 48)));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  lds_barrier();
  m = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmax(m, red[w]);
  double den = 0.0;
#pragma unroll
  for (int u = 0; u < kMl; ++u) {
    const int b = tid + u * kNT;
    if (b < nb) {
      const double w = exp(mb[u] - m);
      wts[b] = w;
      den += w * lb[u];
    }
  }
  for (int b = tid + kMl * kNT; b < nb; b += kNT) {
    const double w = exp(p[(size_t)b * stride + hd] - m);
    wts[b] = w;
    den += w * p[(size_t)b * stride + hd + 1];
  }
  // block_sum's first barrier orders the reads of red above before red is
  // reused; its last one makes wts complete
  den = block_sum(den, red);
  double2 s01 = {0.0, 0.0}, s23 = {0.0, 0.0};
#pragma unroll
  for (int u = 0; u < kCombBatch; ++u) {
    const int b = g + u * kCombGroups;
    if (b >= nb) break;
    const double w = wts[b];
    s01.x += w * x01[u].x;
    s01.y += w * x01[u].y;
    s23.x += w * x23[u].x;
    s23.y += w * x23[u].y;
  }
  if (dv)  // blocks past the first batch (long contexts): one more round trip each batch
    for (int b = g + kCombBatch * kCombGroups; b < nb; b += kCombGroups) {
      const double w = wts[b];
      const double2 y01 = *reinterpret_cast<const double2 *>(p + (size_t)b * stride + d);
      const double2 y23 = *reinterpret_cast<const double2 *>(p + (size_t)b * stride + d + 2);
      s01.x += w * y01.x;
      s01.y += w * y01.y;
      s23.x += w * y23.x;
      s23.y += w * y23.y;
    }
  gsum[g][2 * q] = s01;
  gsum[g][2 * q + 1] = s23;
  lds_barrier();
  if (tid < 32) {
    const int dd = blockIdx.y * 64 + 2 * tid;
    double2 t = gsum[0][tid];
#pragma unroll
    for (int gg = 1; gg < kCombGroups; ++gg) {
      t.x += gsum[gg][tid].x;
      t.y += gsum[gg][tid].y;
    }
    if (ok && dd < hd) {
      a.xo[(size_t)h * hd + dd] = (float)(t.x / den);
      a.xo[(size_t)h * hd + dd + 1] = (float)(t.y / den);
    }
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
  lds_barrier();
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
    lds_barrier();
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
  lds_barrier();
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
    lds_barrier();
  }
  if (threadIdx.x == 0) {
    const int count = step[2];
    if (count >= 0 && count < max_tokens) tokens[count] = si[0];
    step[0] = si[0];
    step[1] = step[1] + 1;
    step[2] = count + 1;
  }
}

// 1024-thread workgroups, one per CU: the prologue is paid once per CU and
// each workgroup streams its rows with one row per row group in flight
// ahead (measured on the 1b/4b q/k/v and gate/up shapes against 256-thread
// workgroups at up to 8 per CU, which pay the prologue up to 8 times).
constexpr int kNormNT = 1024;

template <int L, int CPL, bool GELU, int G>
hipError_t launch_norm_gemv_t(const DecNorm &na, const GemvJobs &jobs, int total, int k,
                              int blocks, hipStream_t stream) {
  const size_t lds = (size_t)(k + 15) / 16 * 16;
  dec_norm_gemv_kernel<L, CPL, GELU, G, kNormNT>
      <<<dim3((unsigned)blocks), kNormNT, lds, stream>>>(na, jobs, total, k);
  return hipGetLastError();
}

// Groups per wave with one workgroup per CU; the weight registers of all
// groups (G * CPL * 4 per lane) are kept within 64 where G > 0.
template <int L, int CPL, bool GELU>
hipError_t norm_gemv_groups(const DecNorm &na, const GemvJobs &jobs, int total, int k,
                            const DeviceInfo &dev, hipStream_t stream) {
  constexpr int rows_per_block = kNormNT / 64 * (64 / L);
  const long need = (total + rows_per_block - 1) / rows_per_block;
  const int blocks = (int)(need < dev.cus ? need : dev.cus);
  const long stride = (long)blocks * rows_per_block;
  const long groups = (total + stride - 1) / stride;
  if (groups <= 1) return launch_norm_gemv_t<L, CPL, GELU, 1>(na, jobs, total, k, blocks, stream);
  if (groups == 2 && 2 * CPL <= 16)
    return launch_norm_gemv_t<L, CPL, GELU, (2 * CPL <= 16 ? 2 : 0)>(na, jobs, total, k, blocks,
                                                                     stream);
  if (groups == 3 && 3 * CPL <= 16)
    return launch_norm_gemv_t<L, CPL, GELU, (3 * CPL <= 16 ? 3 : 0)>(na, jobs, total, k, blocks,
                                                                     stream);
  if (groups == 4 && 4 * CPL <= 16)
    return launch_norm_gemv_t<L, CPL, GELU, (4 * CPL <= 16 ? 4 : 0)>(na, jobs, total, k, blocks,
                                                                     stream);
  return launch_norm_gemv_t<L, CPL, GELU, 0>(na, jobs, total, k, blocks, stream);
}

template <int L, bool GELU, int C, int CMAX>
hipError_t norm_gemv_cpl(int cpl, const DecNorm &na, const GemvJobs &jobs, int total, int k,
                         const DeviceInfo &dev, hipStream_t stream) {
  if (cpl == C) return norm_gemv_groups<L, C, GELU>(na, jobs, total, k, dev, stream);
  if constexpr (C < CMAX)
    return norm_gemv_cpl<L, GELU, C + 1, CMAX>(cpl, na, jobs, total, k, dev, stream);
  return hipErrorInvalidValue;
}

// dec_norm_stream_kernel: L lanes per row (the fewest with CPL <= 10),
// NPT covering dim = k
constexpr int kNsMaxCpl = 10;
typedef hipError_t (*NormStreamFn)(const DecNorm &, const GemvJobs &, int, int,
                                   const DeviceInfo &, hipStream_t);

template <int L, int CPL, bool GELU>
hipError_t launch_norm_stream(const DecNorm &na, const GemvJobs &jobs, int ngroups, int k,
                              const DeviceInfo &dev, hipStream_t stream) {
  constexpr int NPT = (L * CPL * 16 + kNT * 4 - 1) / (kNT * 4);
  const auto kern = dec_norm_stream_kernel<L, CPL, GELU, NPT>;
  const size_t lds = (size_t)(k + 15) / 16 * 16;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kNT, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const long need = (ngroups + kWaves - 1) / kWaves;
  const long cap = (long)dev.cus * per_cu;
  kern<<<dim3((unsigned)(need < cap ? need : cap)), kNT, lds, stream>>>(na, jobs, ngroups, k);
  return hipGetLastError();
}

template <int L, bool GELU, int C, int CMAX = kNsMaxCpl>
NormStreamFn norm_stream_for(int cpl) {
  if (cpl == C) return &launch_norm_stream<L, C, GELU>;
  if constexpr (C < CMAX) return norm_stream_for<L, GELU, C + 1, CMAX>(cpl);
  return nullptr;
}

// nullptr where the streamed kernel does not apply (GELU rows need L <= 32)
NormStreamFn norm_stream_fn(int kc, bool gelu) {
  if (kc <= 8 * kNsMaxCpl)
    return gelu ? norm_stream_for<8, true, 1>((kc + 7) / 8) : norm_stream_for<8, false, 1>((kc + 7) / 8);
  if (kc <= 16 * kNsMaxCpl)
    return gelu ? norm_stream_for<16, true, 6>((kc + 15) / 16)
                : norm_stream_for<16, false, 6>((kc + 15) / 16);
  if (kc <= 32 * kNsMaxCpl)
    return gelu ? norm_stream_for<32, true, 6>((kc + 31) / 32)
                : norm_stream_for<32, false, 6>((kc + 31) / 32);
  if (!gelu && kc <= 64 * 6) return norm_stream_for<64, false, 6, 6>((kc + 63) / 64);
  return nullptr;
}

}  // namespace

namespace {

constexpr int kNfMaxNpt = 6;  // dim <= 6144

template <int L, int CPL, bool GELU, int NPT>
hipError_t launch_norm_f32(const DecNorm &na, const GemvJobs &jobs, int ngroups, int k, int passes,
                           const DeviceInfo &dev, hipStream_t stream) {
  const auto kern = dec_norm_f32_kernel<L, CPL, GELU, NPT>;
  const size_t lds = (size_t)(k / 4) * 16;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kNT, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const long need = (ngroups + kWaves - 1) / kWaves;
  const long cap = (long)dev.cus * per_cu;
  kern<<<dim3((unsigned)(need < cap ? need : cap)), kNT, lds, stream>>>(na, jobs, ngroups, k,
                                                                       passes);
  return hipGetLastError();
}

// f32_stream_shape takes 8 or 16 lanes only for rows of at most 192 chunks
// (one norm chunk per thread) and 32 lanes for plain rows only up to 384
// chunks, so those kernels exist for the NPT they can meet
template <int L, bool GELU>
constexpr int kNfNpt = L <= 16 ? 1 : (L == 32 && !GELU) ? 2 : kNfMaxNpt;

template <int L, int CPL, bool GELU, int N = 1>
hipError_t norm_f32_npt(int npt, const DecNorm &na, const GemvJobs &jobs, int ngroups, int k,
                        int passes, const DeviceInfo &dev, hipStream_t stream) {
  if (npt == N)
    return launch_norm_f32<L, CPL, GELU, N>(na, jobs, ngroups, k, passes, dev, stream);
  if constexpr (N < kNfNpt<L, GELU>)
    return norm_f32_npt<L, CPL, GELU, N + 1>(npt, na, jobs, ngroups, k, passes, dev, stream);
  return hipErrorInvalidValue;
}

template <int L, bool GELU>
hipError_t norm_f32_cpl(int cpl, int npt, const DecNorm &na, const GemvJobs &jobs, int ngroups,
                        int k, int passes, const DeviceInfo &dev, hipStream_t stream) {
  switch (cpl) {
    case 8: return norm_f32_npt<L, 8, GELU>(npt, na, jobs, ngroups, k, passes, dev, stream);
    case 10: return norm_f32_npt<L, 10, GELU>(npt, na, jobs, ngroups, k, passes, dev, stream);
    default: return norm_f32_npt<L, 12, GELU>(npt, na, jobs, ngroups, k, passes, dev, stream);
  }
}

}  // namespace

hipError_t launch_dec_norm_gemv_f32(const DecNorm &na, const GemvJobs &jobs, int total, int k,
                                    bool gelu, const DeviceInfo &dev, hipStream_t stream) {
  if (total <= 0 || k <= 0 || k % 4 != 0 || k != na.dim || k > 4 * kNT * kNfMaxNpt)
    return hipErrorInvalidValue;
  for (int j = 0; j < (gelu ? 2 : jobs.njobs); ++j)
    if ((uintptr_t)jobs.w[j] % 16 != 0) return hipErrorInvalidValue;
  if (!gelu) {
    for (int j = 0, prev = 0; j < jobs.njobs; prev = jobs.end[j], ++j)
      if (jobs.end[j] <= prev) return hipErrorInvalidValue;
  } else if (total % 2 != 0 || jobs.end[0] != total) {
    return hipErrorInvalidValue;
  }
  // lanes per row and chunks per lane as the fp32 stream GEMV (at most 32
  // lanes for the gate/up pairing: two rows per wave)
  const int kc = k / 4;
  const F32StreamShape sh = f32_stream_shape(kc, gelu, total);
  const int lanes = sh.lanes, passes = sh.passes;
  const int rows = 64 / lanes;
  int ngroups = 0;
  if (gelu) {
    ngroups = (total / 2 + rows / 2 - 1) / (rows / 2);
  } else {
    for (int j = 0, prev = 0; j < jobs.njobs; prev = jobs.end[j], ++j)
      ngroups += (jobs.end[j] - prev + rows - 1) / rows;
  }
  const int npt = (kc + kNT - 1) / kNT;
  const int c = sh.cpl;
  switch (lanes) {
    case 8:
      return gelu ? norm_f32_cpl<8, true>(c, npt, na, jobs, ngroups, k, passes, dev, stream)
                  : norm_f32_cpl<8, false>(c, npt, na, jobs, ngroups, k, passes, dev, stream);
    case 16:
      return gelu ? norm_f32_cpl<16, true>(c, npt, na, jobs, ngroups, k, passes, dev, stream)
                  : norm_f32_cpl<16, false>(c, npt, na, jobs, ngroups, k, passes, dev, stream);
    case 32:
      return gelu ? norm_f32_cpl<32, true>(c, npt, na, jobs, ngroups, k, passes, dev, stream)
                  : norm_f32_cpl<32, false>(c, npt, na, jobs, ngroups, k, passes, dev, stream);
    default:
      return norm_f32_cpl<64, false>(c, npt, na, jobs, ngroups, k, passes, dev, stream);
  }
}

hipError_t launch_dec_norm_gemv(const DecNorm &na, const GemvJobs &jobs, int total, int k,
                                bool gelu, const DeviceInfo &dev, hipStream_t stream) {
  if (total <= 0 || k <= 0 || k % 16 != 0 || k > 6144) return hipErrorInvalidValue;
  // every plain job must have rows: the kernels clamp a group's row to its
  // job's last row, which an empty job does not have (the GELU form pairs
  // gate and up rows of one range, given as end[0] = end[1] = 2 * mlp)
  if (!gelu) {
    for (int j = 0, prev = 0; j < jobs.njobs; prev = jobs.end[j], ++j)
      if (jobs.end[j] <= prev) return hipErrorInvalidValue;
  } else if (total % 2 != 0 || jobs.end[0] != total) {
    return hipErrorInvalidValue;
  }
  const int kc = k / 16;
  if (const NormStreamFn fn = norm_stream_fn(kc, gelu)) {
    int lanes = 8;
    while ((kc + lanes - 1) / lanes > kNsMaxCpl) lanes *= 2;
    const int rows = 64 / lanes;
    int ngroups = 0;
    if (gelu) {
      ngroups = (total / 2 + rows / 2 - 1) / (rows / 2);
    } else {
      for (int j = 0, prev = 0; j < jobs.njobs; prev = jobs.end[j], ++j)
        ngroups += (jobs.end[j] - prev + rows - 1) / rows;
    }
    return fn(na, jobs, ngroups, k, dev, stream);
  }
  // 32 lanes per row (two rows per wave, as the gate/up pairing needs) up to
  // 256 chunks (k = 4096); 64 lanes beyond that for plain rows
  if (kc <= 32 * 8 || gelu) {
    const int cpl = (kc + 31) / 32;
    return gelu ? norm_gemv_cpl<32, true, 1, 8>(cpl, na, jobs, total, k, dev, stream)
                : norm_gemv_cpl<32, false, 1, 8>(cpl, na, jobs, total, k, dev, stream);
  }
  return norm_gemv_cpl<64, false, 5, 6>((kc + 63) / 64, na, jobs, total, k, dev, stream);
}

hipError_t launch_dec_embed(const DecEmbed &a, hipStream_t stream) {
  dec_embed_kernel<<<1, kNT, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_dec_final_norm(const DecNorm &na, hipStream_t stream) {
  switch ((na.dim + kNT * 4 - 1) / (kNT * 4)) {
    case 1: dec_final_norm_kernel<1><<<1, kNT, 0, stream>>>(na); break;
    case 2: dec_final_norm_kernel<2><<<1, kNT, 0, stream>>>(na); break;
    case 3: dec_final_norm_kernel<3><<<1, kNT, 0, stream>>>(na); break;
    case 4: dec_final_norm_kernel<4><<<1, kNT, 0, stream>>>(na); break;
    case 5: dec_final_norm_kernel<5><<<1, kNT, 0, stream>>>(na); break;
    case 6: dec_final_norm_kernel<6><<<1, kNT, 0, stream>>>(na); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dec_attention(const DecAttn &a, hipStream_t stream) {
  const dim3 grid(a.max_blocks, a.nkv);
  const size_t lds = dec_attn_lds(a.n_heads / a.nkv, a.hdim);
  switch (a.hdim) {
    case 128: dec_attn_kernel<128><<<grid, kNT, lds, stream>>>(a); break;
    case 256: dec_attn_kernel<256><<<grid, kNT, lds, stream>>>(a); break;
    case 384: dec_attn_kernel<384><<<grid, kNT, lds, stream>>>(a); break;
    case 512: dec_attn_kernel<512><<<grid, kNT, lds, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dec_attn_combine_kernel<<<dim3(a.n_heads, (a.hdim + 63) / 64), kNT, (size_t)a.max_blocks * 8,
                            stream>>>(a);
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
