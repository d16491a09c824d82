#!/usr/bin/env python3
"""Benchmark of the W8A8 matmul hot path on one MI355X.

Headline (BASELINE.json metric "int8 GEMV HBM GB/s + GEMM TOPS (% roofline);
decode tok/s at gemma-3-1b shape", workload = BASELINE.json config 2):

  step  = one pass over the gemma-3-1b decode GEMVs at M = 1, grouped as the
          reference's decode call sites issue them (gemma.c:4768-4966):
          q/k/v as one gemv_int8_multi, o, gate/up as one gemv_int8_multi,
          down and the tied LM head; each launch quantizes the fp32
          activation inside the GEMV kernel (gemma_hip_quantize_matmul).
  value = algorithmic HBM bytes of a step x steps / elapsed, in GB/s.

Weights are int8 uniform in [-127, 127], scales U(1e-3, 1e-2), x ~ N(0,1)
with 1% of channels x20.  Weight copies rotate so that every launch reads
its matrix from HBM, not from the 256 MB Infinity Cache (see rotate_copies).
Steps are replayed from a HIP graph (one graph = ROT_STEPS steps) so the
timed region measures the GPU, not Python's launch overhead.

The JSON line also carries, measured in the same run:
  roofline      the dominant kernel (the LM-head GEMV launch): algorithmic
                bytes / its average launch duration (HIP events on its stream)
  per_gemv      the same for every launch of the sweep
  per_gemv_4b   the same at the gemma-3-4b decode shapes (config 5), and
                their sum ("all": bytes of the five launches / summed time)
  gemm          int8 MFMA GEMM TOPS at the gemma-3-4b prefill shapes (M=2048)
                and the SigLIP tower shapes (M=4096), % of the 5.0 POPS peak
  per_gemv_f32  the fp32 fallback ('U' files, gemv_fpx): the sweep's launches
                with fp32 weights, GB/s per launch
  gemm_f32      the fp32 GEMM (gemm_fpx) at the gemma-3-4b prefill shapes,
                TFLOP/s of fp32 work; by default split-bf16 on the bf16
                matrix cores (six bf16 products per multiply-add: bound
                2500 / 6 = 416.7 TF/s), with GEMMA_HIP_GEMM_F32=mfma the
                fp32-MFMA kernel (bound 157.3 TF/s)
  decode_1b     tokens/s of the full W8A8 matmul path of one gemma-3-1b
                decode token (26 layers x {qkv, o, gate/up, down} + LM head)
  decoder       configs 3 (gemma-3-1b: 512 prompt tokens, then 256 decode
                steps) and 5 (gemma-3-4b: 2048, then 512) fully on the GPU:
                the batched prefill (gemma_hip_decoder_prefill: the int8
                projections as GEMMs, causal attention, norms, GELU) in
                tokens/s and int8 TOPS of its GEMMs, then tokens/s of the
                device-resident greedy decode step (gemma_hip_decoder_generate:
                embedding, norms, q/k/v, RoPE, KV cache, attention, o, GELU,
                down, LM head, argmax); "gemma-3-1b:U" is config 3 as an
                unquantized ('U') model (gemma_hip_decoder_create_f32: fp32
                GEMVs, ~4 GB of weights per token; split-bf16 fp32 GEMMs in
                the prompt pass)
  vision        config 4 end to end: one 896x896 image through the SigLIP
                tower on the GPU (gemma_hip_vision_forward), ms per image;
                ms_per_image_u the same tower from fp32 weights ('U')
  cpu_baseline  the reference's own quantize_act + gemv_int8(_multi), compiled
                from its source (oracle/_ref/gemma_ref_clang), on the host cores
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import subprocess
import sys

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "gemma.c_amd")
for _p in (REPO, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
# the kernel the LM-head launch runs (as rocprofv3 names it)
LM_KERNEL = "gemv_i8_stream_kernel<8, 9, 1, true, 256>"
INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA
FP32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 MFMA
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
ROTATE_BYTES = 512 << 20   # > 2x the 256 MB Infinity Cache
ROT_STEPS = 8              # steps per captured graph
TIMING_RUNS = 5            # per-launch and GEMM timings: median of this many runs
MIN_TIMED_MS = 100.0       # the headline's K-step region is repeated to at least this

METRIC = ("int8 GEMV HBM GB/s + GEMM TOPS (% roofline); decode tok/s at "
          "gemma-3-1b shape")

# gemma-3-1b decode GEMV launches: (name, out rows of each job, reduction K) --
# BASELINE.json config 2; q/k/v and gate/up share one quantized activation and
# one launch, as gemv_int8_multi does at gemma.c:4768-4773 and 4911-4915
SWEEP_1B = [("qkv", (1024, 256, 256), 1152), ("o", (1152,), 1024),
            ("gate_up", (6912, 6912), 1152), ("down", (1152,), 6912),
            ("lm_head", (262144,), 1152)]

# gemma-3-4b decode GEMV launches (BASELINE.json config 5's decode phase), the
# shapes the decode-GEMV target is stated at; reported beside the headline
SWEEP_4B = [("qkv", (2048, 1024, 1024), 2560), ("o", (2560,), 2048),
            ("gate_up", (10240, 10240), 2560), ("down", (2560,), 10240),
            ("lm_head", (262144,), 2560)]

# gemma-3-4b prefill (M = 2048) and SigLIP (M = 4096) GEMMs: (name, M, N, K)
GEMM_SHAPES = [("4b_q", 2048, 2048, 2560), ("4b_kv", 2048, 1024, 2560),
               ("4b_o", 2048, 2560, 2048), ("4b_gate_up", 2048, 10240, 2560),
               ("4b_down", 2048, 2560, 10240),
               ("siglip_qkvo", 4096, 1152, 1152), ("siglip_fc1", 4096, 4304, 1152),
               ("siglip_fc2", 4096, 1152, 4304)]
# per transformer layer, how often each 4b / SigLIP shape occurs
GEMM_COUNTS = {"4b_q": 1, "4b_kv": 2, "4b_o": 1, "4b_gate_up": 2, "4b_down": 1,
               "siglip_qkvo": 4, "siglip_fc1": 1, "siglip_fc2": 1}

# gemma-3-1b: hidden 1152, FFN 6912, 26 layers, 4 q heads / 1 kv head, hd 256
DEC_1B = dict(dim=1152, mlp=6912, layers=26, q=1024, kv=256, vocab=262144)


def gemv_bytes(n: int, k: int) -> int:
    """Algorithmic HBM bytes of one fused quantize+GEMV over n output rows (of
    one or several jobs sharing x): int8 W [n][k], fp32 row scales [n], fp32
    x [k], fp32 y [n]."""
    return n * k + 4 * n + 4 * k + 4 * n


def gemv_f32_bytes(n: int, k: int) -> int:
    """Algorithmic HBM bytes of one fp32 GEMV: fp32 W [n][k], x [k], y [n]."""
    return 4 * n * k + 4 * k + 4 * n


def gemm_ops(m: int, n: int, k: int) -> int:
    return 2 * m * n * k


def rotate_copies(wbytes: int) -> int:
    """Distinct weight copies per shape: ceil(512 MB / W), capped at the
    graph's ROT_STEPS.  Within a graph, a copy is reused only after every
    other shape of ROT_STEPS steps (>= 8 x 330 MB) has been streamed, far
    beyond the 256 MB Infinity Cache."""
    return max(1, min(ROT_STEPS, math.ceil(ROTATE_BYTES / wbytes)))


def outlier_acts(torch, shape, gen):
    x = torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32)
    cols = torch.rand(shape[-1], generator=gen, device="cuda") < 0.01
    x[..., cols] *= 20.0
    return x


def rand_i8(torch, shape, gen):
    return torch.randint(-127, 128, shape, generator=gen, device="cuda", dtype=torch.int8)


def rand_scales(torch, n, gen):
    return torch.rand(n, generator=gen, device="cuda") * 9e-3 + 1e-3


class Timer:
    """HIP-event timing on torch's current stream (the stream every launch
    below is enqueued on)."""

    def __init__(self, torch):
        self.torch = torch

    def elapsed_ms(self, fn, busy=None) -> float:
        torch = self.torch
        if busy is not None:
            busy()  # keep the GPU busy so the host enqueues fn ahead of it
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        end.synchronize()
        return start.elapsed_time(end)


def capture(torch, fn):
    """Capture fn(stream_handle) into a HIP graph (after one eager run)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return graph


def build_sweep(torch, gh, gen, sweep=SWEEP_1B):
    shapes = []
    for name, ns, k in sweep:
        n = sum(ns)
        copies = rotate_copies(n * k)
        ws = [[rand_i8(torch, (r, k), gen) for r in ns] for _ in range(copies)]
        ss = [[rand_scales(torch, r, gen) for r in ns] for _ in range(copies)]
        x = outlier_acts(torch, (k,), gen)
        ys = [torch.empty(r, device="cuda", dtype=torch.float32) for r in ns]
        jobs = [gh.jobs([(w, s, y, r) for w, s, y, r in zip(wc, sc, ys, ns)])
                for wc, sc in zip(ws, ss)]
        shapes.append(dict(name=name, n=list(ns), k=k, copies=copies, w=ws, s=ss, x=x, y=ys,
                           jobs=jobs, bytes=gemv_bytes(n, k)))
    return shapes


def launch_gemv(gh, sh, copy, stream):
    arr, nj = sh["jobs"][copy % sh["copies"]]
    if sh.get("f32"):
        rc = gh.lib.gemma_hip_matmul_f32_multi(arr, nj, sh["x"].data_ptr(), sh["k"], stream)
    else:
        rc = gh.lib.gemma_hip_quantize_matmul(arr, nj, sh["x"].data_ptr(), sh["k"], None, None,
                                              stream)
    if rc != 0:
        raise RuntimeError(gh.lib.gemma_hip_last_error().decode())


def build_sweep_f32(torch, gh, gen, sweep=SWEEP_1B):
    """The sweep's launches on the fp32 path (gemv_fpx / gemv_fpx_multi,
    gemma.c:2730-2752, 2839-2858): fp32 weights N(0, 0.02), fp32 x."""
    shapes = []
    for name, ns, k in sweep:
        n = sum(ns)
        copies = max(1, min(ROT_STEPS, math.ceil(ROTATE_BYTES / (4 * n * k))))
        ws = [[torch.randn((r, k), generator=gen, device="cuda") * 0.02 for r in ns]
              for _ in range(copies)]
        x = outlier_acts(torch, (k,), gen)
        ys = [torch.empty(r, device="cuda", dtype=torch.float32) for r in ns]
        jobs = [gh.jobs([(w, None, y, r) for w, y, r in zip(wc, ys, ns)]) for wc in ws]
        shapes.append(dict(name=name, n=list(ns), k=k, copies=copies, w=ws, x=x, y=ys,
                           jobs=jobs, f32=True, bytes=gemv_f32_bytes(n, k)))
    return shapes


def sweep_graph(torch, gh, shapes, nsteps=ROT_STEPS):
    def steps(stream):
        for step in range(nsteps):
            for sh in shapes:
                launch_gemv(gh, sh, step, stream)
    return capture(torch, steps)


class StepRunner:
    """Replays exactly k sweep steps: k // ROT_STEPS replays of the
    ROT_STEPS-step graph, then one graph of the remaining steps (captured on
    first use)."""

    def __init__(self, torch, gh, shapes):
        self.torch, self.gh, self.shapes = torch, gh, shapes
        self.graphs = {ROT_STEPS: sweep_graph(torch, gh, shapes)}

    def run(self, k):
        for _ in range(k // ROT_STEPS):
            self.graphs[ROT_STEPS].replay()
        r = k % ROT_STEPS
        if r:
            if r not in self.graphs:
                self.graphs[r] = sweep_graph(self.torch, self.gh, self.shapes, r)
            self.graphs[r].replay()


def per_gemv(torch, gh, shapes, timer, busy, reps):
    """Average launch duration of each sweep shape: `reps` back-to-back
    launches over distinct, cold weight copies (after a busy prefix that also
    evicts the caches), timed with HIP events."""
    out = {}
    stream = torch.cuda.current_stream().cuda_stream
    for sh in shapes:
        launches = min(reps, max(sh["copies"], 4))

        def run():
            for i in range(launches):
                launch_gemv(gh, sh, i, stream)

        run()
        med = statistics.median(timer.elapsed_ms(run, busy) for _ in range(TIMING_RUNS)) / launches
        out[sh["name"]] = dict(n=sh["n"], k=sh["k"], us=round(med * 1e3, 3),
                               gbs=round(sh["bytes"] / (med * 1e-3) / 1e9, 1),
                               copies=sh["copies"])
    return out


def bench_gemm(torch, gh, gen, timer, reps):
    out = {}
    stream = torch.cuda.current_stream().cuda_stream
    for name, m, n, k in GEMM_SHAPES:
        a = rand_i8(torch, (m, k), gen)
        asc = rand_scales(torch, m, gen)
        b = rand_i8(torch, (n, k), gen)
        bsc = rand_scales(torch, n, gen)
        d = torch.empty((m, n), device="cuda", dtype=torch.float32)

        def run():
            for _ in range(reps):
                gh.matmul(d, n, b, k, bsc, a, k, asc, m, n, k, stream)

        run()
        ms = statistics.median(timer.elapsed_ms(run) for _ in range(TIMING_RUNS)) / reps
        tops = gemm_ops(m, n, k) / (ms * 1e-3) / 1e12
        out[name] = dict(m=m, n=n, k=k, us=round(ms * 1e3, 2), tops=round(tops, 1),
                         frac=round(tops / INT8_PEAK_TOPS, 4))
        del a, b, d
    # SigLIP patch embedding (gemma.c:4411-4448): fp32 im2col + GEMM, 896 px, P = 14
    img_px, psize, dim = 896, 14, 1152
    npatch, kdim = (img_px // psize) ** 2, 3 * psize * psize
    img = torch.rand((img_px, img_px, 3), generator=gen, device="cuda") * 2 - 1
    pe = torch.randn((dim, kdim), generator=gen, device="cuda") * 0.02
    pe_b = torch.randn(dim, generator=gen, device="cuda") * 0.02
    emb = torch.empty((npatch, dim), device="cuda")

    def run_pe():
        for _ in range(reps):
            gh.patch_embed(emb, img, pe, pe_b, img_px, psize, dim, None, stream)

    run_pe()
    ms = statistics.median(timer.elapsed_ms(run_pe) for _ in range(TIMING_RUNS)) / reps
    tflops = 2 * npatch * dim * kdim / (ms * 1e-3) / 1e12
    patch = dict(img_px=img_px, psize=psize, dim=dim, us=round(ms * 1e3, 2),
                 tflops=round(tflops, 1), frac_fp32=round(tflops / FP32_PEAK_TFLOPS, 4))
    groups = {"siglip_patch_embed_f32": patch}
    for prefix in ("4b", "siglip"):
        ops = sum(gemm_ops(v["m"], v["n"], v["k"]) * GEMM_COUNTS[kk]
                  for kk, v in out.items() if kk.startswith(prefix))
        us = sum(v["us"] * GEMM_COUNTS[kk] for kk, v in out.items() if kk.startswith(prefix))
        tops = ops / (us * 1e-6) / 1e12
        groups[prefix + "_layer"] = dict(tops=round(tops, 1), frac=round(tops / INT8_PEAK_TOPS, 4))
    return dict(peak_tops=INT8_PEAK_TOPS, shapes=out, **groups)


def bench_gemm_f32(torch, gh, gen, timer, reps):
    """The fp32 GEMM (gemm_fpx, gemma.c:3304-3399; 'U' model files) at the
    gemma-3-4b prefill shapes, TFLOP/s of fp32 work against the bound of the
    kernel that runs: the split-bf16 one (the library's default) spends six
    bf16 MFMA products per fp32 multiply-add, so its bound is a sixth of the
    bf16 peak; the fp32-MFMA one (GEMMA_HIP_GEMM_F32=mfma) is bound by the
    fp32 matrix peak."""
    split = os.environ.get("GEMMA_HIP_GEMM_F32") != "mfma"
    peak = BF16_PEAK_TFLOPS / 6 if split else FP32_PEAK_TFLOPS
    out = {}
    stream = torch.cuda.current_stream().cuda_stream
    for name, m, n, k in GEMM_SHAPES[:5]:
        a = torch.randn((m, k), generator=gen, device="cuda")
        b = torch.randn((n, k), generator=gen, device="cuda") * 0.02
        d = torch.empty((m, n), device="cuda", dtype=torch.float32)

        def run():
            for _ in range(reps):
                gh.matmul_f32(d, n, b, k, a, k, m, n, k, stream)

        run()
        ms = statistics.median(timer.elapsed_ms(run) for _ in range(TIMING_RUNS)) / reps
        tf = gemm_ops(m, n, k) / (ms * 1e-3) / 1e12
        out[name] = dict(m=m, n=n, k=k, us=round(ms * 1e3, 2), tflops=round(tf, 1),
                         frac=round(tf / peak, 4))
        del a, b, d
    return {"kernel": "split-bf16" if split else "fp32-mfma", "peak_tflops": round(peak, 1),
            "shapes": out}


def bench_decode_1b(torch, gh, gen, timer, tokens):
    """The W8A8 matmul path of one gemma-3-1b decode token, device-resident:
    per layer quantize+{q,k,v} (one launch), quantize+o, quantize+{gate,up}
    (one launch), quantize+down; then quantize+LM head."""
    c = DEC_1B
    x_dim = outlier_acts(torch, (c["dim"],), gen)
    x_q = outlier_acts(torch, (c["q"],), gen)
    x_mlp = outlier_acts(torch, (c["mlp"],), gen)
    bufs = {n: torch.empty(sz, device="cuda") for n, sz in
            (("q", c["q"]), ("k", c["kv"]), ("v", c["kv"]), ("o", c["dim"]),
             ("g", c["mlp"]), ("u", c["mlp"]), ("d", c["dim"]), ("logits", c["vocab"]))}
    layers = []
    total_bytes = 0
    for _ in range(c["layers"]):
        w = {}
        for name, n, k in (("q", c["q"], c["dim"]), ("k", c["kv"], c["dim"]),
                           ("v", c["kv"], c["dim"]), ("o", c["dim"], c["q"]),
                           ("g", c["mlp"], c["dim"]), ("u", c["mlp"], c["dim"]),
                           ("d", c["dim"], c["mlp"])):
            w[name] = (rand_i8(torch, (n, k), gen), rand_scales(torch, n, gen), n)
        qkv = gh.jobs([(w[t][0], w[t][1], bufs[t], w[t][2]) for t in "qkv"])
        o = gh.jobs([(w["o"][0], w["o"][1], bufs["o"], w["o"][2])])
        gu = gh.jobs([(w[t][0], w[t][1], bufs[t], w[t][2]) for t in "gu"])
        d = gh.jobs([(w["d"][0], w["d"][1], bufs["d"], w["d"][2])])
        layers.append((w, [(qkv, x_dim, c["dim"]), (o, x_q, c["q"]), (gu, x_dim, c["dim"]),
                           (d, x_mlp, c["mlp"])]))
        total_bytes += (gemv_bytes(c["q"] + 2 * c["kv"], c["dim"])
                        + gemv_bytes(c["dim"], c["q"])
                        + gemv_bytes(2 * c["mlp"], c["dim"])
                        + gemv_bytes(c["dim"], c["mlp"]))
    emb = rand_i8(torch, (c["vocab"], c["dim"]), gen)
    emb_s = rand_scales(torch, c["vocab"], gen)
    head = gh.jobs([(emb, emb_s, bufs["logits"], c["vocab"])])
    total_bytes += gemv_bytes(c["vocab"], c["dim"])

    def token(stream):
        for _, calls in layers:
            for (arr, nj), x, k in calls:
                rc = gh.lib.gemma_hip_quantize_matmul(arr, nj, x.data_ptr(), k, None, None,
                                                      stream)
                if rc != 0:
                    raise RuntimeError(gh.lib.gemma_hip_last_error().decode())
        rc = gh.lib.gemma_hip_quantize_matmul(head[0], head[1], x_dim.data_ptr(), c["dim"],
                                              None, None, stream)
        if rc != 0:
            raise RuntimeError(gh.lib.gemma_hip_last_error().decode())

    graph = capture(torch, token)
    for _ in range(5):
        graph.replay()

    def run():
        for _ in range(tokens):
            graph.replay()

    ms = statistics.median(timer.elapsed_ms(run) for _ in range(TIMING_RUNS)) / tokens
    return dict(tok_s=round(1e3 / ms, 1), ms_per_token=round(ms, 4),
                bytes_per_token=total_bytes,
                gbs=round(total_bytes / (ms * 1e-3) / 1e9, 1),
                launches_per_token=4 * c["layers"] + 1,
                what="W8A8 matmul path of one decode token (fused quantize+GEMV launches, "
                     "HIP graph); attention/norms/RoPE are outside this path")


# decode phases of BASELINE.json configs 3 and 5: (model, context before, timed steps)
# BASELINE.json configs 1, 3 and 5: (model, prompt tokens, greedy decode steps)
# name[:U] (":U": an unquantized fp32 model file), prompt tokens, decode steps
DECODER_RUNS = (("gemma-3-270m", 32, 64), ("gemma-3-1b", 512, 256), ("gemma-3-4b", 2048, 512),
                ("gemma-3-1b:U", 512, 256))


def bench_decoder(torch, gh, name: str, prompt: int, steps: int) -> dict:
    """The prompt and the greedy decode fully on the GPU: `prompt` random token
    ids go through the batched prefill (gemma_hip_decoder_prefill; the median
    of TIMING_RUNS calls after a warm-up call that allocates its row buffers,
    with the attention on the fp32 matrix cores, the default, and on the fp64
    ones, the verification mode), then `steps` decode steps from the KV cache
    the default prefill filled are timed (one HIP graph launch each, tokens fed back on the device, one
    readback at the end; the median of TIMING_RUNS generations)."""
    import statistics
    import time

    import numpy as np

    import model_bin

    base, _, kind = name.partition(":")
    quant = kind != "U"
    model = model_bin.synth_model(base, seed=1234, quant=quant)
    c = model["config"]
    ids = np.random.default_rng(1234).integers(0, c["nvocab"], prompt).astype(np.int32)
    dec = gh.decoder(model, prompt + steps + 1)
    try:
        dec.prefill(ids, 0)
        torch.cuda.synchronize()
        t_mode = {}
        for mode in (dec.ATTN_F64, dec.ATTN_F32):  # the default last: its cache is decoded
            dec.set_attention(mode)
            ts = []
            for _ in range(TIMING_RUNS):
                t0 = time.perf_counter()
                first = dec.prefill(ids, 0)
                ts.append(time.perf_counter() - t0)
            t_mode[mode] = statistics.median(ts)
        t_pf, t_pf64 = t_mode[dec.ATTN_F32], t_mode[dec.ATTN_F64]
        # the median of TIMING_RUNS generations, each from the same cache
        # state (the steps overwrite the positions after the prompt)
        runs = []
        for _ in range(TIMING_RUNS):
            t0 = time.perf_counter()
            toks = dec.generate(first, prompt, steps)
            runs.append(time.perf_counter() - t0)
        t_gen = statistics.median(runs)
    finally:
        dec.close()
    q_sz, kv_sz = c["n_heads"] * c["hdim"], c["nkv"] * c["hdim"]
    pf_ops = c["nl"] * (gemm_ops(prompt, q_sz + 2 * kv_sz, c["dim"])
                        + gemm_ops(prompt, c["dim"], q_sz)
                        + gemm_ops(prompt, 2 * c["mlp_dim"], c["dim"])
                        + gemm_ops(prompt, c["dim"], c["mlp_dim"]))
    prefill = dict(tokens=prompt, ms=round(1e3 * t_pf, 3), tok_s=round(prompt / t_pf, 1),
                   ms_attn_f64=round(1e3 * t_pf64, 3), tok_s_attn_f64=round(prompt / t_pf64, 1))
    if quant:
        prefill.update(int8_tops=round(pf_ops / t_pf / 1e12, 1),
                       int8_frac=round(pf_ops / t_pf / 1e12 / INT8_PEAK_TOPS, 4))
    else:  # the fp32 GEMMs (split-bf16 by default: bound a sixth of the bf16 peak)
        split = os.environ.get("GEMMA_HIP_GEMM_F32") != "mfma"
        peak = BF16_PEAK_TFLOPS / 6 if split else FP32_PEAK_TFLOPS
        prefill.update(fp32_tflops=round(pf_ops / t_pf / 1e12, 1),
                       fp32_frac=round(pf_ops / t_pf / 1e12 / peak, 4))
    gb = gemv_bytes if quant else gemv_f32_bytes
    per_layer = (gb(q_sz + 2 * kv_sz, c["dim"]) + gb(c["dim"], q_sz)
                 + gb(2 * c["mlp_dim"], c["dim"]) + gb(c["dim"], c["mlp_dim"]))
    weights = c["nl"] * per_layer + gb(c["nvocab"], c["dim"])
    kv = 0
    for pos in range(prompt, prompt + steps):
        for sw in c["swa"]:
            keys = min(pos + 1, c["slide"]) if sw else pos + 1
            kv += 2 * kv_sz * 4 * keys
    per_token = weights + kv / steps
    tok_s = steps / t_gen
    gbs = per_token * tok_s / 1e9
    return dict(model=name, context=f"{prompt}->{prompt + steps}", prefill=prefill,
                tok_s=round(tok_s, 1),
                ms_per_token=round(1e3 * t_gen / steps, 4), bytes_per_token=int(per_token),
                gbs=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK_GBS, 4),
                hbm_bound_tok_s=round(HBM_PEAK_GBS * 1e9 / per_token, 1),
                distinct_tokens=int(len(set(toks.tolist()))))


def bench_vision(torch, gh) -> dict:
    """BASELINE.json config 4 end to end on the GPU: one 896x896 image through
    the whole SigLIP tower (gemma_hip_vision_forward: patch and position
    embedding, 27 encoder layers, post norm, pooling to 256 tokens, RMSNorm,
    projection to the gemma-3-4b width), random weights of that shape; the
    median of five timed images after one untimed, with the attention on the
    fp32 matrix cores (the default) and on the fp64 matrix cores (the
    verification mode, equal to the fp64 oracle; gemma_hip_vision_set_attention);
    then the same tower from fp32 weights (an unquantized 'U' file:
    gemma_hip_vision_create_f32, fp32 GEMMs on the split-bf16 kernel)."""
    import statistics
    import time

    import model_bin

    vis = model_bin.synth_vision(seed=1234, text_dim=2560)
    img = model_bin.synth_image(vis["config"]["img_px"], seed=1234)
    c = vis["config"]
    ms = {}

    def timed(tower, name):
        tower.forward(img)
        ts = []
        for _ in range(TIMING_RUNS):
            t0 = time.perf_counter()
            tower.forward(img)
            ts.append(time.perf_counter() - t0)
        ms[name] = statistics.median(ts) * 1e3

    tower = gh.vision(vis)
    try:
        for name, mode in (("f64", tower.ATTN_F64), ("f32", tower.ATTN_F32)):
            tower.set_attention(mode)
            timed(tower, name)
    finally:
        tower.close()
    del vis
    tower = gh.vision(model_bin.synth_vision(seed=1234, text_dim=2560, quant=False))
    try:
        timed(tower, "u")
    finally:
        tower.close()
    n = (c["img_px"] // c["psize"]) ** 2
    ops = c["nl"] * (4 * gemm_ops(n, c["dim"], c["dim"]) + gemm_ops(n, c["mlp_dim"], c["dim"])
                     + gemm_ops(n, c["dim"], c["mlp_dim"])) \
        + gemm_ops(c["img_tok"], c["text_dim"], c["dim"])
    return dict(model="siglip (27 layers, 896 px, 4096 patches -> 256 tokens)",
                ms_per_image=round(ms["f32"], 2), images_s=round(1e3 / ms["f32"], 2),
                ms_per_image_attn_f64=round(ms["f64"], 2),
                int8_ops=ops, int8_tops_over_tower=round(ops / ms["f32"] / 1e9, 1),
                ms_per_image_u=round(ms["u"], 2),
                fp32_tflops_over_tower_u=round(ops / ms["u"] / 1e9, 1))


def measured_traffic(kernel: str) -> dict | None:
    """HBM bytes per launch of the LM-head GEMV from the committed rocprofv3
    --pmc measurement (FETCH_SIZE and WRITE_SIZE, each scaled by what the
    counter reads for a copy of known size)."""
    path = os.path.join(REPO, "profiles", "gemv_i8_lm_head_1b.hbm_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    return d if d.get("kernel") == kernel else None


def host_description() -> dict:
    """The host the CPU baseline ran on: lscpu's model, sockets and cores,
    and the compilers' versions."""
    def first_line(cmd):
        try:
            return subprocess.run(cmd, capture_output=True, text=True,
                                  timeout=20).stdout.splitlines()[0].strip()
        except (OSError, IndexError, subprocess.SubprocessError):
            return None
    info = {"nproc": os.cpu_count(), "machine": platform.machine()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip() in ("Model name", "Socket(s)", "Core(s) per socket",
                               "Thread(s) per core", "CPU(s)"):
                info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    info["gcc"] = first_line(["gcc", "--version"])
    info["clang"] = first_line(["/opt/rocm/llvm/bin/clang", "--version"])
    return info


def cpu_baseline(threads: int, seconds_per_shape: float) -> dict | None:
    """The reference's own quantize_act + gemv_int8 (compiled from
    /root/reference/gemma.c by oracle/Makefile; AVX2 clang build) over the
    same sweep shapes and rotation, on `threads` host cores."""
    from oracle.oracle import RefHarness

    if not RefHarness.available("clang"):
        return None
    ref = RefHarness("clang")
    total_bytes, total_s, parts = 0, 0.0, {}
    for name, ns, k in SWEEP_1B:
        n = sum(ns)
        copies = max(2, math.ceil(ROTATE_BYTES / (n * k)))
        est = gemv_bytes(n, k) / 30e9  # rough per-call time, sizes the sample
        calls = max(4, int(seconds_per_shape / est))
        if len(ns) == 1:
            r = ref.bench(["gemv_int8", n, k, copies, calls], threads)
        else:
            r = ref.bench(["gemv_int8_multi", k, copies, calls, len(ns), *ns], threads)
        per_call = r["seconds"] / r["calls"]
        parts[name] = round(gemv_bytes(n, k) / per_call / 1e9, 2)
        total_bytes += gemv_bytes(n, k)
        total_s += per_call
    return dict(value=round(total_bytes / total_s / 1e9, 2), unit="GB/s", cores=threads,
                kind="reference", host=host_description(),
                compiler_note=("clang -O3 -ffast-math -march=x86-64-v3 -fopenmp builds the "
                               "reference's AVX2 path unmodified; the reference Makefile's gcc "
                               "-O3 -ffast-math -march=native needs _mm256_dpbssd_epi32 "
                               "(gemma.c:3741-3800, gcc >= 13), which this image's gcc lacks, "
                               "and no stand-in for it is written"),
                sample=(f"reference quantize_act + gemv_int8 / gemv_int8_multi (gemma.c:2590, "
                        f"2770, 2808) built by clang -O3 -ffast-math -march=x86-64-v3 -fopenmp, "
                        f"{threads} OpenMP threads, the same {len(SWEEP_1B)} launches, >=512 MB "
                        f"weight rotation, ~{seconds_per_shape:.1f} s per launch shape"),
                per_gemv_gbs=parts)


def perf_report(torch, gh, decoder_runs) -> str:
    """The reference's per-op report (PerfBench) for the device-resident
    paths: each decoder model's prompt pass and decode steps (one prefill of
    the prompt, then the steps, eagerly so that each launch is timed), and one
    896 px image through the SigLIP tower.  Each launch's GPU time comes from
    HIP events around it, so the event pairs add a little to each total."""
    import numpy as np

    import gemma_hip
    import model_bin

    out = []
    for name, prompt, steps in decoder_runs:
        base, _, kind = name.partition(":")
        model = model_bin.synth_model(base, seed=1234, quant=kind != "U")
        ids = np.random.default_rng(1234).integers(0, model["config"]["nvocab"],
                                                   prompt).astype(np.int32)
        dec = gh.decoder(model, prompt + steps + 1)
        try:
            first = dec.prefill(ids, 0)
            dec.generate(first, prompt, 4)
            gh.perf_enable(True)
            try:
                first = dec.prefill(ids, 0)
                dec.generate(first, prompt, steps)
                perf = gh.perf_read()
            finally:
                gh.perf_enable(False)
        finally:
            dec.close()
        out.append(f"== {name}: prefill {prompt} tokens, decode {steps} steps ==")
        out.append(gemma_hip.perf_table(perf))
    vis = model_bin.synth_vision(seed=1234, text_dim=2560)
    img = model_bin.synth_image(vis["config"]["img_px"], seed=1234)
    tower = gh.vision(vis)
    try:
        tower.forward(img)
        gh.perf_enable(True)
        try:
            tower.forward(img)
            perf = gh.perf_read()
        finally:
            gh.perf_enable(False)
    finally:
        tower.close()
    out.append("== siglip: one 896 px image ==")
    out.append(gemma_hip.perf_table(perf))
    torch.cuda.synchronize()
    return "\n".join(out)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=2.0,
                    help="CPU-baseline sample time per sweep shape")
    ap.add_argument("--only", choices=["sweep", "lm_head", "decoder", "vision", "gemm", "f32"],
                    default=None,
                    help="profiling aid: run just the timed sweep, the LM-head timing, "
                         "the device-resident decoder, the vision tower or the GEMM shapes")
    ap.add_argument("--decoder-models",
                    default="gemma-3-270m,gemma-3-1b,gemma-3-4b,gemma-3-1b:U",
                    help="models of the decoder timing (comma list of gemma-3-270m, "
                         "gemma-3-1b, gemma-3-4b, gemma-3-1b:U; ':U' an fp32 model)")
    ap.add_argument("--perf-report", action="store_true",
                    help="print the reference's per-op report (PerfBench names) of the "
                         "decoder models and the vision tower, then exit")
    ap.add_argument("--copy-probe", action="store_true",
                    help="profiling aid: 3 dispatches of an elementwise kernel that reads "
                         "and writes exactly 1 GiB (calibrates FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1:
        print("bench.py: this build targets one GPU; the W8A8 matmul path has no "
              "multi-GPU part (collectives and sharding are design-only), so --gpus "
              f"{args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch

    import gemma_hip

    if args.copy_probe:
        src = torch.ones(1 << 30, dtype=torch.int8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print("copy probe: 3 x neg over 1 GiB int8", flush=True)
        return 0

    gh = gemma_hip.GemmaHip(0)
    decoder_runs = [r for r in DECODER_RUNS if r[0] in args.decoder_models.split(",")]
    if args.perf_report:
        print(perf_report(torch, gh, decoder_runs), flush=True)
        gh.close()
        return 0
    if args.only == "decoder":
        for name, prompt, nsteps in decoder_runs:
            print(json.dumps(bench_decoder(torch, gh, name, prompt, nsteps)), flush=True)
        gh.close()
        return 0
    if args.only == "vision":
        print(json.dumps(bench_vision(torch, gh)), flush=True)
        gh.close()
        return 0
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    timer = Timer(torch)
    if args.only == "gemm":
        print(json.dumps(bench_gemm(torch, gh, gen, timer, reps=10)), flush=True)
        gh.close()
        return 0
    if args.only == "f32":
        stream = torch.cuda.current_stream().cuda_stream
        shapes_f32 = build_sweep_f32(torch, gh, gen)
        lm_f32 = shapes_f32[-1]

        def busy_f32():
            for i in range(2):
                launch_gemv(gh, lm_f32, i, stream)

        print(json.dumps({"per_gemv_f32": per_gemv(torch, gh, shapes_f32, timer, busy_f32,
                                                    reps=16),
                          "gemm_f32": bench_gemm_f32(torch, gh, gen, timer, reps=5)}),
              flush=True)
        gh.close()
        return 0
    shapes = build_sweep(torch, gh, gen)
    step_bytes = sum(sh["bytes"] for sh in shapes)
    lm = shapes[-1]
    stream = torch.cuda.current_stream().cuda_stream

    def busy():
        for i in range(8):
            launch_gemv(gh, lm, i, stream)

    if args.only == "lm_head":
        per = per_gemv(torch, gh, [lm], timer, busy, reps=8)
        print(json.dumps(per), flush=True)
        return 0

    # exactly --warmup untimed steps, then regions of exactly --steps steps,
    # each bracketed by synchronisations and timed with HIP events, repeated
    # until MIN_TIMED_MS have been timed (at least 5); the median region counts
    steps = max(1, args.steps)
    runner = StepRunner(torch, gh, shapes)
    runner.run(max(0, args.warmup))
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    regions = []
    while len(regions) < 5 or (sum(regions) < MIN_TIMED_MS and len(regions) < 100000):
        torch.cuda.synchronize()
        start.record()
        runner.run(steps)
        end.record()
        torch.cuda.synchronize()
        regions.append(start.elapsed_time(end))
    ms = statistics.median(regions)
    value = step_bytes * steps / (ms * 1e-3) / 1e9
    print(f"# sweep: {len(regions)} regions of {steps} steps, median {ms:.3f} ms -> "
          f"{value:.1f} GB/s", file=sys.stderr, flush=True)
    if args.only == "sweep":
        return 0

    per = per_gemv(torch, gh, shapes, timer, busy, reps=64)
    print(f"# per-gemv: {json.dumps(per)}", file=sys.stderr, flush=True)
    del runner, shapes
    torch.cuda.empty_cache()
    shapes_4b = build_sweep(torch, gh, gen, SWEEP_4B)
    per_4b = per_gemv(torch, gh, shapes_4b, timer, busy, reps=16)
    per_4b["all"] = dict(
        us=round(sum(v["us"] for v in per_4b.values()), 3),
        gbs=round(sum(sh["bytes"] for sh in shapes_4b)
                  / (sum(v["us"] for v in per_4b.values()) * 1e-6) / 1e9, 1))
    print(f"# per-gemv 4b: {json.dumps(per_4b)}", file=sys.stderr, flush=True)
    del shapes_4b
    torch.cuda.empty_cache()
    gemm = bench_gemm(torch, gh, gen, timer, reps=10)
    print(f"# gemm: {json.dumps(gemm)}", file=sys.stderr, flush=True)
    shapes_f32 = build_sweep_f32(torch, gh, gen)
    per_f32 = per_gemv(torch, gh, shapes_f32, timer, busy, reps=16)
    print(f"# per-gemv fp32: {json.dumps(per_f32)}", file=sys.stderr, flush=True)
    del shapes_f32
    torch.cuda.empty_cache()
    gemm_f32 = bench_gemm_f32(torch, gh, gen, timer, reps=5)
    print(f"# gemm fp32: {json.dumps(gemm_f32)}", file=sys.stderr, flush=True)
    dec = bench_decode_1b(torch, gh, gen, timer, tokens=50)
    print(f"# decode_1b: {json.dumps(dec)}", file=sys.stderr, flush=True)
    decoder = {}
    for name, prompt, nsteps in decoder_runs:
        decoder[name] = bench_decoder(torch, gh, name, prompt, nsteps)
        print(f"# decoder: {json.dumps(decoder[name])}", file=sys.stderr, flush=True)

    vision = bench_vision(torch, gh)
    print(f"# vision: {json.dumps(vision)}", file=sys.stderr, flush=True)

    lm_us = per["lm_head"]["us"]
    traffic = measured_traffic(LM_KERNEL)
    achieved = lm["bytes"] / (lm_us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        threads = min(16, os.cpu_count() or 1)
        cpu = cpu_baseline(threads, args.cpu_seconds)
        print(f"# cpu_baseline: {json.dumps(cpu)}", file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": max(0, args.warmup),
        "ms_per_step": round(ms / steps, 5),
        "timing": {"regions": len(regions), "timed_ms_total": round(sum(regions), 3),
                   "region_ms_median": round(ms, 4), "region_ms_min": round(min(regions), 4),
                   "region_ms_max": round(max(regions), 4),
                   "what": "value from the median of the timed regions, each exactly "
                           "`steps` steps between synchronisations"},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE.json config 2: W8A8 GEMV sweep at gemma-3-1b shapes, M=1, "
                        "as the reference's decode call sites issue it (q/k/v 1152->1024+256+256 "
                        "as one multi-job launch, o 1024->1152, gate/up 1152->2x6912 as one "
                        "multi-job launch, down 6912->1152, LM head 1152->262144), fp32 "
                        "activations quantized in-kernel, weights rotated through >256 MB of "
                        "copies",
            "step_bytes": step_bytes,
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": LM_KERNEL + " (LM head launch, 262144x1152)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "avg_launch_us": lm_us,
            "bytes_per_launch": lm["bytes"],
            "traffic": traffic["traffic_bytes"] if traffic else None,
            "traffic_source": ("profiles/gemv_i8_lm_head_1b.hbm_traffic.json (rocprofv3 --pmc "
                               "FETCH_SIZE x%.3f + WRITE_SIZE x%.3f)"
                               % (traffic["fetch_scale"], traffic["write_scale"])
                               if traffic else None),
        },
        "per_gemv": per,
        "per_gemv_4b": per_4b,
        "gemm": gemm,
        "per_gemv_f32": per_f32,
        "gemm_f32": gemm_f32,
        "decode_1b": dec,
        "decoder": decoder,
        "vision": vision,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    torch.cuda.synchronize()
    gh.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
