"""GPU parity of the HIP library against the oracle and the reference's
golden fixtures, every call through the C ABI (include/gemma_hip.h).

Bar: bit-exact int8 activations, scales, int32 sums (observed through the
rescale, which is itself bit-exact) and fp32 outputs for the W8A8 path; for
the fp32 fallback |y - y_exact| <= 1e-5 * sum|a*b| (TOL_F32).
GEMM products are compared cell for cell at every size: the oracle forms the
exact int32 sums of a large product with a float64 matrix product (exact for
int8 operands, test_oracle.py pins it) and rescales each cell itself.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle as om

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.int32)


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def outlier_acts(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32)
    x[..., rng.random(shape[-1]) < 0.01] *= 20.0
    return x


# --------------------------------------------------------------- quantize
def test_quantize_golden(gh, golden):
    g = golden("quantize_act")
    bounds = np.concatenate([[0], np.cumsum(g["lens"])])
    for i in range(len(g["lens"])):
        vec = g["vec"][bounds[i]:bounds[i + 1]]
        n = len(vec)
        note(f"quantize golden case {i} n={n}")
        src = dev(vec)
        q = torch.empty(n, dtype=torch.int8, device="cuda")
        s = torch.empty(1, dtype=torch.float32, device="cuda")
        gh.quantize(q, s, src, n, 1, n, stream())
        assert np.array_equal(host(q), g["q_gcc"][bounds[i]:bounds[i + 1]]), f"case {i}"
        assert bits(host(s))[0] == bits(g["scale_gcc"][i]), f"case {i}"


def test_quantize_strided_golden(gh, golden):
    g = golden("quantize_acts")
    m, sstr = g["src"].shape
    n = int(g["n"])
    q = torch.empty((m, n), dtype=torch.int8, device="cuda")
    s = torch.empty(m, dtype=torch.float32, device="cuda")
    gh.quantize(q, s, dev(g["src"]), sstr, m, n, stream())
    assert np.array_equal(host(q), g["q"])
    assert np.array_equal(bits(host(s)), bits(g["scale"]))


@pytest.mark.parametrize("m,n", [(4096, 1152), (4096, 4304), (512, 6912), (3, 13)])
def test_quantize_rows_vs_oracle(gh, oracle, m, n):
    note(f"quantize rows m={m} n={n}")
    rng = np.random.default_rng(m + n)
    x = outlier_acts(rng, (m, n))
    q = torch.empty((m, n), dtype=torch.int8, device="cuda")
    s = torch.empty(m, dtype=torch.float32, device="cuda")
    gh.quantize(q, s, dev(x), n, m, n, stream())
    qo, so = oracle.quantize_acts(x)
    assert np.array_equal(host(q), qo)
    assert np.array_equal(bits(host(s)), bits(so))


# --------------------------------------------------------------- GEMV
def test_gemv_golden(gh, golden):
    g = golden("gemv_int8")
    n, k = g["mat"].shape
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    gh.matmul(y, 0, dev(g["mat"]), 0, dev(g["matsc"]), dev(g["xq"]), 0,
              dev(np.array([g["xs"]], np.float32)), 1, n, k, stream())
    assert np.array_equal(bits(host(y)), bits(g["y_gcc"]))


def test_quantize_matmul_golden(gh, golden):
    """fp32 x quantized inside the GEMV kernel (the decode call sites)."""
    g = golden("gemv_int8")
    n, k = g["mat"].shape
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    xq = torch.empty(k, dtype=torch.int8, device="cuda")
    xs = torch.empty(1, dtype=torch.float32, device="cuda")
    gh.quantize_matmul([(dev(g["mat"]), dev(g["matsc"]), y, n)], dev(g["x"]), k, xq, xs,
                       stream())
    assert np.array_equal(host(xq), g["xq"])
    assert bits(host(xs))[0] == bits(g["xs"])
    assert np.array_equal(bits(host(y)), bits(g["y_gcc"]))


def test_gemv_multi_golden(gh, golden):
    g = golden("gemv_int8_multi")
    k = g["xq"].shape[0]
    outs, specs = [], []
    for j in range(3):
        rows = g[f"w{j}"].shape[0]
        outs.append(torch.empty(rows, dtype=torch.float32, device="cuda"))
        specs.append((dev(g[f"w{j}"]), dev(g[f"s{j}"]), outs[-1], rows))
    gh.matmul_multi(specs, dev(g["xq"]), dev(np.array([g["xs"]], np.float32)), k, stream())
    y = np.concatenate([host(o) for o in outs])
    assert np.array_equal(bits(y), bits(g["y"]))


# the gemma-3-1b decode GEMVs (out rows, in K)
SWEEP_1B = [("q", 1024, 1152), ("k", 256, 1152), ("v", 256, 1152), ("o", 1152, 1024),
            ("gate", 6912, 1152), ("up", 6912, 1152), ("down", 1152, 6912),
            ("lm_head", 262144, 1152)]


@pytest.mark.parametrize("name,n,k", SWEEP_1B)
def test_gemv_sweep_1b_vs_oracle(gh, oracle, name, n, k):
    note(f"gemv sweep {name} n={n} k={k}")
    rng = np.random.default_rng(1234 + n + k)
    W = rng.integers(-127, 128, (n, k), dtype=np.int8)
    ws = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    x = outlier_acts(rng, (k,))
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    xq = torch.empty(k, dtype=torch.int8, device="cuda")
    xs = torch.empty(1, dtype=torch.float32, device="cuda")
    gh.quantize_matmul([(dev(W), dev(ws), y, n)], dev(x), k, xq, xs, stream())
    qo, so = oracle.quantize_act(x)
    yo, _ = oracle.gemv_int8(W, ws, qo, so)
    assert np.array_equal(host(xq), qo)
    assert bits(host(xs))[0] == bits(so)
    assert np.array_equal(bits(host(y)), bits(yo))


# The gemma-3-4b decode launches (config 5) as the decode call sites issue
# them: q/k/v and gate/up fused, o, down and the tied LM head.
@pytest.mark.parametrize("rows,k", [((1024, 256, 256), 1152), ((6912, 6912), 1152),
                                    ((2048, 1024, 1024), 2560), ((10240, 10240), 2560),
                                    ((2560,), 2048), ((2560,), 10240), ((262144,), 2560),
                                    ((40, 3, 17, 64), 656)])
def test_fused_multi_vs_oracle(gh, oracle, rows, k):
    """q/k/v and gate/up as one launch (gemma.c:4768-4773, 4911-4915), and
    the single-job launches at the 4b widths (4858-4859, 4929-4930,
    4964-4965)."""
    note(f"fused multi rows={rows} k={k}")
    rng = np.random.default_rng(sum(rows) + k)
    x = outlier_acts(rng, (k,))
    qo, so = oracle.quantize_act(x)
    specs, outs, refs = [], [], []
    for r in rows:
        W = rng.integers(-127, 128, (r, k), dtype=np.int8)
        ws = rng.uniform(1e-3, 1e-2, r).astype(np.float32)
        outs.append(torch.empty(r, dtype=torch.float32, device="cuda"))
        specs.append((dev(W), dev(ws), outs[-1], r))
        refs.append(oracle.gemv_int8(W, ws, qo, so)[0])
    gh.quantize_matmul(specs, dev(x), k, None, None, stream())
    for o, r in zip(outs, refs):
        assert np.array_equal(bits(host(o)), bits(r))


# Above 2048 rows (and below 4096-byte rows) the GEMV streams row groups of one
# job per wave with bounds-checked loads; ragged jobs, an empty job and a group
# that ends inside a job exercise the edges of that decomposition.
@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("rows,k", [((3001, 5, 0, 2999), 1152), ((4099, 1), 2560),
                                    ((5000,), 6912), ((2049,), 16)])
def test_stream_ragged_jobs_vs_oracle(gh, oracle, rows, k, fused):
    note(f"stream ragged rows={rows} k={k} fused={fused}")
    rng = np.random.default_rng(sum(rows) * 7 + k)
    x = outlier_acts(rng, (k,))
    qo, so = oracle.quantize_act(x)
    specs, outs, refs = [], [], []
    for r in rows:
        W = rng.integers(-127, 128, (max(r, 1), k), dtype=np.int8)
        ws = rng.uniform(1e-3, 1e-2, max(r, 1)).astype(np.float32)
        outs.append(torch.full((max(r, 1),), 7.0, dtype=torch.float32, device="cuda"))
        specs.append((dev(W), dev(ws), outs[-1], r))
        refs.append(oracle.gemv_int8(W[:r], ws[:r], qo, so)[0])
    if fused:
        gh.quantize_matmul(specs, dev(x), k, None, None, stream())
    else:
        gh.matmul_multi(specs, dev(qo), dev(np.array([so], np.float32)), k, stream())
    for o, r, ref in zip(outs, rows, refs):
        got = host(o)
        assert np.array_equal(bits(got[:r]), bits(ref))
        assert np.all(got[r:] == 7.0)  # nothing written past a job's rows


def test_gemv_unaligned_rows(gh, oracle):
    """k % 16 != 0 and an odd base address take the generic path."""
    rng = np.random.default_rng(5)
    n, k = 37, 1001
    W = rng.integers(-127, 128, (n, k), dtype=np.int8)
    ws = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    x = outlier_acts(rng, (k,))
    buf = torch.zeros(n * k + 1, dtype=torch.int8, device="cuda")
    buf[1:] = torch.from_numpy(W.reshape(-1)).to("cuda")
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    gh.quantize_matmul([(buf.data_ptr() + 1, dev(ws), y, n)], dev(x), k, None, None, stream())
    qo, so = oracle.quantize_act(x)
    assert np.array_equal(bits(host(y)), bits(oracle.gemv_int8(W, ws, qo, so)[0]))


# --------------------------------------------------------------- GEMM
@pytest.mark.parametrize("tag", ["tails", "strided", "m1", "blocks"])
def test_gemm_golden(gh, golden, tag):
    g = golden("gemm_int8")
    m, n, k, ds, ms, ss = (int(v) for v in g[tag + "_shape"])
    dst = dev(np.full((m, ds), -7.0, np.float32))
    gh.matmul(dst, ds, dev(g[tag + "_b"]), ms, dev(g[tag + "_bs"]), dev(g[tag + "_a"]), ss,
              dev(g[tag + "_as"]), m, n, k, stream())
    assert np.array_equal(bits(host(dst)), bits(g[tag + "_dst"]))


GEMM_SHAPES = [
    # (label, M, N, K): prefill at 1b (M=512) and 4b (M=2048), SigLIP (M=4096)
    ("1b_o", 512, 1152, 1024), ("1b_gate", 512, 6912, 1152), ("1b_down", 512, 1152, 6912),
    ("siglip_qkv", 4096, 1152, 1152), ("siglip_fc1", 4096, 4304, 1152),
    ("siglip_fc2", 4096, 1152, 4304), ("siglip_proj", 256, 2560, 1152),
    ("4b_q", 2048, 2048, 2560), ("4b_kv", 2048, 1024, 2560), ("4b_o", 2048, 2560, 2048),
    ("4b_gate", 2048, 10240, 2560), ("4b_down", 2048, 2560, 10240),
    ("tiny", 2, 8, 16), ("odd", 77, 333, 112),
]


def quantized_block(gh, oracle, rng, m, k):
    """m rows of outlier activations quantized on the GPU, checked bit for
    bit against the oracle's quantize_acts; returns (device q, device
    scales, oracle q, oracle scales)."""
    A = outlier_acts(rng, (m, k))
    Aq = torch.empty((m, k), dtype=torch.int8, device="cuda")
    As = torch.empty(m, dtype=torch.float32, device="cuda")
    gh.quantize(Aq, As, dev(A), k, m, k, stream())
    qo, so = oracle.quantize_acts(A)
    assert np.array_equal(host(Aq), qo)
    assert np.array_equal(bits(host(As)), bits(so))
    return Aq, As, qo, so


def assert_same(got, ref, what=""):
    bad = bits(got) != bits(ref)
    if bad.any():
        r, c = np.argwhere(bad)[0]
        raise AssertionError(f"{what}{int(bad.sum())} of {bad.size} cells differ, first at "
                             f"({r}, {c}): {got[r, c]!r} != {ref[r, c]!r}")


@pytest.mark.parametrize("label,m,n,k", GEMM_SHAPES)
def test_gemm_vs_oracle(gh, oracle, label, m, n, k):
    """Every cell of the product against the oracle (exact int32 sums through
    a float64 product, then the oracle's rescale of each cell)."""
    note(f"gemm {label} m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 7 + n + k)
    Aq, As, qo, so = quantized_block(gh, oracle, rng, m, k)
    B = rng.integers(-127, 128, (n, k), dtype=np.int8)
    bs = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    dst = torch.empty((m, n), dtype=torch.float32, device="cuda")
    gh.matmul(dst, n, dev(B), k, dev(bs), Aq, k, As, m, n, k, stream())
    assert_same(host(dst), oracle.gemm_int8_full(B, bs, qo, so))


# The prefill's fused launches over adjacent weight matrices (gemma_hip_matmul_cols):
# gemma-3-4b q/k/v and gate/up at 2048 tokens, gemma-3-1b at 512, SigLIP
# q/k/v, and a ragged split whose inner boundaries suit no tile width.
GEMM_COLS = [
    ("4b_qkv", 2048, (2048, 1024, 1024), 2560), ("4b_gate_up", 2048, (10240, 10240), 2560),
    ("1b_qkv", 512, (1024, 256, 256), 1152), ("1b_gate_up", 512, (6912, 6912), 1152),
    ("siglip_qkv", 4096, (1152, 1152, 1152), 1152), ("ragged", 300, (200, 72, 136), 1040),
]


@pytest.mark.parametrize("label,m,rows,k", GEMM_COLS)
def test_gemm_cols_vs_oracle(gh, oracle, label, m, rows, k):
    note(f"gemm cols {label} m={m} rows={rows} k={k}")
    rng = np.random.default_rng(m + sum(rows) + k)
    Aq, As, qo, so = quantized_block(gh, oracle, rng, m, k)
    Bs = [rng.integers(-127, 128, (r, k), dtype=np.int8) for r in rows]
    bss = [rng.uniform(1e-3, 1e-2, r).astype(np.float32) for r in rows]
    n = sum(rows)
    dst = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    gh.matmul_cols(dst, n, [(dev(B), dev(b), r) for B, b, r in zip(Bs, bss, rows)], Aq, k, As,
                   m, k, stream())
    ref = oracle.gemm_int8_full(np.concatenate(Bs), np.concatenate(bss), qo, so)
    assert_same(host(dst), ref)


# Every configuration of the ping-pong kernel, forced (GEMMA_HIP_GEMM_PP), on
# shapes off its tile grid in M, N and K (K = 1040: the last 64-byte stage
# partial), row-major with a padded stride and head-major, with scales in
# FTZ/DAZ range so the exact-rescale path runs as well as the plain one.
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_gemm_pp_configs(gh, oracle, monkeypatch, cfg):
    monkeypatch.setenv("GEMMA_HIP_GEMM_PP", str(cfg))
    rng = np.random.default_rng(70 + cfg)
    m, n, k, dstr = 300, 700, 1040, 712
    qa = rng.integers(-127, 128, (m, k), dtype=np.int8)
    sa = rng.uniform(1e-3, 1e-2, m).astype(np.float32)
    B = rng.integers(-127, 128, (n, k), dtype=np.int8)
    bs = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    for rep in range(2):
        if rep == 1:  # FTZ products and DAZ (subnormal) scales
            sa[::7] = 1e-36
            bs[3::11] = np.float32(5e-39)
        dst = torch.full((m, dstr), -7.0, dtype=torch.float32, device="cuda")
        gh.matmul(dst, dstr, dev(B), k, dev(bs), dev(qa), k, dev(sa), m, n, k, stream())
        got = host(dst)
        ref, _ = oracle.gemm_int8(B, bs, qa, sa)
        assert_same(got[:, :n], ref, f"config {cfg} rep {rep}: ")
        assert np.all(got[:, n:] == -7.0), "cells past n of the padded stride were written"
    heads, hdim = 3, 256
    Bh = rng.integers(-127, 128, (heads * hdim, k), dtype=np.int8)
    bh = rng.uniform(1e-3, 1e-2, heads * hdim).astype(np.float32)
    dst = torch.full((heads, m, hdim), -7.0, dtype=torch.float32, device="cuda")
    gh.matmul_heads(dst, dev(Bh), dev(bh), dev(qa), dev(sa), m, heads, hdim, k, stream())
    ref, _ = oracle.gemm_int8(Bh, bh, qa, sa)
    ref = np.ascontiguousarray(ref.reshape(m, heads, hdim).transpose(1, 0, 2))
    assert np.array_equal(bits(host(dst)), bits(ref)), f"config {cfg} head-major"


def test_gemm_heads_vs_oracle(gh, oracle):
    """The prefill QKV site's head-major output (gemma.c:5045-5089)."""
    rng = np.random.default_rng(9)
    m, heads, hdim, k = 300, 4, 256, 1152
    A = outlier_acts(rng, (m, k))
    qo, so = oracle.quantize_acts(A)
    B = rng.integers(-127, 128, (heads * hdim, k), dtype=np.int8)
    bs = rng.uniform(1e-3, 1e-2, heads * hdim).astype(np.float32)
    dst = torch.empty((heads, m, hdim), dtype=torch.float32, device="cuda")
    gh.matmul_heads(dst, dev(B), dev(bs), dev(qo), dev(so), m, heads, hdim, k, stream())
    ref, _ = oracle.gemm_int8(B, bs, qo, so)  # [m][heads*hdim]
    ref = ref.reshape(m, heads, hdim).transpose(1, 0, 2)
    assert np.array_equal(bits(host(dst)), bits(np.ascontiguousarray(ref)))


@pytest.mark.parametrize("splits", [2, 3, 7])
def test_gemm_split_k(gh, oracle, monkeypatch, splits):
    """Split-K (int32 partials summed by the last workgroup of a tile) forced
    on ragged shapes: M, N and K (9 stages of 128 bytes, the last partial)
    off the tile grid, uneven stage ranges, row-major and head-major outputs;
    two launches in a row reuse the tile counters."""
    monkeypatch.setenv("GEMMA_HIP_GEMM_SPLIT", str(splits))
    rng = np.random.default_rng(40 + splits)
    m, n, k = 300, 200, 1040
    A = outlier_acts(rng, (m, k))
    qo, so = oracle.quantize_acts(A)
    for rep in range(2):
        B = rng.integers(-127, 128, (n, k), dtype=np.int8)
        bs = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        dst = torch.empty((m, n), dtype=torch.float32, device="cuda")
        gh.matmul(dst, n, dev(B), k, dev(bs), dev(qo), k, dev(so), m, n, k, stream())
        ref, _ = oracle.gemm_int8(B, bs, qo, so)
        assert np.array_equal(bits(host(dst)), bits(ref)), f"launch {rep}"
    heads, hdim, kh = 4, 256, 1152
    Ah = outlier_acts(rng, (m, kh))
    qh, sh = oracle.quantize_acts(Ah)
    B = rng.integers(-127, 128, (heads * hdim, kh), dtype=np.int8)
    bs = rng.uniform(1e-3, 1e-2, heads * hdim).astype(np.float32)
    dst = torch.empty((heads, m, hdim), dtype=torch.float32, device="cuda")
    gh.matmul_heads(dst, dev(B), dev(bs), dev(qh), dev(sh), m, heads, hdim, kh, stream())
    ref, _ = oracle.gemm_int8(B, bs, qh, sh)
    ref = ref.reshape(m, heads, hdim).transpose(1, 0, 2)
    assert np.array_equal(bits(host(dst)), bits(np.ascontiguousarray(ref)))


# The launcher's own split-K plans (no forcing), each bit-exact against the
# oracle twice in a row: 64x64 tiles in 6, 6, 4 and 3 pieces (10, 40, 20 and
# 144 tiles; K = 2064 ends in a partial stage), 128x128 tiles in 6 pieces
# (72 tiles), and 64x64 pieces with the head-major output.
SPLIT_PLANS = [(77, 301, 4096), (200, 640, 4096), (300, 200, 2064), (512, 1152, 6912),
               (1024, 1152, 6912)]


@pytest.mark.parametrize("m,n,k", SPLIT_PLANS)
def test_gemm_split_plans(gh, oracle, m, n, k):
    rng = np.random.default_rng(m + n + k)
    A = outlier_acts(rng, (m, k))
    qo, so = oracle.quantize_acts(A)
    B = rng.integers(-127, 128, (n, k), dtype=np.int8)
    bs = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    ref, _ = oracle.gemm_int8(B, bs, qo, so)
    for rep in range(2):
        dst = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        gh.matmul(dst, n, dev(B), k, dev(bs), dev(qo), k, dev(so), m, n, k, stream())
        assert np.array_equal(bits(host(dst)), bits(ref)), f"launch {rep}"


def test_gemm_split_plan_heads(gh, oracle):
    m, heads, hdim, k = 300, 2, 256, 4096
    rng = np.random.default_rng(9)
    A = outlier_acts(rng, (m, k))
    qh, sh = oracle.quantize_acts(A)
    B = rng.integers(-127, 128, (heads * hdim, k), dtype=np.int8)
    bs = rng.uniform(1e-3, 1e-2, heads * hdim).astype(np.float32)
    dst = torch.empty((heads, m, hdim), dtype=torch.float32, device="cuda")
    gh.matmul_heads(dst, dev(B), dev(bs), dev(qh), dev(sh), m, heads, hdim, k, stream())
    ref, _ = oracle.gemm_int8(B, bs, qh, sh)
    ref = ref.reshape(m, heads, hdim).transpose(1, 0, 2)
    assert np.array_equal(bits(host(dst)), bits(np.ascontiguousarray(ref)))


# --------------------------------------------------------------- fp32
def check_f32(got, mat, src, oracle):
    exact, mag = oracle.gemm_f64(mat, src)
    err = np.abs(got.astype(np.float64) - exact)
    worst = float(np.max(err / np.maximum(mag, 1e-300)))
    assert np.all(err <= TOL_F32 * mag), f"worst relative error {worst:.3e}"


# The fp32 GEMM has two kernels: split-bf16 on the bf16 matrix cores (the
# default) and fp32 MFMA (GEMMA_HIP_GEMM_F32=mfma); both are held to TOL_F32.
F32_KERNELS = ["split", "mfma"]


@pytest.mark.parametrize("kern", F32_KERNELS)
def test_f32_golden(gh, golden, oracle, monkeypatch, kern):
    monkeypatch.setenv("GEMMA_HIP_GEMM_F32", kern)
    g = golden("fpx")
    n, k = g["gemv_w"].shape
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    gh.matmul_f32(y, 0, dev(g["gemv_w"]), 0, dev(g["gemv_x"]), 0, 1, n, k, stream())
    check_f32(host(y)[None, :], g["gemv_w"], g["gemv_x"][None, :], oracle)
    m, k = g["gemm_a"].shape
    n = g["gemm_b"].shape[0]
    d = torch.empty((m, n), dtype=torch.float32, device="cuda")
    gh.matmul_f32(d, 0, dev(g["gemm_b"]), 0, dev(g["gemm_a"]), 0, m, n, k, stream())
    check_f32(host(d), g["gemm_b"], g["gemm_a"], oracle)
    # the reference's own fp32 results agree with ours to the same tolerance
    exact, mag = oracle.gemm_f64(g["gemm_b"], g["gemm_a"])
    assert np.all(np.abs(host(d) - g["gemm_dst"]) <= 2 * TOL_F32 * mag)


# (2048, 8192, 64) and (1000, 9000, 100) give at least two 128x128 tiles per
# CU, so they take the 128x128 kernel (the others the 64x64 one), the second
# with tails in every dimension
@pytest.mark.parametrize("m,n,k", [(1, 6912, 1152), (1, 1152, 6912), (1, 32768, 2560),
                                   (64, 1152, 588), (300, 640, 2048), (4096, 1152, 588),
                                   (5, 7, 9), (2048, 8192, 64), (1000, 9000, 100)])
@pytest.mark.parametrize("kern", F32_KERNELS)
def test_f32_vs_oracle(gh, oracle, monkeypatch, kern, m, n, k):
    monkeypatch.setenv("GEMMA_HIP_GEMM_F32", kern)
    note(f"f32 {kern} m={m} n={n} k={k}")
    rng = np.random.default_rng(m + n + k)
    A = outlier_acts(rng, (m, k))
    B = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    d = torch.empty((m, n), dtype=torch.float32, device="cuda")
    gh.matmul_f32(d, n, dev(B), k, dev(A), k, m, n, k, stream())
    rows = np.unique(rng.integers(0, m, min(m, 32)))
    check_f32(host(d)[rows], B, A[rows], oracle)


# Every block tile of both kernels (GEMMA_HIP_GEMM_F32_TILE forces one) on
# shapes with tails in every dimension.
@pytest.mark.parametrize("tile", ["128", "128x64", "64"])
@pytest.mark.parametrize("kern", F32_KERNELS)
@pytest.mark.parametrize("m,n,k", [(1000, 900, 100), (130, 70, 36)])
def test_f32_tiles(gh, oracle, monkeypatch, kern, tile, m, n, k):
    monkeypatch.setenv("GEMMA_HIP_GEMM_F32", kern)
    monkeypatch.setenv("GEMMA_HIP_GEMM_F32_TILE", tile)
    note(f"f32 {kern} tile {tile} m={m} n={n} k={k}")
    rng = np.random.default_rng(m * n + k)
    A = outlier_acts(rng, (m, k))
    B = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    d = torch.empty((m, n), dtype=torch.float32, device="cuda")
    gh.matmul_f32(d, n, dev(B), k, dev(A), k, m, n, k, stream())
    check_f32(host(d), B, A, oracle)


# Several weight matrices side by side in one output (gemma_hip_matmul_f32_cols;
# the split kernel runs them in one launch, the fp32-MFMA one per matrix):
# the 1b prompt pass's q|k|v and gate|up at M=512 (split-K and 128x64 tiles)
# and ragged segments whose boundaries cut through tiles.
@pytest.mark.parametrize("kern", F32_KERNELS)
@pytest.mark.parametrize("m,rows,k", [(512, (1024, 256, 256), 1152), (300, (6912, 6912), 1152),
                                      (77, (100, 37, 5), 36), (130, (64,), 260)])
def test_f32_cols(gh, oracle, monkeypatch, kern, m, rows, k):
    monkeypatch.setenv("GEMMA_HIP_GEMM_F32", kern)
    note(f"f32 cols {kern} m={m} rows={rows} k={k}")
    rng = np.random.default_rng(m + sum(rows) + k)
    A = outlier_acts(rng, (m, k))
    Bs = [(rng.standard_normal((r, k)) * 0.02).astype(np.float32) for r in rows]
    n = sum(rows)
    d = torch.full((m, n + 3), 7.0, dtype=torch.float32, device="cuda")
    gh.matmul_f32_cols(d, n + 3, [(dev(B), r) for B, r in zip(Bs, rows)], dev(A), k, m, k,
                       stream())
    got = host(d)
    pick = np.unique(rng.integers(0, m, min(m, 48)))
    check_f32(got[pick, :n], np.concatenate(Bs), A[pick], oracle)
    assert np.all(got[:, n:] == 7.0)


# Split-K of the split kernel (GEMMA_HIP_GEMM_F32_SPLIT forces the ways;
# by default it runs when the tiles leave CUs idle, as at the 1b down shape
# M=512 N=1152 K=6912): within TOL_F32 at every split, and the partials are
# summed in split order, so a repeated launch is bit-identical.
@pytest.mark.parametrize("splits", [None, 2, 3, 7, 16])
@pytest.mark.parametrize("m,n,k", [(512, 1152, 6912), (130, 70, 100), (64, 640, 2048)])
def test_f32_split_k(gh, oracle, monkeypatch, splits, m, n, k):
    if splits is not None:
        monkeypatch.setenv("GEMMA_HIP_GEMM_F32_SPLIT", str(splits))
    note(f"f32 split-k {splits} m={m} n={n} k={k}")
    rng = np.random.default_rng(m + n + k + (splits or 0))
    A = outlier_acts(rng, (m, k))
    B = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    d = torch.empty((m, n), dtype=torch.float32, device="cuda")
    gh.matmul_f32(d, n, dev(B), k, dev(A), k, m, n, k, stream())
    first = host(d)
    pick = np.unique(rng.integers(0, m, min(m, 48)))
    check_f32(first[pick], B, A[pick], oracle)
    d.fill_(0.0)
    gh.matmul_f32(d, n, dev(B), k, dev(A), k, m, n, k, stream())
    assert np.array_equal(bits(host(d)), bits(first))


def test_f32_gemm_in_a_graph(gh, oracle, monkeypatch):
    """Captured into a graph, a launch that would split K runs unsplit (the
    split-K workspace may have to be allocated, which capture forbids): every
    replay equals the unsplit eager launch bit for bit, with eager split-K
    launches of the same product between the replays."""
    m, n, k = 512, 1152, 6912
    note(f"f32 graph m={m} n={n} k={k}")
    rng = np.random.default_rng(77)
    A = outlier_acts(rng, (m, k))
    B = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    a, b = dev(A), dev(B)
    want = torch.empty((m, n), device="cuda")
    monkeypatch.setenv("GEMMA_HIP_GEMM_F32_SPLIT", "1")
    gh.matmul_f32(want, n, b, k, a, k, m, n, k, stream())
    monkeypatch.delenv("GEMMA_HIP_GEMM_F32_SPLIT")
    out = torch.empty((m, n), device="cuda")
    eager = torch.empty((m, n), device="cuda")
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=side):
        out.fill_(0.0)
        gh.matmul_f32(out, n, b, k, a, k, m, n, k, side.cuda_stream)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), f"replay {rep}"
        gh.matmul_f32(eager, n, b, k, a, k, m, n, k, stream())  # split K, eagerly
        torch.cuda.synchronize()
    pick = np.unique(rng.integers(0, m, 32))
    check_f32(host(eager)[pick], B, A[pick], oracle)
    check_f32(host(want)[pick], B, A[pick], oracle)


def test_f32_multi(gh, oracle):
    rng = np.random.default_rng(3)
    k = 1152
    x = outlier_acts(rng, (k,))
    mats = [(rng.standard_normal((r, k)) * 0.02).astype(np.float32) for r in (1024, 256, 256)]
    outs = [torch.empty(len(w), dtype=torch.float32, device="cuda") for w in mats]
    gh.matmul_f32_multi([(dev(w), None, o, len(w)) for w, o in zip(mats, outs)], dev(x), k,
                        stream())
    for w, o in zip(mats, outs):
        check_f32(host(o)[None, :], w, x[None, :], oracle)


# The fp32 GEMV on the streaming schedule: the config-2 launches with fp32
# weights (gemv_fpx / gemv_fpx_multi), rows of 2 and 4 passes (k = 2560, 6912,
# 10240), ragged jobs with an empty one, and the gemma-3-4b LM head, whose
# 2.7 GB of fp32 rows the launcher splits into jobs below 2 GB.
@pytest.mark.parametrize("rows,k", [((1024, 256, 256), 1152), ((1152,), 1024),
                                    ((6912, 6912), 1152), ((1152,), 6912),
                                    ((262144,), 1152), ((2560,), 10240), ((1000, 300), 1408),
                                    ((999,), 720),
                                    ((3001, 5, 0, 2999), 2560), ((17,), 16)])
def test_f32_stream_gemv_vs_oracle(gh, oracle, rows, k):
    note(f"f32 stream rows={rows} k={k}")
    rng = np.random.default_rng(sum(rows) + k)
    x = outlier_acts(rng, (k,))
    mats, outs, specs = [], [], []
    for r in rows:
        w = (rng.standard_normal((max(r, 1), k), dtype=np.float32) * np.float32(0.02))
        mats.append(w)
        outs.append(torch.full((max(r, 1),), 7.0, dtype=torch.float32, device="cuda"))
        specs.append((dev(w), None, outs[-1], r))
    gh.matmul_f32_multi(specs, dev(x), k, stream())
    for w, o, r in zip(mats, outs, rows):
        got = host(o)
        if r:
            check_f32(got[None, :r], w[:r], x[None, :], oracle)
        assert np.all(got[r:] == 7.0)


def test_f32_stream_gemv_split_lm_head(gh, oracle):
    """262144 x 2560 fp32 (the gemma-3-4b tied LM head, 2.7 GB): rows a tiled
    random block, so that every split part reads distinct rows."""
    n, k = 262144, 2560
    rng = np.random.default_rng(9)
    block = (rng.standard_normal((4096, k), dtype=np.float32) * np.float32(0.02))
    W = torch.from_numpy(block).to("cuda").repeat(n // 4096, 1)
    W += torch.arange(n, device="cuda", dtype=torch.float32)[:, None] * 1e-6
    x = outlier_acts(rng, (k,))
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    gh.matmul_f32(y, 0, W, 0, dev(x), 0, 1, n, k, stream())
    rows = np.concatenate([np.arange(0, 8), rng.integers(0, n, 56), np.arange(n - 8, n)])
    Wr = W[torch.from_numpy(rows).cuda()].cpu().numpy()
    check_f32(host(y)[rows][None, :], Wr, x[None, :], oracle)
    del W


# --------------------------------------------------------------- host drop-ins
def test_host_entry_points(gh, oracle):
    """The reference-shaped entry points on host buffers, with weights
    registered once and addressed through interior pointers."""
    import ctypes

    lib = gh.lib
    rng = np.random.default_rng(21)
    heads, hdim, k = 4, 64, 640
    W = rng.integers(-127, 128, (heads * hdim, k), dtype=np.int8)
    ws = rng.uniform(1e-3, 1e-2, heads * hdim).astype(np.float32)
    gh.register_weights(W, W.nbytes)
    gh.register_weights(ws, ws.nbytes)
    try:
        assert gh.device_ptr(W) is not None
        x = outlier_acts(rng, (k,))
        q = np.empty(k, np.int8)
        s = np.zeros(1, np.float32)
        assert lib.gemma_hip_quantize_act_host(q.ctypes.data, s.ctypes.data, x.ctypes.data, k) == 0
        qo, so = oracle.quantize_act(x)
        assert np.array_equal(q, qo) and bits(s)[0] == bits(so)
        # gemv on the rows of head 2 only: an interior pointer
        y = np.empty(hdim, np.float32)
        rc = lib.gemma_hip_gemv_int8_host(y.ctypes.data, W[2 * hdim:].ctypes.data,
                                          ws[2 * hdim:].ctypes.data, q.ctypes.data,
                                          ctypes.c_float(s[0]), hdim, k)
        assert rc == 0, lib.gemma_hip_last_error()
        yo, _ = oracle.gemv_int8(W[2 * hdim:3 * hdim], ws[2 * hdim:3 * hdim], qo, so)
        assert np.array_equal(bits(y), bits(yo))
        # gemm with a padded output stride; the gap keeps its contents
        m = 19
        A = outlier_acts(rng, (m, k))
        Aq = np.empty((m, k), np.int8)
        As = np.empty(m, np.float32)
        assert lib.gemma_hip_quantize_acts_host(Aq.ctypes.data, As.ctypes.data, A.ctypes.data,
                                                0, m, k) == 0
        dst = np.full((m, heads * hdim + 5), -3.0, np.float32)
        rc = lib.gemma_hip_gemm_int8_host(dst.ctypes.data, dst.shape[1], W.ctypes.data, 0,
                                          ws.ctypes.data, Aq.ctypes.data, 0, As.ctypes.data,
                                          m, heads * hdim, k)
        assert rc == 0, lib.gemma_hip_last_error()
        ref = np.full_like(dst, -3.0)
        ref, _ = oracle.gemm_int8(W, ws, Aq, As, dst=ref)
        assert np.array_equal(bits(dst), bits(ref))
        # an unregistered weight pointer is an error, not a CPU fallback
        stray = np.zeros_like(W)
        rc = lib.gemma_hip_gemv_int8_host(y.ctypes.data, stray.ctypes.data, ws.ctypes.data,
                                          q.ctypes.data, ctypes.c_float(1.0), 8, k)
        assert rc == 1 and b"not registered" in lib.gemma_hip_last_error()
    finally:
        gh.release_weights(W)
        gh.release_weights(ws)


def test_host_activation_reuse(gh, oracle):
    """The host entry points reuse the device copy of the last quantized
    activations only when the caller's int8 rows and scales are byte-equal
    to what that quantize returned: interior row blocks (the prefill QKV
    site's token blocks) and single rows hit, edited bytes or scales miss,
    and every result matches the oracle on the caller's actual inputs."""
    import ctypes

    lib = gh.lib
    rng = np.random.default_rng(23)
    n_out, k = 96, 1152
    W = rng.integers(-127, 128, (n_out, k), dtype=np.int8)
    ws = rng.uniform(1e-3, 1e-2, n_out).astype(np.float32)
    gh.register_weights(W, W.nbytes)
    gh.register_weights(ws, ws.nbytes)

    def gemm(Aq, As, r0, m):
        dst = np.zeros((m, n_out), np.float32)
        rc = lib.gemma_hip_gemm_int8_host(dst.ctypes.data, 0, W.ctypes.data, 0, ws.ctypes.data,
                                          Aq[r0:].ctypes.data, 0, As[r0:].ctypes.data,
                                          m, n_out, k)
        assert rc == 0, lib.gemma_hip_last_error()
        ref, _ = oracle.gemm_int8(W, ws, Aq[r0:r0 + m], As[r0:r0 + m])
        assert np.array_equal(bits(dst), bits(ref)), f"rows {r0}..{r0 + m}"

    try:
        # 160 rows of 1152 floats: larger than the zero-copy limit, and a
        # source row stride wider than the row
        m, sstr = 160, k + 8
        A = outlier_acts(rng, (m, sstr))
        Aq = np.empty((m, k), np.int8)
        As = np.empty(m, np.float32)
        assert lib.gemma_hip_quantize_acts_host(Aq.ctypes.data, As.ctypes.data, A.ctypes.data,
                                                sstr, m, k) == 0
        qo, so = oracle.quantize_acts(np.ascontiguousarray(A[:, :k]))
        assert np.array_equal(Aq, qo) and np.array_equal(bits(As), bits(so))
        for r0, mm in ((0, 128), (128, 32), (37, 5)):
            gemm(Aq, As, r0, mm)
        # one row of the batch as a GEMV input
        y = np.empty(n_out, np.float32)
        rc = lib.gemma_hip_gemv_int8_host(y.ctypes.data, W.ctypes.data, ws.ctypes.data,
                                          Aq[3].ctypes.data, ctypes.c_float(As[3]), n_out, k)
        assert rc == 0, lib.gemma_hip_last_error()
        yo, _ = oracle.gemv_int8(W, ws, Aq[3], As[3])
        assert np.array_equal(bits(y), bits(yo))
        # the caller edits one int8 value, then one scale: both must be seen
        Aq[40, 7] = 127 if Aq[40, 7] != 127 else -127
        gemm(Aq, As, 32, 16)
        As[45] *= np.float32(2.0)
        gemm(Aq, As, 32, 16)
        rc = lib.gemma_hip_gemv_int8_host(y.ctypes.data, W.ctypes.data, ws.ctypes.data,
                                          Aq[3].ctypes.data, ctypes.c_float(As[3] * 2), n_out, k)
        assert rc == 0, lib.gemma_hip_last_error()
        yo, _ = oracle.gemv_int8(W, ws, Aq[3], As[3] * np.float32(2))
        assert np.array_equal(bits(y), bits(yo))
    finally:
        gh.release_weights(W)
        gh.release_weights(ws)


def test_host_fp32_entry_points(gh, oracle):
    lib = gh.lib
    rng = np.random.default_rng(22)
    n, k, m = 96, 588, 9
    W = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    gh.register_weights(W, W.nbytes)
    try:
        x = outlier_acts(rng, (k,))
        y = np.empty(n, np.float32)
        assert lib.gemma_hip_gemv_fpx_host(y.ctypes.data, W.ctypes.data, x.ctypes.data, n, k) == 0
        check_f32(y[None, :], W, x[None, :], oracle)
        A = outlier_acts(rng, (m, k))
        d = np.empty((m, n), np.float32)
        assert lib.gemma_hip_gemm_fpx_host(d.ctypes.data, 0, W.ctypes.data, 0, A.ctypes.data,
                                           0, m, n, k) == 0
        check_f32(d, W, A, oracle)
    finally:
        gh.release_weights(W)


def test_argument_errors(gh):
    import gemma_hip

    with pytest.raises(gemma_hip.GemmaHipError, match="njobs"):
        gh.matmul_multi([], 0, 0, 64)
    with pytest.raises(gemma_hip.GemmaHipError, match="stride"):
        gh.matmul(1, 4, 1, 8, 1, 1, 16, 1, 2, 8, 16)
    with pytest.raises(gemma_hip.GemmaHipError, match="k="):
        gh.quantize_matmul([(1, 1, 1, 4)], 1, 70000)
    # the fp32 column-grouped GEMM: job count, an empty job, a null weight
    with pytest.raises(gemma_hip.GemmaHipError, match="njobs"):
        gh.matmul_f32_cols(1, 0, [], 1, 0, 4, 8)
    with pytest.raises(gemma_hip.GemmaHipError, match="njobs"):
        gh.matmul_f32_cols(1, 0, [(1, 4)] * 4, 1, 0, 4, 8)
    with pytest.raises(gemma_hip.GemmaHipError, match="m=0"):
        gh.matmul_f32_cols(1, 0, [(1, 4), (1, 0)], 1, 0, 4, 8)
    with pytest.raises(gemma_hip.GemmaHipError, match="null weight"):
        gh.matmul_f32_cols(1, 0, [(1, 4), (None, 4)], 1, 0, 4, 8)
    with pytest.raises(gemma_hip.GemmaHipError, match="stride"):
        gh.matmul_f32_cols(1, 4, [(1, 4), (1, 4)], 1, 0, 4, 8)


# --------------------------------------------------------------- SigLIP patch embedding
@pytest.mark.parametrize("img_px,psize,dim", [(56, 14, 64), (896, 14, 1152), (30, 5, 17)])
def test_patch_embed_vs_oracle(gh, oracle, img_px, psize, dim):
    """gemma.c:4411-4448 as im2col + fp32 GEMM (896 px,
    P = 14, dim 1152); image normalised as gemma.c:4271-4273."""
    note(f"patch embed img_px={img_px} psize={psize} dim={dim}")
    rng = np.random.default_rng(img_px + dim)
    raw = rng.uniform(0, 255, (img_px, img_px, 3)).astype(np.float32)
    img = ((raw / np.float32(255.0) - np.float32(0.5)) / np.float32(0.5)).astype(np.float32)
    pe = (rng.standard_normal((dim, 3, psize, psize)) * 0.02).astype(np.float32)
    pe_b = (rng.standard_normal(dim) * 0.02).astype(np.float32)
    npatch = (img_px // psize) ** 2
    dst = torch.empty((npatch, dim), dtype=torch.float32, device="cuda")
    gh.patch_embed(dst, dev(img), dev(pe), dev(pe_b), img_px, psize, dim, None, stream())
    got = host(dst)
    rows = np.unique(np.concatenate([np.arange(min(npatch, 4)), rng.integers(0, npatch, 24)]))
    # oracle on the sampled patches only: crop those patches into a strip
    ppi = img_px // psize
    ref, mag = oracle.patch_embed_f64(img, pe, pe_b, psize) if npatch <= 256 else (None, None)
    if ref is None:
        refs, mags = [], []
        for pi in rows:
            oy, ox = divmod(int(pi), ppi)
            tile = np.ascontiguousarray(img[oy * psize:(oy + 1) * psize, ox * psize:(ox + 1) * psize])
            r, mg = oracle.patch_embed_f64(tile, pe, pe_b, psize)
            refs.append(r[0])
            mags.append(mg[0])
        ref, mag = np.array(refs), np.array(mags)
        got = got[rows]
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= TOL_F32 * mag), f"worst {np.max(err / mag):.3e}"


def test_patch_embed_host(gh, oracle):
    lib = gh.lib
    rng = np.random.default_rng(8)
    img_px, psize, dim = 28, 14, 40
    img = rng.standard_normal((img_px, img_px, 3)).astype(np.float32)
    pe = (rng.standard_normal((dim, 3, psize, psize)) * 0.02).astype(np.float32)
    pe_b = rng.standard_normal(dim).astype(np.float32)
    gh.register_weights(pe, pe.nbytes)
    gh.register_weights(pe_b, pe_b.nbytes)
    try:
        out = np.empty(((img_px // psize) ** 2, dim), np.float32)
        rc = lib.gemma_hip_patch_embed_host(out.ctypes.data, img.ctypes.data, pe.ctypes.data,
                                            pe_b.ctypes.data, img_px, psize, dim)
        assert rc == 0, lib.gemma_hip_last_error()
        ref, mag = oracle.patch_embed_f64(img, pe, pe_b, psize)
        assert np.all(np.abs(out - ref) <= TOL_F32 * mag)
    finally:
        gh.release_weights(pe)
        gh.release_weights(pe_b)


# ------------------------------------------------------------- per-op timing
def test_perf_counts_ops_under_reference_names(gh):
    """gemma_hip_perf_*: GPU time per (phase, op) under the reference's
    PerfBench names (gemma.c:2426-2431)."""
    rng = np.random.default_rng(5)
    k, n, m = 640, 512, 96
    W = dev(rng.integers(-127, 128, (n, k), dtype=np.int8))
    ws = dev(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    x = dev(rng.standard_normal((m, k)).astype(np.float32))
    xq = torch.empty((m, k), dtype=torch.int8, device="cuda")
    xs = torch.empty(m, dtype=torch.float32, device="cuda")
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    gh.perf_enable(True)
    try:
        gh.perf_phase("prefill")
        gh.quantize(xq, xs, x, k, m, k, stream())
        gh.matmul(y, n, W, k, ws, xq, k, xs, m, n, k, stream())
        gh.matmul(y, n, W, k, ws, xq, k, xs, m, n, k, stream())
        gh.perf_phase("decode")
        for _ in range(3):
            gh.quantize_matmul([(W, ws, y, n)], x, k, None, None, stream())
        got = gh.perf_read()
    finally:
        gh.perf_enable(False)
    assert set(got) == {"prefill", "decode"}
    assert got["prefill"]["quantize_act"][1] == 1
    assert got["prefill"]["gemm_int8"][1] == 2
    assert got["decode"] == {"gemv_int8": got["decode"]["gemv_int8"]}
    assert got["decode"]["gemv_int8"][1] == 3
    for ph in got.values():
        for sec, calls in ph.values():
            assert 0 < sec < 1.0
