"""The device-resident vision tower (gemma_hip_vision_*) against the vision
oracle (oracle/vision_oracle.py), and the oracle's glue pinned by closed
forms.

Bar: as for the decoder (tests/test_decoder.py).  The int8 GEMMs are the
bit-exact kernels of test_gpu_parity.py; the fp32 glue (patch-embedding sums,
layer norms, attention, GELU, pooling, RMSNorm) is evaluated in fp64 by both
the device and the oracle and rounded once, so the soft tokens must agree to
|out_gpu - out_oracle| <= TOL * max|out_oracle| -- a bar that a single fp32
reassociation anywhere upstream of an int8 requantization would fail.  The
tower is held to it with its attention in fp64 (ATTN_F64); the library's
default, fp32 attention, has its own tests below.
"""

from __future__ import annotations

import copy
import os
import subprocess

import numpy as np
import pytest

import model_bin
from gemma_hip import ATTN_F32, ATTN_F64
from oracle import vision_oracle as vorc

import flips

TOL = 1e-5

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
E2E_CPU = os.path.join(REPO, "oracle", "_ref", "gemma_e2e_cpu")
needs_e2e = pytest.mark.skipif(not os.path.exists(E2E_CPU),
                               reason="oracle/_ref/gemma_e2e_cpu not built (needs /root/reference)")


# ------------------------------------------------------------ oracle pins (CPU)
def test_layernorm_closed_forms():
    w = np.array([2.0, -1.0, 0.5, 3.0], np.float32)
    b = np.array([0.1, 0.2, -0.3, 0.0], np.float32)
    # a constant row normalizes to zero: the output is the bias
    assert np.array_equal(vorc.layernorm(np.full(4, 7.0, np.float32), w, b, 1e-6), b)
    # a row of +a and -a: mean 0, variance a^2, so the output is +-w (up to eps) plus b
    x = np.array([3.0, -3.0, 3.0, -3.0], np.float32)
    want = np.array([1, -1, 1, -1]) * w / np.sqrt(1 + np.float32(1e-6) / 9.0) + b
    assert np.allclose(vorc.layernorm(x, w, b, 1e-6), want, rtol=1e-7)


def test_avg_pool_of_block_constant_grid():
    ppi, k, dim = 8, 4, 3
    blocks = np.arange(4 * dim, dtype=np.float32).reshape(2, 2, dim)
    grid = np.repeat(np.repeat(blocks, k, axis=0), k, axis=1).reshape(ppi * ppi, dim)
    assert np.array_equal(vorc.avg_pool(grid, ppi, k), blocks.reshape(4, dim))


def test_attention_closed_forms():
    rng = np.random.default_rng(3)
    k = rng.standard_normal((10, 8)).astype(np.float32)
    v = rng.standard_normal((10, 8)).astype(np.float32)
    q = np.stack([k[2] * 60, np.zeros(8, np.float32)])
    out = vorc.attention(q, k, v, 1.0)
    assert np.allclose(out[0], v[2], atol=1e-5)         # one key dominates
    assert np.allclose(out[1], v.mean(axis=0), atol=1e-6)  # equal scores: the mean


# ------------------------------------------------------------------ GPU
SHAPES = {
    # SigLIP's head dim (72), 16 patches pooled to 4 tokens
    "hd72": dict(nl=2, n_heads=2, img_px=56, psize=14, dim=144, mlp_dim=288, img_tok=4),
    # 64 patches (two query tiles, four key tiles), 16 tokens, head dim 16
    "hd16": dict(nl=3, n_heads=4, img_px=112, psize=14, dim=64, mlp_dim=128, img_tok=16),
    # SigLIP's own widths (dim 1152, 16 heads of 72, mlp 4304) at 224 px: 256
    # patches, two query blocks per head (32 blocks, so the XCD renumbering
    # runs), the 1152-wide layer-norm rows and multi-chunk GELU rows of
    # config 4, pooled 4x4 to 16 tokens
    "siglip": dict(nl=2, n_heads=16, img_px=224, psize=14, dim=1152, mlp_dim=4304, img_tok=16),
    # one layer over 1 and 4 patches: few enough quantized values that the
    # margin criterion (tests/flips.py) can clear whole passes
    "tiny": dict(nl=1, n_heads=2, img_px=28, psize=14, dim=32, mlp_dim=64, img_tok=4),
    "small": dict(nl=1, n_heads=2, img_px=56, psize=14, dim=32, mlp_dim=64, img_tok=4),
}


@pytest.mark.gpu
@pytest.mark.parametrize("shape", sorted(SHAPES))
def test_vision_matches_oracle(gh, oracle, shape):
    vis = model_bin.synth_vision(seed=7, text_dim=64, **SHAPES[shape])
    img = model_bin.synth_image(SHAPES[shape]["img_px"], seed=8)
    want = vorc.VisionOracle(vis, oracle).forward(img)
    tower = gh.vision(vis, attention=ATTN_F64)
    try:
        got = tower.forward(img)
        again = tower.forward(img)
    finally:
        tower.close()
    scale = float(np.abs(want).max())
    diff = float(np.abs(got - want).max())
    print(f"vision {shape}: |d|/max|out| = {diff / scale:.3g}", flush=True)
    assert diff <= TOL * scale
    assert np.array_equal(got, again)  # deterministic


@pytest.mark.gpu
def test_vision_perf_breakdown(gh):
    """The tower under per-op timing: one forward broken down in the vision
    phase under the reference's PerfBench names (gemma.c:2409-2431)."""
    vis = model_bin.synth_vision(seed=7, text_dim=64, **SHAPES["tiny"])
    img = model_bin.synth_image(SHAPES["tiny"]["img_px"], seed=8)
    nl = vis["config"]["nl"]
    tower = gh.vision(vis)
    try:
        want = tower.forward(img)
        gh.perf_enable(True)
        try:
            got = tower.forward(img)
            perf = gh.perf_read()
        finally:
            gh.perf_enable(False)
    finally:
        tower.close()
    assert np.array_equal(got, want)
    assert set(perf) == {"vision"}
    calls = {op: c for op, (sec, c) in perf["vision"].items()}
    assert calls == {"gemm_fpx": 1, "layernorm": 2 * nl + 1, "gemm_int8": 4 * nl + 1,
                     "softmax": nl, "quantize_act": nl, "gelu": nl, "rmsnorm": 1}
    for op, (sec, c) in perf["vision"].items():
        assert 0 < sec < 1.0, op


# The default arithmetic (GEMMA_HIP_ATTN_F32: the patch embedding and the
# attention on the fp32 matrix cores) in the whole tower, against the fp64
# oracle.  The bar of each case is decided before the device runs, from the
# oracle's requantization margins (tests/flips.py): a pass with no quantizer
# argument within reach of fp32 rounding of a boundary agrees to fp32
# rounding (F32_PRE_FLIP); any other may flip an int8 activation, which moves
# the pooled soft tokens by ~1% (F32_FLIP_LEVEL).  The attention and patch
# kernels themselves are pinned directly (below, and test_gpu_parity.py).
F32_TOWER_CASES = [("tiny", 2, 102), ("tiny", 4, 104), ("small", 1, 101), ("small", 5, 105),
                   ("hd16", 7, 8), ("hd72", 8, 9)]
F32_PRE_FLIP = 1e-6
F32_FLIP_LEVEL = 5e-2


def oracle_tower(oracle, shape, seed, img_seed, text_dim=64):
    """(weights, image, the oracle's soft tokens, whether the pass is flip-free)"""
    vis = model_bin.synth_vision(seed=seed, text_dim=text_dim, **SHAPES[shape])
    img = model_bin.synth_image(SHAPES[shape]["img_px"], seed=img_seed)
    want, margin = flips.tracked(oracle, vorc.VisionOracle(vis, oracle).forward, img)
    return vis, img, want, margin > flips.MARGIN_BOUND


def test_f32_tower_cases_exercise_both_bars(oracle):
    """The case list holds passes the criterion clears (so the fp32-rounding
    bar is really applied) and passes it does not."""
    free = [oracle_tower(oracle, *case)[3] for case in F32_TOWER_CASES]
    assert sum(free) >= 2 and not all(free)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,seed,img_seed", F32_TOWER_CASES)
def test_vision_f32_matches_oracle(gh, oracle, shape, seed, img_seed):
    vis, img, want, free = oracle_tower(oracle, shape, seed, img_seed)
    tower = gh.vision(vis)
    try:
        got = tower.forward(img)  # the default: ATTN_F32
        again = tower.forward(img)
        tower.set_attention(ATTN_F64)
        exact = tower.forward(img)
        tower.set_attention(ATTN_F32)
        back = tower.forward(img)
    finally:
        tower.close()
    rel = float(np.abs(got - want).max() / np.abs(want).max())
    print(f"vision f32 {shape} seed {seed} ({'flip-free' if free else 'may flip'}): {rel:.3g}",
          flush=True)
    assert rel <= (F32_PRE_FLIP if free else F32_FLIP_LEVEL)
    assert np.array_equal(got, again)
    assert float(np.abs(exact - want).max()) <= TOL * float(np.abs(want).max())  # fp64 mode
    assert np.array_equal(back, got)  # and back


@pytest.mark.gpu
def test_vision_f32_attention_siglip_width_flip_level(gh, oracle):
    vis = model_bin.synth_vision(seed=7, text_dim=64, **SHAPES["siglip"])
    img = model_bin.synth_image(SHAPES["siglip"]["img_px"], seed=8)
    want = vorc.VisionOracle(vis, oracle).forward(img)
    tower = gh.vision(vis, attention=ATTN_F32)
    try:
        got = tower.forward(img)
    finally:
        tower.close()
    rel = float(np.abs(got - want).max() / np.abs(want).max())
    print(f"vision f32 attention siglip width: {rel:.3g}", flush=True)
    assert rel <= F32_FLIP_LEVEL


# The attention block alone (gemma_hip_vision_attention) against the fp64
# oracle's attention, before any quantization: the fp64 kernel to one fp32
# rounding, the fp32 kernel to the fp32 accumulation error over n keys.
ATT_CASES = {
    # n, heads, dim: SigLIP at 896 px; ragged query and key tiles at head
    # dims 16, 32, 128; SigLIP's head dim at an odd patch count
    "siglip896": (4096, 16, 1152),
    "hd16": (200, 4, 64),
    "hd32": (77, 3, 96),
    "hd128": (300, 2, 256),
    "hd72": (1000, 4, 288),
}
ATT_F64_TOL = 2.4e-7  # two fp32 ulps of the largest output
ATT_F32_TOL = 2e-5


def _attention_inputs(n, heads, dim, seed):
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((n, 3 * dim)).astype(np.float32)
    bias = (0.5 * rng.standard_normal(3 * dim)).astype(np.float32)
    hd = dim // heads
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    q = qkv[:, :dim] + bias[:dim]
    k = qkv[:, dim:2 * dim] + bias[dim:2 * dim]
    v = qkv[:, 2 * dim:] + bias[2 * dim:]
    want = np.concatenate([vorc.attention(q[:, h * hd:(h + 1) * hd], k[:, h * hd:(h + 1) * hd],
                                          v[:, h * hd:(h + 1) * hd], scale)
                           for h in range(heads)], axis=1)
    return qkv, bias, want


@pytest.mark.gpu
@pytest.mark.parametrize("case", sorted(ATT_CASES))
def test_vision_attention_kernels_match_oracle(gh, case, monkeypatch):
    import torch

    n, heads, dim = ATT_CASES[case]
    qkv, bias, want = _attention_inputs(n, heads, dim, seed=n + heads)
    dq, db = torch.from_numpy(qkv).cuda(), torch.from_numpy(bias).cuda()
    scale = float(np.abs(want).max())
    # mode 1 twice: the split-bf16 kernel (the default) and the plain fp32
    # matrix-core kernel that GEMMA_HIP_VIS_ATTN=f32 selects per launch
    for mode, kernel, tol in ((0, "f64", ATT_F64_TOL), (1, "split", ATT_F32_TOL),
                              (1, "f32", ATT_F32_TOL)):
        if kernel == "f32":
            monkeypatch.setenv("GEMMA_HIP_VIS_ATTN", "f32")
        else:
            monkeypatch.delenv("GEMMA_HIP_VIS_ATTN", raising=False)
        out = torch.full((n, dim), float("nan"), device="cuda")
        gh.vision_attention(out, dq, db, n, heads, dim, mode,
                            stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        rel = float(np.abs(got - want).max()) / scale
        print(f"vision attention {case} {kernel}: |d|/max = {rel:.3g}", flush=True)
        assert rel <= tol, (case, kernel, rel)


@pytest.mark.gpu
def test_vision_argument_errors(gh):
    import ctypes

    import gemma_hip

    from gemma_hip import GemmaHipError

    bad = model_bin.synth_vision(seed=1, text_dim=64, **dict(SHAPES["hd16"], n_heads=3))
    with pytest.raises(GemmaHipError, match="unsupported config"):
        gh.vision(bad)
    c = SHAPES["hd16"]
    cfg = gemma_hip.VisionConfig(c["nl"], c["n_heads"], c["img_px"], c["psize"], c["dim"],
                                 c["mlp_dim"], 1e-6, c["img_tok"], 64)
    layers = (gemma_hip.VisionLayer * c["nl"])()
    stray = np.zeros(64, np.float32)
    h = gh.lib.gemma_hip_vision_create(ctypes.byref(cfg), layers, *([stray.ctypes.data] * 9))
    assert not h and b"not registered" in gh.lib.gemma_hip_last_error()


# ------------------------------------------------- against the reference program
# forward_vision itself (compiled from the reference's source by oracle/Makefile,
# run by oracle/e2e_harness.c on a multimodal .bin written by model_bin) on the
# same weights and image.  The reference evaluates the glue in fp32, so where
# the oracle's margin criterion (tests/flips.py) clears the pass the two agree
# to fp32 rounding (measured 1e-7 .. 3e-7 of the largest output; bound
# REL_PRE_FLIP), and elsewhere to the flip level.  The planted-mistake test
# shows the tight bound is sharp: a dropped bias, a squared attention scale or
# transposed pooling moves the output by 1.5% to 100%.
REL_PRE_FLIP = 1e-5
REL_FLIP_LEVEL = 5e-2
REF_CASES = {  # shape, weight seed, image seed
    "tiny": ("tiny", 2, 102), "small": ("small", 1, 101),
    "hd72": ("hd72", 1, 101), "hd16": ("hd16", 3, 8), "hd72_s5": ("hd72", 5, 105)}


def run_reference_vision(tmp_path, case):
    shape, seed, img_seed = REF_CASES[case]
    vis = model_bin.synth_vision(seed=seed, text_dim=640, **SHAPES[shape])
    path = model_bin.write_bin(str(tmp_path / f"mm_{case}.bin"), "gemma-3-270m", seed=5,
                               nvocab=512, layers=2, vision=vis)
    img = model_bin.synth_image(SHAPES[shape]["img_px"], seed=img_seed)
    img_path, out_path = str(tmp_path / "img.f32"), str(tmp_path / "soft.f32")
    img.tofile(img_path)
    env = dict(os.environ, GEMMA_E2E_VISION_IMAGE=img_path, GEMMA_E2E_VISION_OUT=out_path)
    out = subprocess.run([E2E_CPU, path, "1", "0", "1", "4"], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    ref = np.fromfile(out_path, np.float32).reshape(SHAPES[shape]["img_tok"], 640)
    return model_bin.read_bin(path)["vision"], img, ref


def rel_to(ref, got):
    return float(np.abs(got - ref).max() / np.abs(ref).max())


def test_multimodal_bin_round_trip(tmp_path):
    vis = model_bin.synth_vision(seed=2, text_dim=640, **SHAPES["hd16"])
    path = model_bin.write_bin(str(tmp_path / "mm.bin"), "gemma-3-270m", seed=5, nvocab=512,
                               layers=2, vision=vis)
    back = model_bin.read_bin(path)
    assert back["end"] == os.path.getsize(path)
    v = back["vision"]
    assert v["config"] == dict(vis["config"])
    assert np.array_equal(v["pe"], vis["pe"]) and np.array_equal(v["pos"][0], vis["pos"][0])
    for a, b in zip(v["layers"], vis["layers"]):
        for key in ("wq", "w1", "w2"):
            assert np.array_equal(a[key][0], b[key][0]) and np.array_equal(a[key][1], b[key][1])
        for key in ("bv", "b1", "n2_b"):
            assert np.array_equal(a[key], b[key])
    assert np.array_equal(v["proj"][1], vis["proj"][1]) and np.array_equal(v["norm"], vis["norm"])


@needs_e2e
@pytest.mark.parametrize("case", sorted(REF_CASES))
def test_vision_oracle_follows_reference_program(tmp_path, oracle, case):
    vis, img, ref = run_reference_vision(tmp_path, case)
    want, margin = flips.tracked(oracle, vorc.VisionOracle(vis, oracle).forward, img)
    free = margin > flips.MARGIN_BOUND
    rel = rel_to(ref, want)
    print(f"vision oracle vs reference ({case}, {'flip-free' if free else 'may flip'}): "
          f"{rel:.3g}", flush=True)
    assert rel <= (REL_PRE_FLIP if free else REL_FLIP_LEVEL)


@needs_e2e
def test_vision_comparison_catches_planted_mistakes(tmp_path, oracle, monkeypatch):
    vis, img, ref = run_reference_vision(tmp_path, "hd16")
    bad = copy.deepcopy(vis)
    bad["post_nb"] = np.zeros_like(bad["post_nb"])
    assert rel_to(ref, vorc.VisionOracle(bad, oracle).forward(img)) > 100 * REL_PRE_FLIP
    attention = vorc.attention
    monkeypatch.setattr(vorc, "attention", lambda q, k, v, s: attention(q, k, v, s * s))
    assert rel_to(ref, vorc.VisionOracle(vis, oracle).forward(img)) > 100 * REL_PRE_FLIP
    monkeypatch.setattr(vorc, "attention", attention)
    pool = vorc.avg_pool
    monkeypatch.setattr(vorc, "avg_pool", lambda h, ppi, k: pool(
        h.reshape(ppi, ppi, -1).transpose(1, 0, 2).reshape(ppi * ppi, -1), ppi, k))
    assert rel_to(ref, vorc.VisionOracle(vis, oracle).forward(img)) > 100 * REL_PRE_FLIP


@pytest.mark.gpu
@needs_e2e
@pytest.mark.parametrize("case", sorted(REF_CASES))
@pytest.mark.parametrize("mode", ["f32", "f64"])
def test_device_vision_follows_reference_program(gh, oracle, tmp_path, case, mode):
    vis, img, ref = run_reference_vision(tmp_path, case)
    _, margin = flips.tracked(oracle, vorc.VisionOracle(vis, oracle).forward, img)
    free = margin > flips.MARGIN_BOUND
    tower = gh.vision(vis, attention=ATTN_F32 if mode == "f32" else ATTN_F64)
    try:
        got = tower.forward(img)
    finally:
        tower.close()
    rel = rel_to(ref, got)
    print(f"device vision ({mode}) vs reference ({case}, {'flip-free' if free else 'may flip'}): "
          f"{rel:.3g}", flush=True)
    assert rel <= (REL_PRE_FLIP if free else REL_FLIP_LEVEL)


# ------------------------------------------------- unquantized ('U') towers
# forward_vision's !quant branches (gemma.c:4454, 4488, 4562, 4604, 4626,
# 4709): fp32 projections, position embedding and output projection, no
# activation quantize.  With no int8 requantization to amplify a rounding
# difference, the oracle (float64 products rounded once) agrees with the
# reference program to fp32 rounding, and the device (fp32 matrix-core GEMMs
# and attention by default) with the oracle to U_TOL of the largest output;
# in the verification mode (fp64 GEMMs and attention, every output rounded
# once) to the W8A8 tower's TOL.
U_TOL = 1e-4
U_CASES = {"tiny": ("tiny", 2, 102), "hd72": ("hd72", 1, 101), "hd16": ("hd16", 3, 8),
           "siglip": ("siglip", 4, 7)}


def u_tower(case, text_dim=640):
    shape, seed, img_seed = U_CASES[case]
    vis = model_bin.synth_vision(seed=seed, text_dim=text_dim, quant=False, **SHAPES[shape])
    return vis, model_bin.synth_image(SHAPES[shape]["img_px"], seed=img_seed)


def test_u_multimodal_bin_round_trip(tmp_path):
    vis, _ = u_tower("hd16")
    path = model_bin.write_bin(str(tmp_path / "mmu.bin"), "gemma-3-270m", seed=5, nvocab=512,
                               layers=2, vision=vis, quant=False)
    back = model_bin.read_bin(path)
    assert back["end"] == os.path.getsize(path)
    v = back["vision"]
    assert v["config"] == dict(vis["config"]) and v["config"]["quant"] is False
    assert np.array_equal(v["pos"], vis["pos"]) and np.array_equal(v["proj"], vis["proj"])
    for a, b in zip(v["layers"], vis["layers"]):
        for key in ("wq", "wo", "w1", "w2", "b1", "n2_b"):
            assert np.array_equal(a[key], b[key])
    with pytest.raises(ValueError):
        model_bin.write_bin(str(tmp_path / "mix.bin"), "gemma-3-270m", seed=5, nvocab=512,
                            layers=2, vision=vis, quant=True)


@needs_e2e
@pytest.mark.parametrize("case", ["tiny", "hd72", "hd16"])
def test_u_vision_oracle_follows_reference_program(tmp_path, oracle, case):
    vis, img = u_tower(case)
    path = model_bin.write_bin(str(tmp_path / f"mmu_{case}.bin"), "gemma-3-270m", seed=5,
                               nvocab=512, layers=2, vision=vis, quant=False)
    img_path, out_path = str(tmp_path / "img.f32"), str(tmp_path / "soft.f32")
    img.tofile(img_path)
    env = dict(os.environ, GEMMA_E2E_VISION_IMAGE=img_path, GEMMA_E2E_VISION_OUT=out_path)
    out = subprocess.run([E2E_CPU, path, "1", "0", "1", "4"], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    ref = np.fromfile(out_path, np.float32).reshape(vis["config"]["img_tok"], 640)
    want = vorc.VisionOracle(model_bin.read_bin(path)["vision"], oracle).forward(img)
    rel = rel_to(ref, want)
    print(f"U vision oracle vs reference ({case}): {rel:.3g}", flush=True)
    assert rel <= REL_PRE_FLIP  # no requantization: fp32 rounding throughout
    # sharp: the fp32 position embedding left out moves the output far past it
    bad = copy.deepcopy(model_bin.read_bin(path)["vision"])
    bad["pos"] = np.zeros_like(bad["pos"])
    assert rel_to(ref, vorc.VisionOracle(bad, oracle).forward(img)) > 100 * REL_PRE_FLIP


@pytest.mark.gpu
@pytest.mark.parametrize("case", sorted(U_CASES))
@pytest.mark.parametrize("mode", ["f32", "f64"])
def test_u_vision_matches_oracle(gh, oracle, case, mode):
    vis, img = u_tower(case)
    want = vorc.VisionOracle(vis, oracle).forward(img)
    tower = gh.vision(vis, attention=ATTN_F32 if mode == "f32" else ATTN_F64)
    try:
        got = tower.forward(img)
        again = tower.forward(img)
        if case == "tiny" and mode == "f32":
            gh.perf_enable(True)
            try:
                tower.forward(img)
                perf = gh.perf_read()
            finally:
                gh.perf_enable(False)
            nl = vis["config"]["nl"]
            calls = {op: c for op, (s, c) in perf["vision"].items()}
            # patch GEMM; per layer q|k|v (one launch), o, fc1, fc2; projector
            assert calls == {"gemm_fpx": 1 + 4 * nl + 1, "layernorm": 2 * nl + 1,
                             "softmax": nl, "gelu": nl, "rmsnorm": 1}
    finally:
        tower.close()
    rel = rel_to(want, got)
    print(f"U vision {case} ({mode}): |d|/max|out| = {rel:.3g}", flush=True)
    assert rel <= (U_TOL if mode == "f32" else TOL)
    assert np.array_equal(got, again)
