"""The device-resident vision tower (gemma_hip_vision_*) against the vision
oracle (oracle/vision_oracle.py), and the oracle's glue pinned by closed
forms.

Bar: as for the decoder (tests/test_decoder.py).  The int8 GEMMs are the
bit-exact kernels of test_gpu_parity.py; the fp32 glue (patch-embedding sums,
layer norms, attention, GELU, pooling, RMSNorm) is evaluated in fp64 by both
the device and the oracle and rounded once, so the soft tokens must agree to
|out_gpu - out_oracle| <= TOL * max|out_oracle| -- a bar that a single fp32
reassociation anywhere upstream of an int8 requantization would fail.
"""

from __future__ import annotations

import numpy as np
import pytest

import model_bin
from oracle import vision_oracle as vorc

TOL = 1e-5


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
}


@pytest.mark.gpu
@pytest.mark.parametrize("shape", sorted(SHAPES))
def test_vision_matches_oracle(gh, oracle, shape):
    vis = model_bin.synth_vision(seed=7, text_dim=64, **SHAPES[shape])
    img = model_bin.synth_image(SHAPES[shape]["img_px"], seed=8)
    want = vorc.VisionOracle(vis, oracle).forward(img)
    tower = gh.vision(vis)
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
