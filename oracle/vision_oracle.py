"""CPU restatement of the reference's vision tower, the checker of the device
vision tower (gemma_hip_vision_*).  TEST INFRASTRUCTURE ONLY: tests/ use it;
nothing in the product imports it.

Follows forward_vision (gemma.c:4394-4725) step by step, with the conventions
of decode_oracle.py: the int8 parts are the pinned oracle's (quantize_acts
from oracle/gemma_oracle.c, int32 sums in int64 numpy, the rescale
(float)acc * (xs * ws) in float32); single fp32 additions (biases, residuals,
the dequantized position embedding) are float32 operations as in the
reference; the rest of the fp32 glue -- the patch embedding's sums (the
pinned oracle_patch_embed_f64), layernorm (2526-2549), scores and softmax
(4533-4561, 4091-4117), gelu_tanh (4139-4145), the average pooling
(4673-4694) and rmsnorm (2508-2521) -- is computed in float64 and rounded to
float32 where the reference stores a float32 tensor.

Pins: patch_embed_f64 and the int8 pieces are the pinned oracle functions;
layernorm, pooling and the attention are pinned by closed-form tests in
tests/test_vision.py (a constant row, a per-block constant image, one key
dominating).
"""

from __future__ import annotations

import numpy as np

from oracle.decode_oracle import clamp_f32, gelu_tanh, int_dot, rmsnorm

F32 = np.float32
F64 = np.float64


def layernorm(x, w, b, eps):
    """gemma.c:2526-2549: (x - mean) / sqrt(var + eps) * w + b per row."""
    x = np.asarray(x, F64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    inv = 1.0 / np.sqrt(var + F64(F32(eps)))
    return ((x - mean) * inv * np.asarray(w, F64) + np.asarray(b, F64)).astype(F32)


def attention(q, k, v, scale):
    """One head, every query over every key (gemma.c:4533-4561)."""
    s = np.asarray(q, F64) @ np.asarray(k, F64).T * F64(scale)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return (p @ np.asarray(v, F64)).astype(F32)


def avg_pool(h, ppi, ksize):
    """AvgPool2d(ksize, ksize) of the [ppi*ppi][dim] patch grid (4673-4694)."""
    dim = h.shape[1]
    g = np.asarray(h, F64).reshape(ppi // ksize, ksize, ppi // ksize, ksize, dim)
    return g.mean(axis=(1, 3)).reshape(-1, dim).astype(F32)


class VisionOracle:
    """A VisionEncoder's weights (dict of numpy arrays) on the CPU."""

    def __init__(self, vis, oracle):
        self.v = vis
        self.c = vis["config"]
        self.o = oracle

    def gemm(self, w, x_f32):
        """quantize_acts + gemm_int8 (gemma.c:2652-2674, 3937-4054): exact.
        For an fp32 ('U') tower, gemm_fpx (3308): the float64 product rounded
        once."""
        if not self.c.get("quant", True):
            return (np.asarray(x_f32, F64) @ np.asarray(w, F64).T).astype(F32)
        q, xs = self.o.quantize_acts(np.ascontiguousarray(x_f32, F32))
        acc = int_dot(q, w[0])
        return acc.astype(F32) * (xs[:, None] * np.asarray(w[1], F32)[None, :])

    def forward(self, img):
        c, v = self.c, self.v
        dim, nh = c["dim"], c["n_heads"]
        hd = dim // nh
        ppi = c["img_px"] // c["psize"]
        side = int(round(np.sqrt(c["img_tok"])))
        eps = c["eps"]
        emb, _ = self.o.patch_embed_f64(img, v["pe"], v["pe_b"], c["psize"])
        x = clamp_f32(emb)
        if c.get("quant", True):
            pos = v["pos"][0].astype(F32) * v["pos"][1][:, None].astype(F32)
        else:  # the fp32 table (gemma.c:4453-4456)
            pos = np.asarray(v["pos"], F32)
        x = clamp_f32(x + pos)
        scale = F32(1.0) / F32(np.sqrt(F32(hd)))
        for ly in v["layers"]:
            resid = x
            h = layernorm(x, ly["n1"], ly["n1_b"], eps)
            q = self.gemm(ly["wq"], h) + ly["bq"]
            k = self.gemm(ly["wk"], h) + ly["bk"]
            vv = self.gemm(ly["wv"], h) + ly["bv"]
            att = np.empty_like(q)
            for hh in range(nh):
                sl = slice(hh * hd, (hh + 1) * hd)
                att[:, sl] = attention(q[:, sl], k[:, sl], vv[:, sl], scale)
            y = self.gemm(ly["wo"], att) + ly["bo"]
            x = clamp_f32(y + resid)
            resid = x
            h = layernorm(x, ly["n2"], ly["n2_b"], eps)
            f = self.gemm(ly["w1"], h) + ly["b1"]
            g = gelu_tanh(f).astype(F32)
            y = self.gemm(ly["w2"], g) + ly["b2"]
            x = clamp_f32(y + resid)
        h = layernorm(x, v["post_n"], v["post_nb"], eps)
        pooled = avg_pool(h, ppi, ppi // side)
        tok = np.stack([rmsnorm(r, v["norm"], eps) for r in pooled])
        return self.gemm(v["proj"], tok)
