"""CPU restatement of the reference's decode step, the checker of the
device-resident decoder.  TEST INFRASTRUCTURE ONLY: tests/ use it; nothing in
the product imports it.

Follows forward_gemma_decode (gemma.c:5456-5499) and forward_text_decode
(4727-4983) step by step.  The int8 parts are the pinned oracle's: quantize_act
from oracle/gemma_oracle.c and int32 sums in int64 numpy (exact), rescaled as
(float)acc * (xs * ws) in float32 (IEEE, the gcc -ffast-math order; no
operand here is near the FTZ range).  The fp32 glue -- rmsnorm (2508-2521),
clamp_fpx (2504-2506), RoPE (4178-4246), scores, att_finalize/softmax
(4091-4131), values, gelu_tanh (4139-4170) -- is computed in float64 from the
reference's formulas and rounded to float32 where the reference stores a
float32 tensor.  The reference leaves the fp32 summation order to its
compiler, so no bit pattern is canonical for the glue; float64 is the exact
value the GPU's and the CPU's float32 results are both checked against.

Pins: the int8 pieces are the pinned oracle functions; the glue formulas are
pinned by closed-form tests in tests/test_decoder.py (a one-hot attention,
RoPE's rotation invariants, rmsnorm of a constant vector) and by the
comparison with the reference program's own logits (tests/test_e2e.py).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
F64 = np.float64


def int_dot(a, b):
    """Exact int32 sums a @ b.T of int8 operands a [m][k], b [n][k] (or
    vectors), computed as a float64 product: every partial sum is an integer
    of magnitude <= k * 127^2 < 2^53 for k < 5e11, so float64 represents it
    exactly and the summation order cannot matter."""
    assert np.shape(a)[-1] * 127 * 127 < 2 ** 53
    r = np.asarray(a, F64) @ np.asarray(b, F64).T
    return r.astype(np.int64).astype(np.int32)


def rmsnorm(x, w, eps):
    """gemma.c:2508-2521: x * rsqrt(mean(x^2) + eps) * (w + 1), per row of x."""
    x = np.asarray(x, F64)
    rms = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + F64(F32(eps)))
    return (x * rms * (np.asarray(w, F64) + 1.0)).astype(F32)


def clamp_f32(x):
    """clamp_fpx (gemma.c:2504-2506) for fp32."""
    m = F64(np.finfo(F32).max)
    return np.clip(np.asarray(x, F64), -m, m).astype(F32)


def gelu_tanh(x):
    """gemma.c:4139-4145."""
    x = np.asarray(x, F64)
    return 0.5 * x * (1.0 + np.tanh(F64(F32(0.79788456080287)) * (x + F64(F32(0.044715)) * x ** 3)))


def rope_table(theta, hdim, pos):
    """rope_freqs_pos (gemma.c:4178-4196): freq = theta^(-2d/hdim) and the
    angle freq*pos rounded to float32 as the reference computes them; pos
    may be an array of positions (one table row each)."""
    d = np.arange(hdim // 2)
    ex = (F32(-2) * d.astype(F32)) / F32(hdim)
    freq = np.power(F64(F32(theta)), ex.astype(F64)).astype(F32)
    ang = (freq * np.asarray(pos, F32)[..., None]).astype(F32)
    return np.cos(ang.astype(F64)).astype(F32), np.sin(ang.astype(F64)).astype(F32)


def rope(x, cos, sin):
    """rope_apply (gemma.c:4223-4246) on head vectors (the last axis)."""
    h = np.shape(x)[-1] // 2
    a, b = np.asarray(x[..., :h], F64), np.asarray(x[..., h:], F64)
    c, s = cos.astype(F64), sin.astype(F64)
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1).astype(F32)


def attend(q, keys, vals, asc, sc_att):
    """One query head over its keys (gemma.c:4826-4851): scores k.q * asc,
    optional tanh softcap, softmax (att_finalize 4119-4131), value sum."""
    s = np.asarray(keys, F64) @ np.asarray(q, F64) * F64(asc)
    if sc_att != 0.0:
        s = np.tanh(s / F64(sc_att)) * F64(sc_att)
    p = np.exp(s - s.max())
    p /= p.sum()
    return (p @ np.asarray(vals, F64)).astype(F32)


class DecodeOracle:
    """One model's decode state (KV cache) on the CPU."""

    def __init__(self, model, oracle, clen: int):
        self.m = model
        self.c = model["config"]
        self.o = oracle
        c = self.c
        self.kc = np.zeros((c["nl"], c["nkv"], clen, c["hdim"]), F32)
        self.vc = np.zeros_like(self.kc)
        self.clen = clen

    def gemv(self, w, x_f32):
        """quantize_act + gemv_int8 (gemma.c:2590-2788): exact.  For an fp32
        ('U') model, gemv_fpx (2734-2757): the fp32 dot products evaluated in
        float64 and rounded once (the reference sums in its compiler's fp32
        order, so no fp32 result is canonical; the exact one is what both
        are checked against)."""
        if not self.c.get("quant", True):
            return (np.asarray(w, F64) @ np.asarray(x_f32, F64)).astype(F32)
        q, xs = self.o.quantize_act(np.ascontiguousarray(x_f32, F32))
        acc = int_dot(q, w[0])
        return acc.astype(F32) * (F32(xs) * np.asarray(w[1], F32))

    def gemm(self, w, x_f32):
        """quantize_acts + gemm_int8 (gemma.c:2652-2674, 3937-4054) over the
        rows of x_f32, exact; row i equals gemv(w, x_f32[i]) (for a 'U' model
        gemm_fpx, gemma.c:3308, as gemv does it)."""
        if not self.c.get("quant", True):
            return (np.asarray(x_f32, F64) @ np.asarray(w, F64).T).astype(F32)
        q, xs = self.o.quantize_acts(np.ascontiguousarray(x_f32, F32))
        acc = int_dot(q, w[0])
        return acc.astype(F32) * (xs[:, None] * np.asarray(w[1], F32)[None, :])

    def step(self, token: int, pos: int) -> np.ndarray:
        c, m = self.c, self.m
        dim, hd, nh, nkv = c["dim"], c["hdim"], c["n_heads"], c["nkv"]
        eps = c["eps"]
        esc = F32(1.0) if c["mlp_pre"] else F32(np.sqrt(F32(dim)))
        if c.get("quant", True):
            esc = F32(esc * m["emb"][1][token])
            x = (m["emb"][0][token].astype(F32) * esc).astype(F32)
        else:  # the fp32 row (gemma.c:5484-5486)
            x = (np.asarray(m["emb"][token], F32) * esc).astype(F32)
        asc = F32(1.0) / F32(np.sqrt(F32(c["q_scale"])))
        for li, ly in enumerate(m["layers"]):
            resid = x
            h = rmsnorm(x, ly["n1"], eps)
            q = self.gemv(ly["wq"], h).reshape(nh, hd)
            k = self.gemv(ly["wk"], h).reshape(nkv, hd)
            v = self.gemv(ly["wv"], h).reshape(nkv, hd)
            if c["qk_norm"]:
                q = np.stack([rmsnorm(qh, ly["nq"], eps) for qh in q])
                k = np.stack([rmsnorm(kh, ly["nk"], eps) for kh in k])
            sliding = bool(c["swa"][li])
            cos, sin = rope_table(c["theta_l"] if sliding else c["theta_g"], hd, pos)
            q = np.stack([rope(qh, cos, sin) for qh in q])
            k = np.stack([rope(kh, cos, sin) for kh in k])
            self.kc[li, :, pos] = k
            self.vc[li, :, pos] = v
            spos = pos + 1 - c["slide"] if (sliding and pos >= c["slide"]) else 0
            hn = nh // nkv
            xo = np.empty((nh, hd), F32)
            for hh in range(nh):
                kvh = hh // hn
                xo[hh] = attend(q[hh], self.kc[li, kvh, spos:pos + 1],
                                self.vc[li, kvh, spos:pos + 1], asc, c["sc_att"])
            y = self.gemv(ly["wo"], xo.reshape(-1))
            if c["mlp_pre"]:
                y = rmsnorm(y, ly["n2"], eps)
            x = clamp_f32(y.astype(F64) + resid.astype(F64))
            resid = x
            h = rmsnorm(x, ly["n3"] if c["mlp_pre"] else ly["n2"], eps)
            gate = self.gemv(ly["w2"], h)
            up = self.gemv(ly["w1"], h)
            g = (gelu_tanh(gate) * up.astype(F64)).astype(F32)
            y = self.gemv(ly["w3"], g)
            if c["mlp_pst"]:
                y = rmsnorm(y, ly["n4"], eps)
            x = clamp_f32(y.astype(F64) + resid.astype(F64))
        h = rmsnorm(x, m["fnorm"], eps)
        logits = self.gemv(m["emb"], h)
        if c["sc_log"] != 0.0:
            logits = (np.tanh(logits.astype(F64) / c["sc_log"]) * c["sc_log"]).astype(F32)
        return logits

    def prefill(self, tokens, pos0: int, rows=None, mask: bool = True) -> np.ndarray:
        """The prompt chunk of forward_gemma_prefill (gemma.c:5501) and
        forward_text_chunk (4985-5453): the tokens at positions pos0, pos0+1,
        ... go through each layer together, row i with step()'s formulas at
        position pos0 + i (causal, sliding-window attention over the cache).
        Fills the KV cache and returns the last row's logits.  Row for row it
        is step() vectorized; tests/test_decoder.py checks the two agree.

        rows (n x dim fp32) replaces the embedded tokens (tokens is then
        ignored): what forward_gemma_image (5561-5595) places in tb->x.
        mask=False is forward_text_chunk's dense path (5258-5290): every row
        attends to every key 0 .. pos0+n-1, with no sliding window."""
        c, m = self.c, self.m
        dim, hd, nh, nkv = c["dim"], c["hdim"], c["n_heads"], c["nkv"]
        eps = c["eps"]
        if rows is not None:
            x = np.array(rows, F32).reshape(-1, dim)
        else:
            toks = np.asarray(tokens, np.int64)
            esc0 = F32(1.0) if c["mlp_pre"] else F32(np.sqrt(F32(dim)))
            if c.get("quant", True):
                esc = (esc0 * np.asarray(m["emb"][1], F32)[toks]).astype(F32)
                x = (np.asarray(m["emb"][0])[toks].astype(F32) * esc[:, None]).astype(F32)
            else:
                x = (np.asarray(m["emb"], F32)[toks] * esc0).astype(F32)
        n = len(x)
        asc = F32(1.0) / F32(np.sqrt(F32(c["q_scale"])))
        pos = pos0 + np.arange(n)
        hn = nh // nkv
        for li, ly in enumerate(m["layers"]):
            resid = x
            h = rmsnorm(x, ly["n1"], eps)
            q = self.gemm(ly["wq"], h).reshape(n, nh, hd)
            k = self.gemm(ly["wk"], h).reshape(n, nkv, hd)
            v = self.gemm(ly["wv"], h).reshape(n, nkv, hd)
            if c["qk_norm"]:
                q = rmsnorm(q, ly["nq"], eps)
                k = rmsnorm(k, ly["nk"], eps)
            sliding = bool(c["swa"][li])
            cos, sin = rope_table(c["theta_l"] if sliding else c["theta_g"], hd, pos)
            q = rope(q, cos[:, None, :], sin[:, None, :])
            k = rope(k, cos[:, None, :], sin[:, None, :])
            self.kc[li, :, pos0:pos0 + n] = k.transpose(1, 0, 2)
            self.vc[li, :, pos0:pos0 + n] = v.transpose(1, 0, 2)
            if sliding:
                spos = np.where(pos >= c["slide"], pos + 1 - c["slide"], 0)
            else:
                spos = np.zeros(n, np.int64)
            ctx = pos0 + n
            xo = np.empty((n, nh, hd), F32)
            for hh in range(nh):
                keys = np.asarray(self.kc[li, hh // hn, :ctx], F64)
                vals = np.asarray(self.vc[li, hh // hn, :ctx], F64)
                for r0 in range(0, n, 512):
                    r1 = min(n, r0 + 512)
                    s = np.asarray(q[r0:r1, hh], F64) @ keys.T * F64(asc)
                    if c["sc_att"] != 0.0:
                        s = np.tanh(s / F64(c["sc_att"])) * F64(c["sc_att"])
                    j = np.arange(ctx)[None, :]
                    if mask:
                        live = (j <= pos[r0:r1, None]) & (j >= spos[r0:r1, None])
                    else:
                        live = np.ones((r1 - r0, ctx), bool)
                    s = np.where(live, s, -np.inf)
                    p = np.exp(s - s.max(axis=1, keepdims=True))
                    p /= p.sum(axis=1, keepdims=True)
                    xo[r0:r1, hh] = (p @ vals).astype(F32)
            y = self.gemm(ly["wo"], xo.reshape(n, -1))
            if c["mlp_pre"]:
                y = rmsnorm(y, ly["n2"], eps)
            x = clamp_f32(y.astype(F64) + resid.astype(F64))
            resid = x
            h = rmsnorm(x, ly["n3"] if c["mlp_pre"] else ly["n2"], eps)
            gate = self.gemm(ly["w2"], h)
            up = self.gemm(ly["w1"], h)
            g = (gelu_tanh(gate) * up.astype(F64)).astype(F32)
            y = self.gemm(ly["w3"], g)
            if c["mlp_pst"]:
                y = rmsnorm(y, ly["n4"], eps)
            x = clamp_f32(y.astype(F64) + resid.astype(F64))
        h = rmsnorm(x[-1], m["fnorm"], eps)
        logits = self.gemv(m["emb"], h)
        if c["sc_log"] != 0.0:
            logits = (np.tanh(logits.astype(F64) / c["sc_log"]) * c["sc_log"]).astype(F32)
        return logits
