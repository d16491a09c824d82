"""The prompt pass's attention kernels alone (gemma_hip_prefill_attention:
forward_text_chunk's blockwise attention, gemma.c:5152-5293, and its dense
form 5258-5290) against the decode oracle's attention formulas, before any
int8 requantization can amplify a difference.

Bars, relative to the largest output: the fp64 kernels (the verification
mode) round each output once from the fp64 value, so two fp32 ulps
(ATT_F64_TOL); the fp32 kernels (the default) carry the fp32 accumulation
error of the score, softmax and value sums over up to a few thousand keys
(ATT_F32_TOL, the vision tower's attention bar).  A wrong scale, mask, window
edge, softcap or key-split merge moves outputs by orders of magnitude more
(test_attention_bars_catch_planted_mistakes)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import decode_oracle as dorc

ATT_F64_TOL = 2.4e-7
ATT_F32_TOL = 2e-5
F32, F64 = np.float32, np.float64

# name: n rows, first position, q heads, kv heads, head dim, window (0: none),
# softcap, dense
CASES = {
    # gemma-3-1b widths (4 q heads on 1 kv head), a global layer
    "1b_global": (200, 0, 4, 1, 256, 0, 0.0, False),
    # gemma-3-4b widths (8 q heads on 4 kv heads): 2048 prompt rows through a
    # global layer, the longest key ranges (several key-split chunks)
    "4b_global_2048": (2048, 0, 8, 4, 256, 0, 0.0, False),
    # a sliding window of 16 at head dim 128, rows continuing a cache
    "hd128_window": (77, 30, 4, 2, 128, 16, 0.0, False),
    # the tanh softcap of the scores
    "softcap": (96, 5, 4, 1, 256, 0, 50.0, False),
    # the dense (image) rows: every key, no window
    "dense_256": (256, 1, 4, 1, 256, 8, 0.0, True),
    # a long cache behind a short chunk
    "long_cache": (48, 3000, 2, 1, 128, 0, 0.0, False),
}


def reference(q, kc, vc, n, pos0, nh, nkv, hd, slide, asc, sc_att, dense):
    """The oracle's attention (DecodeOracle.prefill's loop, decode_oracle.py)
    over given q rows and a given cache."""
    hn = nh // nkv
    ctx = pos0 + n
    pos = pos0 + np.arange(n)
    spos = np.where((pos >= slide) & (slide > 0), pos + 1 - slide, 0)
    out = np.empty((n, nh, hd), F32)
    j = np.arange(ctx)[None, :]
    live = np.ones((n, ctx), bool) if dense else (j <= pos[:, None]) & (j >= spos[:, None])
    for h in range(nh):
        keys = np.asarray(kc[h // hn, :ctx], F64)
        vals = np.asarray(vc[h // hn, :ctx], F64)
        s = np.asarray(q[:, h * hd:(h + 1) * hd], F64) @ keys.T * F64(asc)
        if sc_att != 0.0:
            s = np.tanh(s / F64(sc_att)) * F64(sc_att)
        s = np.where(live, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, h] = (p @ vals).astype(F32)
    return out.reshape(n, nh * hd)


def inputs(case):
    n, pos0, nh, nkv, hd, slide, sc_att, dense = CASES[case]
    rng = np.random.default_rng(n + pos0 + nh)
    stride = nh * hd + 2 * nkv * hd  # the fused q/k/v rows of the prompt pass
    q = rng.standard_normal((n, stride)).astype(F32)
    clen = pos0 + n + 3
    kc = rng.standard_normal((nkv, clen, hd)).astype(F32)
    vc = rng.standard_normal((nkv, clen, hd)).astype(F32)
    # cache rows past the last row's position are never read: NaN there
    # would reach every output of a kernel that multiplies one by a zero weight
    kc[:, pos0 + n:] = np.nan
    vc[:, pos0 + n:] = np.nan
    asc = F32(1.0) / np.sqrt(F32(hd))
    return q, kc, vc, clen, asc


def test_reference_matches_single_row_attend():
    """The batched reference against decode_oracle.attend, one row at a time."""
    q, kc, vc, clen, asc = inputs("hd128_window")
    n, pos0, nh, nkv, hd, slide, sc_att, dense = CASES["hd128_window"]
    want = reference(q, kc, vc, n, pos0, nh, nkv, hd, slide, asc, sc_att, dense)
    for i in (0, 17, n - 1):
        p = pos0 + i
        lo = max(0, p + 1 - slide)
        for h in range(nh):
            got = dorc.attend(q[i, h * hd:(h + 1) * hd], kc[h // 2, lo:p + 1], vc[h // 2, lo:p + 1],
                              asc, sc_att)
            assert np.allclose(got, want[i, h * hd:(h + 1) * hd], rtol=0, atol=1e-6)


def test_attention_bars_catch_planted_mistakes():
    """Plausible mistakes (window off by one, no softcap, the scale squared,
    causal rows in the dense path) move the outputs far past both bars."""
    for case, change in (("hd128_window", dict(slide=17)), ("softcap", dict(sc_att=0.0)),
                         ("1b_global", dict(asc2=True)), ("dense_256", dict(dense=False))):
        q, kc, vc, clen, asc = inputs(case)
        n, pos0, nh, nkv, hd, slide, sc_att, dense = CASES[case]
        good = reference(q, kc, vc, n, pos0, nh, nkv, hd, slide, asc, sc_att, dense)
        bad = reference(q, kc, vc, n, pos0, nh, nkv, hd, change.get("slide", slide),
                        asc * asc if change.get("asc2") else asc, change.get("sc_att", sc_att),
                        change.get("dense", dense))
        rel = float(np.abs(bad - good).max() / np.abs(good).max())
        assert rel > 100 * ATT_F32_TOL, (case, rel)


@pytest.mark.gpu
@pytest.mark.parametrize("case", sorted(CASES))
def test_prefill_attention_kernels_match_oracle(gh, case, monkeypatch):
    import torch

    from gemma_hip import ATTN_F32, ATTN_F64

    q, kc, vc, clen, asc = inputs(case)
    n, pos0, nh, nkv, hd, slide, sc_att, dense = CASES[case]
    want = reference(q, kc, vc, n, pos0, nh, nkv, hd, slide, asc, sc_att, dense)
    dq, dk, dv = (torch.from_numpy(a).cuda() for a in (q, kc, vc))
    scale = float(np.abs(want).max())
    # ATTN_F32 three times: the default choice (the split-bf16 kernel, or the
    # fp32-MFMA one for the smallest passes) and each kernel forced per launch
    # by GEMMA_HIP_PF_ATTN
    for mode, kernel, tol in ((ATTN_F64, "f64", ATT_F64_TOL), (ATTN_F32, "default", ATT_F32_TOL),
                              (ATTN_F32, "bf3", ATT_F32_TOL), (ATTN_F32, "f32", ATT_F32_TOL)):
        if kernel in ("bf3", "f32"):
            monkeypatch.setenv("GEMMA_HIP_PF_ATTN", kernel)
        else:
            monkeypatch.delenv("GEMMA_HIP_PF_ATTN", raising=False)
        out = torch.full((n, nh * hd), float("nan"), device="cuda")
        gh.prefill_attention(out, dq, q.shape[1], dk, dv, n, pos0, nh, nkv, hd, clen, slide, asc,
                             sc_att, dense, mode, stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        rel = float(np.abs(got - want).max()) / scale
        print(f"prefill attention {case} {kernel}: |d|/max = {rel:.3g}", flush=True)
        assert rel <= tol, (case, kernel, rel)
