"""The device-resident decoder on unquantized ('U') model files
(gemma_hip_decoder_create_f32) against the decode oracle's fp32 mode, and that
mode against the reference program's own fp32 forward pass.

A 'U' file takes the reference's !quant branches: gemv_fpx / gemv_fpx_multi in
the decode step (gemma.c:4762, 4855, 4906, 4925, 4960) and gemm_fpx in the
prompt pass (5079, 5297, 5358, 5384, 5431), with no activation quantize.  The
oracle evaluates those products in float64 and rounds once; the device sums
them in fp32 on its own order (the fp32 GEMV and the fp32 matrix-core GEMM,
each within 1e-5 of sum|a*b|, test_gpu_parity.py), the reference in its
compiler's.  With no int8 requantization to turn a rounding difference into a
whole int8 step, the differences stay at fp32 rounding through the layers:
logits must agree to U_LOGIT_TOL of the largest logit at every position, and
the argmax wherever the leader is clear of that bar.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import flips
import model_bin
from gemma_hip import ATTN_F32, ATTN_F64
from oracle import decode_oracle as dorc

U_LOGIT_TOL = 1e-4

CASES = {
    # gemma 3: qk norm, pre/post FFN norms, sliding window of 8, a global layer (5)
    "gemma3": dict(name="gemma-3-270m", layers=6, slide=8, flags=7),
    # gemma 2 style: no qk norm, attention and logit softcaps
    "softcap": dict(name="gemma-3-270m", layers=2, slide=8, flags=3, sc_att=50.0, sc_log=30.0),
    # gemma 1 style: no pre/post FFN norms (embedding scaled by sqrt(dim))
    "plain": dict(name="gemma-3-270m", layers=2, slide=4096, flags=0),
    # head dim 128, two q heads per kv head; widths off every GEMM tile
    "hd128": dict(name="test-hd128", layers=2, slide=8, flags=7),
    "odd": dict(name="test-odd", layers=2, slide=8, flags=7),
}


def write_u(path, key, seed=11, nvocab=1024):
    spec = dict(CASES[key])
    name = spec.pop("name")
    return model_bin.write_bin(str(path), name, seed=seed, nvocab=nvocab, norm_std=0.1,
                               quant=False, **spec)


@pytest.fixture(scope="module")
def u_models(tmp_path_factory):
    d = tmp_path_factory.mktemp("udec")
    return {key: model_bin.read_bin(write_u(d / f"{key}.bin", key)) for key in CASES}


def rel_err(got, want):
    return float(np.abs(got - want).max() / np.abs(want).max())


def check(got, want, nxt, what):
    rel = rel_err(got, want)
    assert rel <= U_LOGIT_TOL, f"{what}: {rel:.3g}"
    if flips.clear_argmax(want, U_LOGIT_TOL):
        assert nxt == int(np.argmax(want)), f"{what}: argmax"
    return rel


# ------------------------------------------------------------------ CPU
def test_u_models_are_fp32(u_models):
    m = u_models["gemma3"]
    assert m["config"]["quant"] is False
    assert m["emb"].dtype == np.float32 and m["layers"][0]["wq"].dtype == np.float32


def test_oracle_u_prefill_equals_steps(oracle, u_models):
    """The oracle's vectorized fp32 prefill against its own step(): the
    products are the same float64 sums, so logits and cache agree to float64
    rounding."""
    for key in CASES:
        model = u_models[key]
        nv = model["config"]["nvocab"]
        prompt = np.random.default_rng(4).integers(0, nv, 17).astype(np.int32)
        a = dorc.DecodeOracle(model, oracle, 20)
        b = dorc.DecodeOracle(model, oracle, 20)
        for pos, t in enumerate(prompt):
            want = a.step(int(t), pos)
        b.prefill(prompt[:9], 0)
        got = b.prefill(prompt[9:], 9)
        assert np.allclose(got, want, rtol=0, atol=1e-6 * float(np.abs(want).max())), key
        assert np.allclose(b.kc, a.kc, rtol=1e-6, atol=1e-6), key


def test_oracle_u_gemv_is_the_exact_product(oracle, u_models):
    """gemv/gemm of a 'U' model: the float64 product rounded once -- against
    math.fsum on a few rows (exact sums, an independent route)."""
    import math

    model = u_models["odd"]
    dec = dorc.DecodeOracle(model, oracle, 4)
    w = model["layers"][0]["w3"]
    x = np.random.default_rng(3).standard_normal(w.shape[1]).astype(np.float32)
    y = dec.gemv(w, x)
    for r in (0, 7, w.shape[0] - 1):
        exact = math.fsum(float(a) * float(b) for a, b in zip(w[r], x))
        assert y[r] == np.float32(exact)
    ym = dec.gemm(w, np.stack([x, 2 * x]))
    assert np.array_equal(ym[0], y) and np.array_equal(ym[1], dec.gemv(w, 2 * x))


REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
E2E_CPU = os.path.join(REPO, "oracle", "_ref", "gemma_e2e_cpu")
needs_e2e = pytest.mark.skipif(not os.path.exists(E2E_CPU),
                               reason="oracle/_ref/gemma_e2e_cpu not built (needs /root/reference)")


@needs_e2e
@pytest.mark.parametrize("key", ["gemma3", "plain", "softcap"])
def test_oracle_u_follows_reference_program(tmp_path, oracle, key):
    """The oracle's fp32 mode against the reference's own forward_gemma_decode
    on a 'U' file (teacher-forced on the reference's tokens): every row within
    U_LOGIT_TOL, the argmax where clear."""
    from test_e2e import run_reference_decode_only

    path = write_u(tmp_path / "u.bin", key, seed=21, nvocab=2048)
    seq, ref = run_reference_decode_only(path, 10, 10, tmp_path)
    model = model_bin.read_bin(path)
    dec = dorc.DecodeOracle(model, oracle, len(seq) + 1)
    worst = 0.0
    for pos, tok in enumerate(seq):
        got = dec.step(tok, pos)
        worst = max(worst, check(got, ref[pos], int(np.argmax(got)), f"{key} row {pos}"))
    print(f"U oracle vs reference ({key}): worst |d|/max|logit| {worst:.3g}", flush=True)


@needs_e2e
def test_u_reference_comparison_catches_a_planted_mistake(tmp_path, oracle):
    """The comparison above is sharp for the fp32 branches: the gemma 1
    embedding scale dropped (sqrt(dim) on the fp32 row, gemma.c:5470) or the
    up and gate projections swapped fails it at once."""
    from test_e2e import run_reference_decode_only

    path = write_u(tmp_path / "u.bin", "plain", seed=21, nvocab=2048)
    seq, ref = run_reference_decode_only(path, 4, 2, tmp_path)
    model = model_bin.read_bin(path)
    dim = model["config"]["dim"]
    model["emb"] = model["emb"] / np.float32(np.sqrt(np.float32(dim)))  # the scale undone
    dec = dorc.DecodeOracle(model, oracle, len(seq) + 1)
    got = [dec.step(t, p) for p, t in enumerate(seq)]
    assert max(rel_err(g, r) for g, r in zip(got, ref)) > 100 * U_LOGIT_TOL
    model = model_bin.read_bin(path)
    for ly in model["layers"]:
        ly["w1"], ly["w2"] = ly["w2"], ly["w1"]
    dec = dorc.DecodeOracle(model, oracle, len(seq) + 1)
    got = [dec.step(t, p) for p, t in enumerate(seq)]
    assert max(rel_err(g, r) for g, r in zip(got, ref)) > 100 * U_LOGIT_TOL


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
@pytest.mark.parametrize("key", sorted(CASES))
def test_u_decoder_steps_match_oracle(gh, oracle, u_models, key):
    model = u_models[key]
    clen = 40
    dec = gh.decoder(model, clen)
    try:
        ref = dorc.DecodeOracle(model, oracle, clen)
        logits = np.empty(model["config"]["nvocab"], np.float32)
        token, worst = 2, 0.0
        for pos in range(36):
            nxt = dec.step(token, pos, logits)
            want = ref.step(token, pos)
            worst = max(worst, check(logits, want, nxt, f"{key} step {pos}"))
            assert nxt == int(np.argmax(logits))
            token = int(np.argmax(want))
        print(f"U decoder {key}: worst |d|/max|logit| = {worst:.3g}", flush=True)
    finally:
        dec.close()


# One layer at the real widths of gemma-3-1b (dim 1152: 32 lanes per row in
# the norm-fused GEMVs) and gemma-3-4b (dim 2560: 64 lanes for q/k/v, 32 in
# three passes for the gate/up pairing), and at dim 704 (one pass of 12
# chunks per lane), decode steps and then a prompt pass (the fp32 GEMMs at
# these widths split K).
@pytest.mark.gpu
@pytest.mark.parametrize("name", ["gemma-3-1b", "gemma-3-4b", "test-cpl12"])
def test_u_decoder_real_widths_match_oracle(gh, oracle, tmp_path, name):
    path = model_bin.write_bin(str(tmp_path / "w.bin"), name, seed=5, nvocab=1024,
                               norm_std=0.1, quant=False, layers=1, slide=8, flags=7)
    model = model_bin.read_bin(path)
    nv = model["config"]["nvocab"]
    clen = 40
    dec = gh.decoder(model, clen)
    try:
        ref = dorc.DecodeOracle(model, oracle, clen)
        logits = np.empty(nv, np.float32)
        token, worst = 3, 0.0
        for pos in range(6):
            nxt = dec.step(token, pos, logits)
            want = ref.step(token, pos)
            worst = max(worst, check(logits, want, nxt, f"{name} step {pos}"))
            token = int(np.argmax(want))
        prompt = np.random.default_rng(4).integers(0, nv, 20).astype(np.int32)
        want = ref.prefill(prompt, 6)
        nxt = dec.prefill(prompt, 6, logits)
        worst = max(worst, check(logits, want, nxt, f"{name} prefill"))
        token = int(np.argmax(want))
        for pos in range(26, 30):
            nxt = dec.step(token, pos, logits)
            want = ref.step(token, pos)
            worst = max(worst, check(logits, want, nxt, f"{name} step {pos}"))
            token = int(np.argmax(want))
        print(f"U decoder {name} (1 layer): worst |d|/max|logit| = {worst:.3g}", flush=True)
    finally:
        dec.close()


@pytest.mark.gpu
@pytest.mark.parametrize("key", ["gemma3", "softcap", "plain", "odd"])
@pytest.mark.parametrize("mode", [ATTN_F64, ATTN_F32])
def test_u_prefill_matches_oracle(gh, oracle, u_models, key, mode):
    """The fp32 prompt pass (two chunks) against the oracle's prefill, then
    decode steps on the cache it filled."""
    model = u_models[key]
    nv = model["config"]["nvocab"]
    prompt = np.random.default_rng(9).integers(0, nv, 29).astype(np.int32)
    clen = 40
    dec = gh.decoder(model, clen, attention=mode)
    try:
        ref = dorc.DecodeOracle(model, oracle, clen)
        ref.prefill(prompt[:11], 0)
        want = ref.prefill(prompt[11:], 11)
        logits = np.empty(nv, np.float32)
        dec.prefill(prompt[:11], 0)
        nxt = dec.prefill(prompt[11:], 11, logits)
        worst = check(logits, want, nxt, f"{key} prefill")
        token = int(np.argmax(want))
        for pos in range(29, 35):
            nxt = dec.step(token, pos, logits)
            want = ref.step(token, pos)
            worst = max(worst, check(logits, want, nxt, f"{key} step {pos}"))
            token = int(np.argmax(want))
        print(f"U prefill {key} mode {mode}: worst {worst:.3g}", flush=True)
    finally:
        dec.close()


@pytest.mark.gpu
def test_u_decoder_generate_and_perf(gh, u_models):
    """generate() equals step-by-step greedy decoding, and the per-op timing
    names the fp32 products as the reference's fp32 ops (gemv_fpx in the
    step, gemm_fpx in the prompt pass)."""
    model = u_models["gemma3"]
    nl = model["config"]["nl"]
    dec = gh.decoder(model, 48)
    try:
        toks = list(dec.generate(5, 0, 30))
        token, seq = 5, []
        for pos in range(30):
            token = dec.step(token, pos)
            seq.append(token)
        assert toks == seq
        gh.perf_enable(True)
        try:
            dec.prefill([3, 1, 4, 1, 5], 0)
            assert list(dec.generate(9, 5, 4)) == list(dec.generate(9, 5, 4))
            perf = gh.perf_read()
        finally:
            gh.perf_enable(False)
        calls = {ph: {op: c for op, (s, c) in ops.items()} for ph, ops in perf.items()}
        # per layer q|k|v and gate|up one launch each over the adjacent
        # matrices, o and down one each (the decode step's grouping)
        assert calls["prefill"]["gemm_fpx"] == 4 * nl
        assert calls["prefill"]["gemv_fpx"] == 1 and calls["prefill"]["gelu"] == nl
        assert "gemm_int8" not in calls["prefill"] and "quantize_act" not in calls["prefill"]
        # per token: the norm-fused q/k/v and gate/up GEMVs (GELU fused), o,
        # down, the LM head; the final norm the only separate one
        assert calls["decode"]["gemv_fpx"] == 8 * (4 * nl + 1)
        assert calls["decode"]["rmsnorm"] == 8
        assert "gelu" not in calls["decode"]
        assert "gemv_int8" not in calls["decode"]
    finally:
        dec.close()


@pytest.mark.gpu
def test_u_decoder_argument_errors(gh, u_models):
    import ctypes

    import gemma_hip

    model = u_models["plain"]
    c = model["config"]
    swa = np.asarray(c["swa"], np.uint8)
    cfg = gemma_hip.TextConfig(c["nl"], c["n_heads"], c["nkv"], c["hdim"], c["dim"],
                               c["mlp_dim"], c["q_scale"], c["slide"], c["nvocab"],
                               c["theta_l"], c["theta_g"], c["eps"], 0.0, 0.0, 0, 0, 0,
                               swa.ctypes.data)
    layers = (gemma_hip.LayerF32 * c["nl"])()
    stray = np.zeros(16, np.float32)
    h = gh.lib.gemma_hip_decoder_create_f32(ctypes.byref(cfg), layers, stray.ctypes.data,
                                            stray.ctypes.data, 16)
    assert not h and b"not registered" in gh.lib.gemma_hip_last_error()
    h = gh.lib.gemma_hip_decoder_create_f32(ctypes.byref(cfg), layers, None, None, 16)
    assert not h and b"null argument" in gh.lib.gemma_hip_last_error()
