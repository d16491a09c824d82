"""Image prompts: the vision tower's soft tokens through the decoder with the
dense (mask=false) attention of forward_gemma_image (gemma.c:5561-5595,
forward_text_chunk's dense path 5258-5290), on the device
(gemma_hip_decoder_prefill_rows, gemma_hip_gemma_image) against the decode
oracle (oracle/decode_oracle.py, DecodeOracle.prefill(rows=..., mask=False))
and against the reference program itself (oracle/e2e_harness.c,
GEMMA_E2E_IMAGE).

Bars: device against oracle as in tests/test_decoder.py (both evaluate the
glue in fp64 and round once: logits to LOGIT_TOL of their largest entry, the
same argmax).  Oracle or device against the reference program: the reference
evaluates the glue in fp32, so the two agree to fp32 rounding (measured
6e-8 .. 3.2e-7 of the largest logit) until an fp32 difference straddles an
int8 requantization boundary, which moves this random model's logits by 1%
to 4% from there on.  Which applies is decided before the run from the
oracle's requantization margins over the whole chain (tests/flips.py): a
chain the criterion clears is held to REL_PRE_FLIP, any other to the flip
level, with the argmax wherever the reference's lead exceeds what that level
can move.  The tight bound is sharp: causal attention over the image block
moves the logits by 13% to 20%, and a sliding window kept in the dense path
(16 image tokens under a window of 8) by 48%.
"""

from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import pytest

import model_bin
from gemma_hip import ATTN_F32, ATTN_F64
from oracle import decode_oracle as dorc
from oracle import vision_oracle as vorc

import flips

LOGIT_TOL = 1e-5
REL_PRE_FLIP = 1e-5
REL_FLIP_LEVEL = 5e-2

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
E2E_CPU = os.path.join(REPO, "oracle", "_ref", "gemma_e2e_cpu")
needs_e2e = pytest.mark.skipif(not os.path.exists(E2E_CPU),
                               reason="oracle/_ref/gemma_e2e_cpu not built (needs /root/reference)")

VISION = {
    # SigLIP's head dim (72), 16 patches pooled to 4 tokens
    "hd72": dict(nl=2, n_heads=2, img_px=56, psize=14, dim=144, mlp_dim=288, img_tok=4),
    # 64 patches pooled to 16 tokens: the image block is longer than the window of 8
    "hd16": dict(nl=3, n_heads=4, img_px=112, psize=14, dim=64, mlp_dim=128, img_tok=16),
    # SigLIP's own widths at 224 px, pooled to 16 tokens
    "siglip": dict(nl=2, n_heads=16, img_px=224, psize=14, dim=1152, mlp_dim=4304, img_tok=16),
    # 256 patches, unpooled: a gemma-3 image's 256 soft tokens
    "tok256": dict(nl=1, n_heads=2, img_px=224, psize=14, dim=64, mlp_dim=128, img_tok=256),
}
# shape, vision weight seed, image seed, text layers (the bar of each comes
# from the margin criterion; hd72_s7 and hd16_s8 are seeds taken as they come)
REF_CASES = {"hd72": ("hd72", 1, 101, 2), "hd16": ("hd16", 4, 104, 2),
             "tok256": ("tok256", 2, 102, 1), "hd72_s7": ("hd72", 7, 107, 2),
             "hd16_s8": ("hd16", 8, 108, 2)}


def mm_model(path, shape, seed, layers=2, text="gemma-3-270m"):
    """A multimodal file: text layers of `text`'s widths (a sliding window of
    8, then a global layer) under the tower `shape`."""
    dim = model_bin.CONFIGS[text]["dim"]
    vis = model_bin.synth_vision(seed=seed, text_dim=dim, **VISION[shape])
    return model_bin.read_bin(model_bin.write_bin(str(path), text, seed=5, nvocab=512,
                                                  layers=layers, vision=vis, norm_std=0.1,
                                                  slide=8, swa=[1, 0][:layers]))


def oracle_chain(model, oracle, img, bos, prompt, tokens, steps, clen):
    """The oracle through sample()'s image prompt: <bos>, the image's soft
    tokens (dense), the text prompt, then `steps` teacher-forced decode steps
    on `tokens`; the logits after each stage."""
    soft = vorc.VisionOracle(model["vision"], oracle).forward(img)
    d = dorc.DecodeOracle(model, oracle, clen)
    d.prefill([bos], 0)
    out = [d.prefill(None, 1, rows=soft, mask=False)]
    pos = 1 + len(soft)
    if len(prompt):
        out.append(d.prefill(prompt, pos))
        pos += len(prompt)
    for i in range(steps):
        out.append(d.step(int(tokens[i]), pos))
        pos += 1
    return np.array(out), soft


def device_chain(gh, model, img, bos, prompt, tokens, steps, clen, attention):
    """The device through the same stages (gemma_hip_gemma_image for the
    image), the tower's and the prompt passes' attention in `attention`."""
    nv = model["config"]["nvocab"]
    dec = gh.decoder(model, clen, attention=attention)
    tower = gh.vision(model["vision"], attention=attention)
    try:
        out, nxt = [], []
        lg = np.empty(nv, np.float32)
        dec.prefill(np.array([bos], np.int32), 0)
        pos, first = dec.image(tower, img, 1, lg)
        out.append(lg.copy())
        nxt.append(first)
        if len(prompt):
            nxt.append(dec.prefill(np.asarray(prompt, np.int32), pos, lg))
            out.append(lg.copy())
            pos += len(prompt)
        for i in range(steps):
            nxt.append(dec.step(int(tokens[i]), pos, lg))
            out.append(lg.copy())
            pos += 1
        return np.array(out), nxt, pos
    finally:
        tower.close()
        dec.close()


def rel_rows(got, ref):
    return np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)


def check_against_reference(got, ref, margin, what):
    """Every stage's logits within the bar the oracle's margin sets, and the
    argmax of every stage where the reference's lead is clear of that bar."""
    free = margin > flips.MARGIN_BOUND
    bar = REL_PRE_FLIP if free else REL_FLIP_LEVEL
    rel = rel_rows(got, ref)
    print(f"{what} ({'flip-free' if free else 'may flip'}): "
          f"{np.array2string(rel, precision=2)}", flush=True)
    assert rel.max() <= bar
    for i, (g, r) in enumerate(zip(got, ref)):
        if flips.clear_argmax(r, bar):
            assert int(np.argmax(g)) == int(np.argmax(r)), f"{what}: stage {i}"


def run_reference_image(tmp_path, case, prompt_len=5, steps=3):
    shape, seed, img_seed, layers = REF_CASES[case]
    path = tmp_path / f"mm_{case}.bin"
    model = mm_model(path, shape, seed, layers)
    img = model_bin.synth_image(VISION[shape]["img_px"], seed=img_seed)
    img_path, lg_path = tmp_path / "img.f32", tmp_path / "logits.f32"
    img.tofile(img_path)
    env = dict(os.environ, GEMMA_E2E_IMAGE=str(img_path), GEMMA_E2E_LOGITS=str(lg_path))
    out = subprocess.run([E2E_CPU, str(path), str(prompt_len), str(steps), "77", "4"], env=env,
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])
    ref = np.fromfile(lg_path, np.float32).reshape(-1, model["config"]["nvocab"])
    assert len(ref) == 2 + steps and res["img_tok"] == VISION[shape]["img_tok"]
    return model, img, res, ref


# ------------------------------------------------------------ oracle pins (CPU)
@pytest.fixture(scope="module")
def text_models(tmp_path_factory):
    d = tmp_path_factory.mktemp("img_text")
    out = {}
    for key, layers in (("one", 1), ("two", 2)):
        out[key] = model_bin.read_bin(model_bin.write_bin(
            str(d / f"{key}.bin"), "gemma-3-270m", seed=13, nvocab=512, layers=layers,
            swa=[0] * layers, norm_std=0.1))
    return out


def _embed(model, toks):
    emb_q, emb_s = model["emb"]
    return (emb_q[toks].astype(np.float32) * emb_s[toks][:, None]).astype(np.float32)


def test_oracle_rows_equal_tokens(oracle, text_models):
    """Rows that are the tokens' own embeddings (gemma 3: esc = 1, times the
    row scale, gemma.c:5468-5493) give the token prefill's logits and cache."""
    model = text_models["two"]
    toks = np.random.default_rng(1).integers(0, 512, 11)
    a = dorc.DecodeOracle(model, oracle, 16)
    b = dorc.DecodeOracle(model, oracle, 16)
    want = a.prefill(toks, 2)
    got = b.prefill(None, 2, rows=_embed(model, toks))
    assert np.array_equal(got, want)
    assert np.array_equal(a.kc, b.kc) and np.array_equal(a.vc, b.vc)


def test_oracle_dense_closed_forms(oracle, text_models):
    """The last row of a chunk sees every key 0 .. pos0+n-1 with or without the
    causal mask, so in a single global layer its logits are the same both ways
    (and k/v, written before attention, are too); with a second layer the
    earlier rows' dense outputs reach it through that layer's keys and values,
    so the logits must move."""
    toks = np.random.default_rng(2).integers(0, 512, 9)
    for key, same in (("one", True), ("two", False)):
        model = text_models[key]
        rows = _embed(model, toks)
        a = dorc.DecodeOracle(model, oracle, 16)
        b = dorc.DecodeOracle(model, oracle, 16)
        a.prefill([2], 0)
        b.prefill([2], 0)
        causal = a.prefill(None, 1, rows=rows, mask=True)
        dense = b.prefill(None, 1, rows=rows, mask=False)
        rel = float(np.abs(dense - causal).max() / np.abs(causal).max())
        if same:
            assert rel <= 1e-12, rel
            assert np.array_equal(a.kc, b.kc) and np.array_equal(a.vc, b.vc)
        else:
            assert rel > 1e-3, rel


@needs_e2e
@pytest.mark.parametrize("case", sorted(REF_CASES))
def test_oracle_image_follows_reference_program(tmp_path, oracle, case):
    """forward_gemma_image and the text after it, compiled from the
    reference's source, against the oracle's chain, stage by stage."""
    model, img, res, ref = run_reference_image(tmp_path, case)
    clen = 1 + res["img_tok"] + len(res["prompt"]) + len(res["tokens"])
    (got, _), margin = flips.tracked(oracle, oracle_chain, model, oracle, img, res["bos"],
                                     res["prompt"], res["tokens"], len(ref) - 2, clen)
    check_against_reference(got, ref, margin, f"oracle vs reference image prompt ({case})")


@needs_e2e
def test_image_comparison_catches_causal_mask(tmp_path, oracle, monkeypatch):
    """The same comparison with the image block under the causal mask (the
    text path's attention) fails by far."""
    model, img, res, ref = run_reference_image(tmp_path, "hd16")
    prefill = dorc.DecodeOracle.prefill
    monkeypatch.setattr(dorc.DecodeOracle, "prefill",
                        lambda self, t, p, rows=None, mask=True: prefill(self, t, p, rows, True))
    clen = 1 + res["img_tok"] + len(res["prompt"]) + len(res["tokens"])
    got, _ = oracle_chain(model, oracle, img, res["bos"], res["prompt"], res["tokens"],
                          len(ref) - 2, clen)
    assert rel_rows(got, ref)[0] > 100 * REL_PRE_FLIP


# ------------------------------------------------------------------ GPU
@pytest.fixture(scope="module")
def gqa_model(tmp_path_factory):
    """gemma-3-4b widths (8 q heads over 4 kv heads of 256), a sliding layer
    (window 8) then a global one: the shape config 2's 256 image tokens take."""
    d = tmp_path_factory.mktemp("img_gqa")
    return model_bin.read_bin(model_bin.write_bin(str(d / "gqa.bin"), "gemma-3-4b", seed=5,
                                                  nvocab=1024, layers=2, slide=8, swa=[1, 0],
                                                  norm_std=0.1))


def _check(got, want, what):
    scale = float(np.abs(want).max())
    diff = float(np.abs(got - want).max())
    assert diff <= LOGIT_TOL * scale, f"{what}: |d| {diff:.3g} vs {scale:.3g}"
    return diff / scale


@pytest.mark.gpu
def test_prefill_rows_equal_token_prefill(gh, text_models):
    """Rows holding the tokens' embeddings through the causal path give the
    token prefill's logits bit for bit (the device embeds in the same fp32
    product), and the same next token."""
    model = text_models["two"]
    toks = np.random.default_rng(3).integers(0, 512, 40).astype(np.int32)
    lg_a, lg_b = np.empty(512, np.float32), np.empty(512, np.float32)
    dec = gh.decoder(model, 48)
    try:
        na = dec.prefill(toks, 3, lg_a)
        nb = dec.prefill_rows(_embed(model, toks), 3, True, lg_b)
    finally:
        dec.close()
    assert na == nb and np.array_equal(lg_a, lg_b)


@pytest.mark.gpu
@pytest.mark.parametrize("n,pos0", [(256, 1), (77, 30), (1, 5)])
def test_prefill_rows_dense_matches_oracle(gh, oracle, gqa_model, n, pos0):
    """Dense rows at gemma-3-4b widths: 256 rows (one image of config 2) after
    <bos>, a ragged block that starts past the window and ends inside an
    attention tile, and a single row; then decode steps over the cache."""
    model = gqa_model
    nv, dim = model["config"]["nvocab"], model["config"]["dim"]
    rng = np.random.default_rng(n)
    rows = (rng.standard_normal((n, dim)) * 0.5).astype(np.float32)
    prefix = rng.integers(0, nv, pos0).astype(np.int32)
    clen = pos0 + n + 4
    dec = gh.decoder(model, clen, attention=ATTN_F64)
    try:
        ref = dorc.DecodeOracle(model, oracle, clen)
        ref.prefill(prefix, 0)
        want = ref.prefill(None, pos0, rows=rows, mask=False)
        lg = np.empty(nv, np.float32)
        dec.prefill(prefix, 0)
        nxt = dec.prefill_rows(rows, pos0, False, lg)
        worst = _check(lg, want, f"dense rows {n} at {pos0}")
        assert nxt == int(np.argmax(want))
        token, pos = nxt, pos0 + n
        for _ in range(3):
            nxt = dec.step(token, pos, lg)
            want = ref.step(token, pos)
            worst = max(worst, _check(lg, want, f"step at {pos} after dense rows"))
            assert nxt == int(np.argmax(want))
            token, pos = nxt, pos + 1
    finally:
        dec.close()
    print(f"dense rows {n} at {pos0}: worst |d|/max|logit| = {worst:.3g}", flush=True)


# The dense rows with the prompt pass's attention on the fp32 matrix cores
# (GEMMA_HIP_ATTN_F32: the fp32 kernel's bidirectional form, head dims 256
# and 128) against the fp64 oracle, the bar from the margin criterion as in
# test_decoder.py (fp32 rounding where the oracle's pass is clear of every
# requantization boundary; else the flip level, measured 1.2% .. 1.8%, and
# the argmax where its lead is clear).  The dense kernels themselves are
# pinned before any requantization in tests/test_attention.py.
F32_PRE_FLIP = 1e-6
F32_FLIP_LEVEL = 5e-2
F32_DENSE_CASES = [  # model, rows, first position
    ("two", 77, 30), ("two", 256, 1), ("hd128", 77, 30), ("hd128", 200, 3), ("gqa", 1, 5),
    ("gqa", 77, 30), ("gqa", 256, 1)]


@pytest.fixture(scope="module")
def hd128_model(tmp_path_factory):
    d = tmp_path_factory.mktemp("hd128")
    return model_bin.read_bin(model_bin.write_bin(str(d / "hd128.bin"), "test-hd128", seed=7,
                                                  nvocab=512, layers=2, slide=16, flags=7,
                                                  norm_std=0.1))


@pytest.mark.gpu
@pytest.mark.parametrize("key,n,pos0", F32_DENSE_CASES)
def test_prefill_rows_dense_f32_attention(gh, oracle, text_models, hd128_model, gqa_model, key,
                                          n, pos0):
    model = {"two": text_models.get("two"), "hd128": hd128_model, "gqa": gqa_model}[key]
    nv, dim = model["config"]["nvocab"], model["config"]["dim"]
    rng = np.random.default_rng(n)
    rows = (rng.standard_normal((n, dim)) * 0.5).astype(np.float32)
    prefix = rng.integers(0, nv, pos0).astype(np.int32)
    clen = pos0 + n + 4
    dec = gh.decoder(model, clen)
    try:
        dec.set_attention(dec.ATTN_F32)
        ref = dorc.DecodeOracle(model, oracle, clen)
        oracle.track_margins()
        try:
            ref.prefill(prefix, 0)
            want = ref.prefill(None, pos0, rows=rows, mask=False)
            free = oracle.min_margin() > flips.MARGIN_BOUND
        finally:
            oracle.margins = None
        lg = np.empty(nv, np.float32)
        dec.prefill(prefix, 0)
        nxt = dec.prefill_rows(rows, pos0, False, lg)
    finally:
        dec.close()
    bar = F32_PRE_FLIP if free else F32_FLIP_LEVEL
    rel = float(np.abs(lg - want).max() / np.abs(want).max())
    print(f"dense rows {key} {n} at {pos0}, fp32 attention "
          f"({'flip-free' if free else 'may flip'}): {rel:.3g}", flush=True)
    assert rel <= bar
    if flips.clear_argmax(want, bar):
        assert nxt == int(np.argmax(want))


@pytest.mark.gpu
@pytest.mark.parametrize("shape", sorted(VISION))
def test_gemma_image_matches_oracle(gh, oracle, tmp_path, shape):
    """gemma_hip_gemma_image (tower -> soft tokens in HBM -> dense prefill)
    and the text after it against the oracle's chain, stage by stage."""
    model = mm_model(tmp_path / f"{shape}.bin", shape, 2)
    img = model_bin.synth_image(VISION[shape]["img_px"], seed=9)
    prompt = np.random.default_rng(5).integers(0, 512, 6)
    tokens = np.random.default_rng(6).integers(0, 512, 3)
    clen = 1 + VISION[shape]["img_tok"] + 6 + 3
    got, nxt, pos = device_chain(gh, model, img, 2, prompt, tokens, 3, clen, ATTN_F64)
    want, _ = oracle_chain(model, oracle, img, 2, prompt, tokens, 3, clen)
    assert pos == clen
    worst = max(_check(g, w, f"{shape} stage {i}") for i, (g, w) in enumerate(zip(got, want)))
    assert nxt == [int(np.argmax(w)) for w in want]
    print(f"image {shape}: worst |d|/max|logit| = {worst:.3g}", flush=True)


@pytest.mark.gpu
@needs_e2e
@pytest.mark.parametrize("case", sorted(REF_CASES))
@pytest.mark.parametrize("mode", ["f32", "f64"])
def test_device_image_follows_reference_program(gh, oracle, tmp_path, case, mode):
    """The device chain against forward_gemma_image compiled from the
    reference's source (bars from the margin criterion, as above), with the
    attention in fp32 (the default) and in fp64."""
    model, img, res, ref = run_reference_image(tmp_path, case)
    clen = 1 + res["img_tok"] + len(res["prompt"]) + len(res["tokens"])
    _, margin = flips.tracked(oracle, oracle_chain, model, oracle, img, res["bos"],
                              res["prompt"], res["tokens"], len(ref) - 2, clen)
    got, nxt, _ = device_chain(gh, model, img, res["bos"], res["prompt"], res["tokens"],
                               len(ref) - 2, clen, ATTN_F32 if mode == "f32" else ATTN_F64)
    check_against_reference(got, ref, margin, f"device ({mode}) vs reference image prompt ({case})")


@pytest.mark.gpu
def test_image_argument_errors(gh, tmp_path, text_models):
    from gemma_hip import GemmaHipError

    model = mm_model(tmp_path / "mm.bin", "hd72", 1)
    img = model_bin.synth_image(VISION["hd72"]["img_px"], seed=1)
    dec = gh.decoder(model, 8)
    tower = gh.vision(model["vision"])
    other = gh.decoder(text_models["two"], 8)
    narrow = gh.vision(model_bin.synth_vision(seed=1, text_dim=64, **VISION["hd72"]))
    try:
        with pytest.raises(GemmaHipError, match="out of range"):
            dec.image(tower, img, 5)  # 4 soft tokens at 5 .. 8 do not fit a cache of 8
        with pytest.raises(GemmaHipError, match="projects to 64"):
            other.image(narrow, img, 0)
        with pytest.raises(GemmaHipError, match="out of range"):
            dec.prefill_rows(np.zeros((0, 640), np.float32), 0, False)
        assert dec.image(tower, img, 4)[0] == 8  # and the last fitting position works
    finally:
        narrow.close()
        other.close()
        tower.close()
        dec.close()
