"""End-to-end greedy generation through the reference program itself.

oracle/_ref/gemma_e2e_cpu is gemma.c as it is; oracle/_ref/gemma_e2e_hip is
the same source with its forward passes' quantize_act / quantize_acts /
gemv_int8 / gemv_int8_multi / gemm_int8 calls going to libgemma_hip's host
entry points (oracle/e2e_harness.c, oracle/e2e_retarget.sed).  Everything
else (embedding, norms, RoPE, attention, GELU, argmax) is the reference's
code in both, built with the same flags, so the bar is bit-identical logits
at every step -- hashed over all steps -- and the same greedy tokens.

Models are random-init .bin files in the reference's layout
(gemma.c_amd/model_bin.py), at the BASELINE.json end-to-end shapes: config 1
(gemma-3-270m, 32 prompt ids, 64 decode steps) and config 3's prefill
(gemma-3-1b, 512 prompt ids) with a shortened decode.
"""

from __future__ import annotations

import json
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

import flips
import model_bin

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
E2E_CPU = os.path.join(REPO, "oracle", "_ref", "gemma_e2e_cpu")
E2E_HIP = os.path.join(REPO, "oracle", "_ref", "gemma_e2e_hip")
THREADS = max(1, min(16, os.cpu_count() or 1))

needs_e2e = pytest.mark.skipif(
    not (os.path.exists(E2E_CPU) and os.path.exists(E2E_HIP)),
    reason="oracle/_ref e2e harnesses not built (they need /root/reference)")


def run_e2e(binary, model, prompt_len, steps, threads=THREADS, chunk=None, seed=1234,
            logits=None):
    cmd = [binary, model, str(prompt_len), str(steps), str(seed), str(threads)]
    if chunk is not None:
        cmd.append(str(chunk))
    print("run:", " ".join(cmd), flush=True)
    env = dict(os.environ)
    if logits is not None:
        env["GEMMA_E2E_LOGITS"] = str(logits)
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600, env=env)
    assert out.returncode == 0, f"{binary} exited {out.returncode}: {out.stderr[-2000:]}"
    res = json.loads(out.stdout.strip().splitlines()[-1])
    summary = {k: res[k] for k in ("build", "prefill_tok_s", "decode_tok_s", "setup_s",
                                   "logits_fnv")}
    print(json.dumps(summary), flush=True)
    sys.stdout.flush()
    return res


# ------------------------------------------------------------------ CPU
def test_model_bin_header_round_trip(tmp_path):
    """The writer's header, read back field by field (gemma.c:770-816)."""
    path = model_bin.write_bin(str(tmp_path / "m.bin"), "gemma-3-1b", seed=3,
                               nvocab=300, layers=7)
    with open(path, "rb") as f:
        assert f.read(8) == b"GEMAf32Q"
        cfg = struct.unpack(">BBBHHHHHHIIfffff", f.read(43))
        assert cfg[:11] == (7, 4, 1, 256, 1152, 6912, 256, 512, 256, 32768, 300)
        assert cfg[11:] == (10000.0, 1000000.0, struct.unpack(">f", struct.pack(">f", 1e-6))[0],
                            0.0, 0.0)
        nbytes = f.read(1)[0]
        swa = f.read(nbytes)
        bits = [(swa[i // 8] >> (7 - i % 8)) & 1 for i in range(7)]
        assert bits == [1, 1, 1, 1, 1, 0, 1]  # every sixth layer is global
        assert f.read(1)[0] == 7
        words = []
        for _ in range(300):
            n = f.read(1)[0]
            words.append(f.read(n).decode())
        assert words[:6] == model_bin.SPECIALS and words[299] == "t299"
        assert struct.unpack(">I", f.read(4))[0] == 1
        f.read(2 + 2)  # the one merge: "t" + "0"
        tensors_at = f.tell()
    dim, q, kv, mlp = 1152, 1024, 256, 6912
    qt = lambda n, k: n * k + 4 * n  # noqa: E731
    per_layer = (qt(q, dim) + 2 * qt(kv, dim) + qt(dim, q) + 2 * 256 * 4
                 + 2 * qt(mlp, dim) + qt(dim, mlp) + 4 * dim * 4)
    assert os.path.getsize(path) == tensors_at + qt(300, dim) + 7 * per_layer + dim * 4


def test_model_bin_weights_quantize_like_export():
    """Per-row int8 weights: the largest |w| of each row maps to +-127 and the
    scale is max(amax, 1e-8) / 127 (model.py:151-161)."""
    import numpy as np

    rng = np.random.default_rng(0)
    w = rng.standard_normal((64, 96)).astype(np.float32) * np.float32(0.02)
    w[5] = 0.0
    q, s = model_bin.quantize_rows(w)
    amax = np.abs(w).max(axis=1)
    assert np.all(np.abs(q[np.arange(64) != 5]).max(axis=1) == 127)
    assert not q[5].any() and s[5] == np.float32(1e-8) / np.float32(127)
    err = np.abs(q.astype(np.float32) * s[:, None] - w)
    assert np.all(err <= s[:, None] * 0.5000001)
    assert np.allclose(s[np.arange(64) != 5], amax[np.arange(64) != 5] / 127, rtol=1e-7)


@needs_e2e
def test_reference_runs_written_model_deterministically(tmp_path):
    """The reference's loader accepts the writer's file, and its greedy run
    does not depend on the thread count (the GPU comparison below runs both
    builds with the same count, but must not hinge on it).  The prefill chunk
    size does change the reference's fp32 attention order, and so its
    logits, so both runs use the same chunk."""
    path = model_bin.write_bin(str(tmp_path / "tiny.bin"), "gemma-3-270m", seed=5,
                               nvocab=2048, layers=3)
    a = run_e2e(E2E_CPU, path, 9, 6, threads=2, chunk=4)
    b = run_e2e(E2E_CPU, path, 9, 6, threads=5, chunk=4)
    assert a["tokens"] == b["tokens"] and a["logits_fnv"] == b["logits_fnv"]
    assert len(a["tokens"]) == 7 and all(0 <= t < 2048 for t in a["tokens"])


@needs_e2e
def test_reference_runs_written_fp32_model(tmp_path):
    """An unquantized ('U') file from the writer: the reference's loader
    accepts it (check_head, gemma.c:1915-1939), runs its fp32 path, and its
    greedy tokens do not depend on the thread count."""
    path = model_bin.write_bin(str(tmp_path / "u.bin"), "gemma-3-270m", seed=5,
                               nvocab=2048, layers=3, quant=False)
    with open(path, "rb") as f:
        assert f.read(8) == b"GEMAf32U"
    a = run_e2e(E2E_CPU, path, 9, 6, threads=2, chunk=4)
    b = run_e2e(E2E_CPU, path, 9, 6, threads=5, chunk=4)
    assert a["tokens"] == b["tokens"]
    assert "gemv_fpx" in a["ops"]["decode"] and "gemm_fpx" in a["ops"]["prefill"]
    assert "gemv_int8" not in a["ops"]["decode"]


# ------------------------------------------------------------------ GPU
@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    return str(tmp_path_factory.mktemp("models"))


@pytest.mark.gpu
@needs_e2e
@pytest.mark.timeout(600)
@pytest.mark.parametrize("name,prompt_len,steps,chunk", [
    ("gemma-3-270m", 32, 64, None),   # config 1
    ("gemma-3-270m", 40, 8, 16),      # chunked prefill: M = 16, 16, 8
    ("gemma-3-1b", 512, 256, None),   # config 3: prefill M = 512, 256 decode steps
])
def test_e2e_hip_build_matches_reference(model_dir, name, prompt_len, steps, chunk):
    path = model_bin.ensure_bin(model_dir, name)
    ref = run_e2e(E2E_CPU, path, prompt_len, steps, chunk=chunk)
    hip = run_e2e(E2E_HIP, path, prompt_len, steps, chunk=chunk)
    assert hip["prompt"] == ref["prompt"]
    assert hip["tokens"] == ref["tokens"], "greedy token streams differ"
    assert hip["logits_fnv"] == ref["logits_fnv"], "logits differ in some bit"
    # the library really ran: every int8 op of the HIP build went through it
    assert hip["weight_bytes"] > 0
    assert "gemm_int8" in hip["ops"]["prefill"] and "gemv_int8" in hip["ops"]["decode"]
    # the library's own GPU timing counts the same calls under the same names
    for phase in ("prefill", "decode"):
        for op, (sec, calls) in hip["device_ops"][phase].items():
            assert op in hip["ops"][phase], (phase, op)
            assert calls == hip["ops"][phase][op][1], (phase, op)
            assert 0 < sec <= hip["ops"][phase][op][0] * 1.01 + 1e-3, (phase, op)


# The fp32 ('U') path: the reference's gemv_fpx / gemv_fpx_multi / gemm_fpx call
# sites (gemma.c:4766-5432) on the library.  There is no bit target (the
# reference's fp32 sums are in its compiler's order), and no int8 requantization
# amplifies rounding differences, so the HIP build's logits must stay within
# FP32_E2E_TOL of the reference's (relative to the step's largest logit) at
# every step both runs have reached with the same tokens; greedy streams may
# part where two logits are closer than that, and the agreement is reported.
FP32_E2E_TOL = 1e-4


@pytest.mark.gpu
@needs_e2e
@pytest.mark.timeout(600)
def test_e2e_hip_build_follows_reference_fp32(tmp_path):
    """Config 1's shape (gemma-3-270m: 18 layers, vocab 262144) as an fp32
    file: 32 prompt ids, 64 greedy steps."""
    path = model_bin.write_bin(str(tmp_path / "u270m.bin"), "gemma-3-270m", seed=1234,
                               quant=False)
    nv = model_bin.read_bin(path)["config"]["nvocab"]
    ref = run_e2e(E2E_CPU, path, 32, 64, logits=tmp_path / "ref.f32")
    hip = run_e2e(E2E_HIP, path, 32, 64, logits=tmp_path / "hip.f32")
    assert hip["prompt"] == ref["prompt"]
    a = np.fromfile(tmp_path / "ref.f32", np.float32).reshape(-1, nv)
    b = np.fromfile(tmp_path / "hip.f32", np.float32).reshape(-1, nv)
    assert a.shape == b.shape == (65, nv)
    same = 0  # steps whose input token both runs share
    while same < 64 and hip["tokens"][same] == ref["tokens"][same]:
        same += 1
    worst = 0.0
    for i in range(same + 1):  # logits row i comes from the token of step i - 1
        rel = float(np.abs(a[i] - b[i]).max() / np.abs(a[i]).max())
        worst = max(worst, rel)
        assert rel <= FP32_E2E_TOL, f"step {i}: {rel:.3g}"
    print(f"fp32 e2e: tokens agree for {same} of 65, worst |d|/max|logit| {worst:.3g}",
          flush=True)
    assert same >= 16
    assert "gemv_fpx" in hip["device_ops"]["decode"]
    assert "gemm_fpx" in hip["device_ops"]["prefill"]
    assert hip["weight_bytes"] > 0


# ------------------------------------------- decode glue vs the reference program
# The device-resident decoder runs the fp32 glue in fp64 and rounds once, the
# reference in fp32 in its compiler's order.  Until an activation lands on the
# other side of an int8 rounding boundary the two agree to ~1e-7; after such
# a flip this random model's logits differ by 1-3% relative to the largest
# logit.  Which applies to a row is decided before the comparison from the
# decode oracle's requantization margins up to that row (tests/flips.py):
# rows the criterion clears are held to REL_PRE_FLIP, the rest to REL_MAX,
# and the argmax must agree on every row whose reference lead is clear of
# the row's bar.
REL_PRE_FLIP = 1e-5
REL_MAX = 5e-2


def run_reference_decode_only(model_path, prompt_len, steps, tmp_path):
    import numpy as np

    dump = str(tmp_path / "ref_logits.bin")
    env = dict(os.environ, GEMMA_E2E_DECODE_ONLY="1", GEMMA_E2E_LOGITS=dump)
    cmd = [E2E_CPU, model_path, str(prompt_len), str(steps), "1234", str(THREADS)]
    out = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])
    seq = [res["bos"]] + res["prompt"] + res["tokens"][:-1]
    nvocab = model_bin.read_bin(model_path)["config"]["nvocab"]
    logits = np.fromfile(dump, np.float32).reshape(-1, nvocab)
    assert logits.shape[0] == len(seq)
    return seq, logits


def tracked_rows(oracle, calls):
    """Each zero-argument call produces one row of the oracle's logits; the
    rows, and per row whether no quantization up to it came within the
    margin bound of a rounding boundary."""
    import numpy as np

    oracle.track_margins()
    rows, free = [], []
    try:
        for call in calls:
            rows.append(call())
            free.append(oracle.min_margin() > flips.MARGIN_BOUND)
    finally:
        oracle.margins = None
    return rows, np.array(free)


def assert_close_to_reference(got_rows, ref_rows, free, what):
    """Row i within REL_PRE_FLIP (free[i]) or REL_MAX of the reference's
    largest logit, and the same argmax wherever the reference's lead over its
    runner-up is clear of that bar."""
    import numpy as np

    rel = np.array([float(np.abs(g - r).max() / np.abs(r).max())
                    for g, r in zip(got_rows, ref_rows)])
    bars = np.where(free, REL_PRE_FLIP, REL_MAX)
    bad = np.nonzero(rel > bars)[0]
    assert not len(bad), f"{what}: row {bad[0]} differs by {rel[bad[0]]:.3g} (bar {bars[bad[0]]:g})"
    checked = 0
    for i, (g, r) in enumerate(zip(got_rows, ref_rows)):
        if flips.clear_argmax(r, bars[i]):
            assert int(np.argmax(g)) == int(np.argmax(r)), f"{what}: argmax differs at row {i}"
            checked += 1
    first = int(np.argmax(rel > REL_PRE_FLIP)) if (rel > REL_PRE_FLIP).any() else len(rel)
    print(f"{what}: {int(free.sum())} of {len(rel)} rows flip-free by the margin criterion, "
          f"first row above {REL_PRE_FLIP:g}: {first}, max {rel.max():.3g}, median "
          f"{float(np.median(rel)):.3g}, argmax checked on {checked} rows", flush=True)


@needs_e2e
@pytest.mark.parametrize("name,layers,seed", [("gemma-3-270m", 6, 21), ("test-hd128", 1, 34)])
def test_decode_oracle_follows_reference_program(tmp_path, oracle, name, layers, seed):
    """The decode oracle (the decoder's checker) against the reference's own
    forward_gemma_decode, teacher-forced on the reference's tokens: sliding
    window (8), a global layer (5), random norm weights.  The one-layer
    narrow model's leading rows clear the margin criterion, so there the
    oracle's glue is held to the reference's to fp32 rounding."""
    from oracle import decode_oracle as dorc

    path = model_bin.write_bin(str(tmp_path / "m.bin"), name, seed=seed, nvocab=2048,
                               layers=layers, slide=8, norm_std=0.1)
    seq, ref = run_reference_decode_only(path, 12, 12, tmp_path)
    model = model_bin.read_bin(path)
    dec = dorc.DecodeOracle(model, oracle, len(seq) + 1)
    got, free = tracked_rows(oracle, [lambda t=tok, p=pos: dec.step(t, p)
                                      for pos, tok in enumerate(seq)])
    if layers == 1:
        assert free.sum() >= 1, "the narrow model's leading rows clear the criterion"
    assert_close_to_reference(got, ref, free, f"decode oracle vs reference ({name})")


@needs_e2e
def test_reference_comparison_catches_a_planted_mistake(tmp_path, oracle, monkeypatch):
    """The comparison above is sharp: the oracle with the global RoPE base
    used on sliding layers (a one-word mistake) fails it at once."""
    from oracle import decode_oracle as dorc

    path = model_bin.write_bin(str(tmp_path / "m.bin"), "gemma-3-270m", seed=21, nvocab=2048,
                               layers=6, slide=8, norm_std=0.1)
    seq, ref = run_reference_decode_only(path, 4, 2, tmp_path)
    model = model_bin.read_bin(path)
    model["config"] = dict(model["config"], theta_l=model["config"]["theta_g"])
    dec = dorc.DecodeOracle(model, oracle, len(seq) + 1)
    got = [dec.step(tok, pos) for pos, tok in enumerate(seq)]
    rel = [float(np.abs(g - r).max() / np.abs(r).max()) for g, r in zip(got, ref)]
    assert rel[0] <= REL_PRE_FLIP  # position 0: RoPE is the identity for every base
    assert max(rel[1:]) > 100 * REL_PRE_FLIP


@pytest.mark.gpu
@needs_e2e
@pytest.mark.timeout(600)
def test_device_decoder_follows_reference_program(gh, oracle, tmp_path):
    """BASELINE.json config 1 (gemma-3-270m, 32 prompt ids, 64 greedy steps)
    on the device-resident decoder, teacher-forced on the reference
    program's tokens, logits against the reference's at every position."""
    import numpy as np

    from oracle import decode_oracle as dorc

    path = model_bin.write_bin(str(tmp_path / "m270.bin"), "gemma-3-270m", seed=1234)
    seq, ref = run_reference_decode_only(path, 32, 64, tmp_path)
    model = model_bin.read_bin(path)
    orc = dorc.DecodeOracle(model, oracle, len(seq) + 1)
    _, free = tracked_rows(oracle, [lambda t=tok, p=pos: orc.step(t, p)
                                    for pos, tok in enumerate(seq)])
    dec = gh.decoder(model, len(seq) + 1)
    try:
        got = []
        lg = np.empty(model["config"]["nvocab"], np.float32)
        for pos, tok in enumerate(seq):
            dec.step(tok, pos, lg)
            got.append(lg.copy())
    finally:
        dec.close()
    # the decoder equals the oracle bit for bit (tests/test_decoder.py)
    assert_close_to_reference(got, ref, free, "device decoder vs reference (270m)")


def run_reference_prefill(model_path, prompt_len, steps, tmp_path):
    """The reference program's own path: <bos> and the prompt through
    forward_gemma_prefill (GEMMs, blockwise causal attention in fp32), then
    `steps` greedy decode steps; logits after the prompt and after each step."""
    import numpy as np

    dump = str(tmp_path / "ref_prefill_logits.bin")
    env = dict(os.environ, GEMMA_E2E_LOGITS=dump)
    env.pop("GEMMA_E2E_DECODE_ONLY", None)
    cmd = [E2E_CPU, model_path, str(prompt_len), str(steps), "1234", str(THREADS)]
    out = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])
    nvocab = model_bin.read_bin(model_path)["config"]["nvocab"]
    logits = np.fromfile(dump, np.float32).reshape(-1, nvocab)
    assert logits.shape[0] == 1 + steps
    return res, logits


@pytest.mark.gpu
@needs_e2e
@pytest.mark.timeout(600)
@pytest.mark.parametrize("mode", ["f32", "f64"])
def test_device_prefill_follows_reference_program(gh, oracle, tmp_path, mode):
    """BASELINE.json config 1 (gemma-3-270m, 32 prompt ids): the device's
    batched prefill (gemma_hip_decoder_prefill) against the reference's own
    chunked prefill, then 16 decode steps teacher-forced on the reference's
    tokens.  The reference evaluates the prefill attention in fp32 in its own
    blockwise order; the device in fp32 in another order (the default) or in
    fp64 (the decode oracle's arithmetic), so the flip-level bounds of the
    decoder comparison apply to both."""
    import numpy as np

    from gemma_hip import ATTN_F32, ATTN_F64

    from oracle import decode_oracle as dorc

    path = model_bin.write_bin(str(tmp_path / "m270.bin"), "gemma-3-270m", seed=1234)
    res, ref = run_reference_prefill(path, 32, 16, tmp_path)
    model = model_bin.read_bin(path)
    prompt, toks = res["prompt"], res["tokens"]
    orc = dorc.DecodeOracle(model, oracle, len(prompt) + len(toks) + 2)

    def oracle_prompt():
        orc.prefill([res["bos"]], 0)
        return orc.prefill(np.array(prompt, np.int32), 1)

    _, free = tracked_rows(oracle, [oracle_prompt] + [
        lambda i=i: orc.step(toks[i], 1 + len(prompt) + i) for i in range(16)])
    dec = gh.decoder(model, len(prompt) + len(toks) + 2,
                     attention=ATTN_F32 if mode == "f32" else ATTN_F64)
    try:
        lg = np.empty(model["config"]["nvocab"], np.float32)
        dec.prefill(np.array([res["bos"]], np.int32), 0)
        dec.prefill(np.array(prompt, np.int32), 1, lg)
        got = [lg.copy()]
        for i in range(16):
            dec.step(toks[i], 1 + len(prompt) + i, lg)
            got.append(lg.copy())
    finally:
        dec.close()
    assert len(got) == 17
    assert_close_to_reference(got, ref, free, f"device prefill ({mode}) vs reference prefill (270m)")
