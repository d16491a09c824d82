"""Writes the golden fixtures of tests/golden/*.npz from the REFERENCE's own
functions, compiled from /root/reference/gemma.c by oracle/Makefile
(oracle/_ref/gemma_ref_gcc and gemma_ref_clang; the reference holds no golden
vectors of its own).  Run in the build container, where /root/reference
exists:

    make -C oracle ref && python tests/golden/make_golden.py

Each fixture stores inputs and the reference's outputs only.  Inputs are
chosen so that a plausible mistake in a restatement fails: values within a
few ulp of the rounding boundaries (k + 0.5) * amax / 127, the FTZ/DAZ edges
of the scale, M/N tails that are not multiples of the reference's 8x8
micro-tiles (gemma.c:3967-3968), padded strides, and rescale products whose
two association orders differ.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.oracle import RefHarness  # noqa: E402


def outlier_acts(rng, shape):
    """N(0,1) activations with 1% of channels scaled by 20."""
    x = rng.standard_normal(shape).astype(np.float32)
    cols = rng.random(shape[-1]) < 0.01
    x[..., cols] *= 20.0
    return x


def near_half(rng, n, amax):
    """Values within +-3 ulp of (k + 0.5) * amax / 127, plus amax itself."""
    k = rng.integers(-127, 127, n)
    base = ((k + 0.5) * np.float64(amax) / 127.0).astype(np.float32)
    v = (base.view(np.int32) + rng.integers(-3, 4, n).astype(np.int32)).view(np.float32)
    v[0] = np.float32(amax)
    return v


def quantize_cases(rng):
    cases = []
    for k in (640, 1152, 6912, 13):
        cases.append(outlier_acts(rng, (k,)))
    for amax in (1.0, 3.7, 20.0, 1e-30, 1e-37, 1.4e-36, 1.5e-36, 1.6e-36, 3e38):
        cases.append(near_half(rng, 2048, amax))
    cases.append(np.zeros(64, np.float32))
    sub = np.zeros(64, np.float32)
    sub[[3, 5, 9]] = [1e-40, -2e-41, -0.0]
    cases.append(sub)
    mixed = np.zeros(64, np.float32)
    mixed[[3, 5]] = [1e-40, 1e-30]
    cases.append(mixed)
    tiny_norm = np.zeros(64, np.float32)
    tiny_norm[[1, 2]] = [1.17549435e-38, -3e-38]
    cases.append(tiny_norm)
    return cases


def main() -> None:
    gcc, clang = RefHarness("gcc"), RefHarness("clang")
    rng = np.random.default_rng(20251201)
    out = {}

    # --- quantize_act (gemma.c:2590) -------------------------------------
    cases = quantize_cases(rng)
    lens = np.array([len(c) for c in cases], np.int64)
    flat = np.concatenate(cases)
    q_g, s_g, q_c, s_c = [], [], [], []
    for c in cases:
        q, s = gcc.quantize_act(c)
        q_g.append(q)
        s_g.append(s)
        q, s = clang.quantize_act(c)
        q_c.append(q)
        s_c.append(s)
    np.savez(os.path.join(HERE, "quantize_act.npz"), lens=lens, vec=flat,
             q_gcc=np.concatenate(q_g), scale_gcc=np.array(s_g, np.float32),
             q_clang=np.concatenate(q_c), scale_clang=np.array(s_c, np.float32))
    out["quantize_act"] = {"cases": len(cases), "values": int(flat.size)}

    # --- quantize_acts with a padded source stride (gemma.c:2656, 5302) --
    m, n, sstr = 7, 1152, 1160
    src = outlier_acts(rng, (m, sstr))
    src[2, :n] = near_half(rng, n, 5.0)
    q, s = gcc.quantize_acts(src, n=n, omp=True, threads=4)
    np.savez(os.path.join(HERE, "quantize_acts.npz"), src=src, n=np.int64(n), q=q, scale=s)
    out["quantize_acts"] = {"m": m, "n": n, "sstr": sstr}

    # --- gemv_int8 (gemma.c:2770) and gemv_int8_multi (gemma.c:2818) -----
    nout, kin = 96, 1152
    W = rng.integers(-127, 128, (nout, kin), dtype=np.int8)
    ws = rng.uniform(1e-3, 1e-2, nout).astype(np.float32)
    ws[:4] = [1e-20, 3e-19, 2.5e-21, 7e-3]  # products near the FTZ limit
    x = outlier_acts(rng, (kin,))
    xq, xs = gcc.quantize_act(x)
    y = gcc.gemv_int8(W, ws, xq, xs, omp=True, threads=4)
    y_clang = clang.gemv_int8(W, ws, xq, xs, omp=True, threads=4)
    np.savez(os.path.join(HERE, "gemv_int8.npz"), mat=W, matsc=ws, x=x, xq=xq,
             xs=np.float32(xs), y_gcc=y, y_clang=y_clang)
    out["gemv_int8"] = {"n": nout, "k": kin}

    kin = 640
    jobs = [(rng.integers(-127, 128, (rows, kin), dtype=np.int8),
             rng.uniform(1e-3, 1e-2, rows).astype(np.float32)) for rows in (64, 16, 16)]
    x = outlier_acts(rng, (kin,))
    xq, xs = gcc.quantize_act(x)
    y = gcc.gemv_int8_multi(jobs, xq, xs, threads=4)
    np.savez(os.path.join(HERE, "gemv_int8_multi.npz"),
             w0=jobs[0][0], s0=jobs[0][1], w1=jobs[1][0], s1=jobs[1][1],
             w2=jobs[2][0], s2=jobs[2][1], xq=xq, xs=np.float32(xs), y=y)
    out["gemv_int8_multi"] = {"rows": [64, 16, 16], "k": kin}

    # --- gemm_int8 (gemma.c:3943): tails, strides, M = 1 ------------------
    gemm = {}
    for tag, (m, n, k, dstr, mstr, sstr) in {
        "tails": (13, 40, 1152, 0, 0, 0),
        "strided": (20, 36, 256, 44, 272, 288),
        "m1": (1, 24, 640, 0, 0, 0),
        "blocks": (136, 264, 320, 0, 0, 0),
    }.items():
        ds, ms, ss = dstr or n, mstr or k, sstr or k
        A = outlier_acts(rng, (m, ss))
        Aq, As = gcc.quantize_acts(A, n=ss, omp=False)
        B = rng.integers(-127, 128, (n, ms), dtype=np.int8)
        bs = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        d0 = np.full((m, ds), -7.0, np.float32)  # stride gaps must survive
        d, status = gcc.gemm_int8(B, bs, Aq, As, k, d0, omp=True, threads=4)
        assert status == 0
        gemm.update({f"{tag}_a": Aq, f"{tag}_as": As, f"{tag}_b": B, f"{tag}_bs": bs,
                     f"{tag}_dst": d, f"{tag}_shape": np.array([m, n, k, ds, ms, ss])})
    np.savez(os.path.join(HERE, "gemm_int8.npz"), **gemm)
    out["gemm_int8"] = ["tails", "strided", "m1", "blocks"]

    # --- fp32 fallback (gemma.c:2734 gemv_fpx, 3308 gemm_fpx) ------------
    Wf = (rng.standard_normal((32, 1152)) * 0.02).astype(np.float32)
    xf = outlier_acts(rng, (1152,))
    yf = gcc.gemv_fpx(Wf, xf, omp=True, threads=4)
    Af = outlier_acts(rng, (21, 588))
    Bf = (rng.standard_normal((40, 588)) * 0.02).astype(np.float32)
    df, status = gcc.gemm_fpx(Bf, Af, 588, np.zeros((21, 40), np.float32), omp=True, threads=4)
    assert status == 0
    np.savez(os.path.join(HERE, "fpx.npz"), gemv_w=Wf, gemv_x=xf, gemv_y=yf,
             gemm_a=Af, gemm_b=Bf, gemm_dst=df)
    out["fpx"] = {"gemv": [32, 1152], "gemm": [21, 40, 588]}

    meta = {
        "generator": "tests/golden/make_golden.py",
        "reference": "/root/reference/gemma.c (compiled by oracle/Makefile)",
        "gcc": subprocess.run(["gcc", "--version"], capture_output=True,
                              text=True).stdout.splitlines()[0],
        "flags_gcc": "-std=c11 -O3 -ffast-math -fopenmp -march=x86-64-v2",
        "flags_clang": "-std=c11 -O3 -ffast-math -fopenmp -march=x86-64-v3",
        "fixtures": out,
    }
    with open(os.path.join(HERE, "golden_meta.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print(json.dumps(meta, indent=1))


if __name__ == "__main__":
    main()
