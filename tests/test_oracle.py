"""Pins the CPU oracle (oracle/gemma_oracle.c) before it is trusted as the
checker of the HIP kernels.

Three independent pins:
 * the golden fixtures written by the reference's OWN functions compiled from
   /root/reference/gemma.c (tests/golden/make_golden.py) -- bit-exact;
 * exact integer arithmetic (int32 sums against an int64 brute force) and
   closed-form properties of the quantizer that any correct restatement has;
 * a live comparison against the compiled reference when oracle/_ref is
   built (skipped elsewhere).
The fixtures are chosen so that plausible mistakes fail: the test
``test_fixtures_reject_wrong_formulas`` plants two (the other compiler's
association of the scale reciprocal and of the rescale) in the oracle and
checks that the fixtures catch both.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as om


def split_cases(g, key_q, key_s):
    bounds = np.concatenate([[0], np.cumsum(g["lens"])])
    for i in range(len(g["lens"])):
        sl = slice(bounds[i], bounds[i + 1])
        yield i, g["vec"][sl], g[key_q][sl], g[key_s][i]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.int32)


@pytest.mark.parametrize("flavor,suffix", [(om.GCC, "gcc"), (om.CLANG, "clang")])
def test_quantize_act_matches_reference(oracle, golden, flavor, suffix):
    g = golden("quantize_act")
    for i, vec, q_ref, s_ref in split_cases(g, "q_" + suffix, "scale_" + suffix):
        q, s = oracle.quantize_act(vec, flavor)
        assert np.array_equal(q, q_ref), f"case {i}: {(q != q_ref).sum()} q mismatches"
        assert bits(s) == bits(s_ref), f"case {i}: scale {s} != {s_ref}"


def test_quantize_acts_strided_matches_reference(oracle, golden):
    g = golden("quantize_acts")
    q, s = oracle.quantize_acts(g["src"], n=int(g["n"]))
    assert np.array_equal(q, g["q"])
    assert np.array_equal(bits(s), bits(g["scale"]))


def test_gemv_int8_matches_reference(oracle, golden):
    g = golden("gemv_int8")
    xq, xs = oracle.quantize_act(g["x"])
    assert np.array_equal(xq, g["xq"]) and bits(xs) == bits(g["xs"])
    y, acc = oracle.gemv_int8(g["mat"], g["matsc"], g["xq"], g["xs"], om.GCC)
    assert np.array_equal(bits(y), bits(g["y_gcc"]))
    y_c, _ = oracle.gemv_int8(g["mat"], g["matsc"], g["xq"], g["xs"], om.CLANG)
    assert np.array_equal(bits(y_c), bits(g["y_clang"]))
    # the int32 group accumulator: exact integer arithmetic
    brute = g["mat"].astype(np.int64) @ g["xq"].astype(np.int64)
    assert np.array_equal(acc.astype(np.int64), brute)


def test_gemv_int8_multi_matches_reference(oracle, golden):
    g = golden("gemv_int8_multi")
    ys = [oracle.gemv_int8(g[f"w{j}"], g[f"s{j}"], g["xq"], g["xs"])[0] for j in range(3)]
    assert np.array_equal(bits(np.concatenate(ys)), bits(g["y"]))


@pytest.mark.parametrize("tag", ["tails", "strided", "m1", "blocks"])
def test_gemm_int8_matches_reference(oracle, golden, tag):
    g = golden("gemm_int8")
    m, n, k, ds, ms, ss = (int(v) for v in g[tag + "_shape"])
    dst = np.full((m, ds), -7.0, np.float32)
    dst, acc = oracle.gemm_int8(g[tag + "_b"], g[tag + "_bs"], g[tag + "_a"],
                                g[tag + "_as"], k=k, dst=dst)
    assert np.array_equal(bits(dst), bits(g[tag + "_dst"]))
    brute = g[tag + "_a"][:, :k].astype(np.int64) @ g[tag + "_b"][:, :k].astype(np.int64).T
    assert np.array_equal(acc.astype(np.int64), brute)


@pytest.mark.parametrize("tag", ["tails", "blocks", "m1"])
def test_gemm_int8_full_matches_reference(oracle, golden, tag):
    """The large-shape path of the GPU tests (exact sums by a float64 product,
    then the file's own rescale of every cell) against the reference's
    fixtures and the scalar restatement, with FTZ-range scales added."""
    g = golden("gemm_int8")
    m, n, k, ds, ms, ss = (int(v) for v in g[tag + "_shape"])
    a, b = g[tag + "_a"][:, :k], g[tag + "_b"][:, :k]
    full = oracle.gemm_int8_full(b, g[tag + "_bs"], a, g[tag + "_as"])
    assert np.array_equal(bits(full), bits(g[tag + "_dst"][:, :n]))
    rng = np.random.default_rng(3)
    asc = g[tag + "_as"].copy()
    bsc = g[tag + "_bs"].copy()
    asc[::3] = 1e-20  # products of 1e-20 and 1e-3..1e-2 scales fall below FLT_MIN
    bsc[1::4] = rng.uniform(1e-39, 1e-38, bsc[1::4].shape).astype(np.float32)  # subnormal: DAZ
    slow, _ = oracle.gemm_int8(b, bsc, a, asc)
    assert np.array_equal(bits(oracle.gemm_int8_full(b, bsc, a, asc)), bits(slow))


def test_int_sums_exact_at_full_length(oracle):
    """int_sums against an int64 brute force at the longest K of the path
    (gemma-3-4b down, K = 10240) with all-extreme operands, where every
    partial sum is largest."""
    rng = np.random.default_rng(5)
    k = 10240
    a = rng.choice(np.array([-127, 127], np.int8), (3, k))
    b = rng.choice(np.array([-127, 127], np.int8), (4, k))
    b[0] = a[0]  # a sum of exactly 127*127*k
    got = oracle.int_sums(b, a)
    assert got[0, 0] == 127 * 127 * k
    assert np.array_equal(got.astype(np.int64), a.astype(np.int64) @ b.astype(np.int64).T)


def test_requantization_margins(oracle):
    """The margin record (tests/flips.py) in closed form: an element whose
    scaled magnitude sits exactly on a boundary has margin 0; one at an
    integer has 1/2; perturbing a vector by less than its margin keeps every
    int8 value, and by more than the margin changes one."""
    amax = np.float32(127.0)  # t = |v|
    oracle.track_margins()
    oracle.quantize_act(np.array([amax, 3.5, -2.0], np.float32))
    assert oracle.min_margin() == 0.0
    oracle.track_margins()
    oracle.quantize_acts(np.array([[amax, 3.0, -2.0], [0, 0, 0]], np.float32))
    assert oracle.min_margin() == 0.5
    oracle.margins = None
    rng = np.random.default_rng(1)
    v = rng.standard_normal(512).astype(np.float32)
    m = oracle.row_margins(v)
    q, _ = oracle.quantize_act(v)
    amx = float(np.abs(v).max())
    safe = v + np.float32(0.4 * m * amx / 127.0) * np.sign(rng.standard_normal(512)).astype(np.float32)
    safe[np.argmax(np.abs(v))] = v[np.argmax(np.abs(v))]  # keep amax
    assert np.array_equal(oracle.quantize_act(safe)[0], q)
    i = int(np.argmin(np.abs(np.abs(v) * 127.0 / amx - np.floor(np.abs(v) * 127.0 / amx) - 0.5)))
    t = abs(float(v[i])) * 127.0 / amx
    push = v.copy()
    push[i] = np.float32(np.sign(v[i]) * (np.floor(t) + 0.5 + (0.01 if t < np.floor(t) + 0.5 else -0.01)) * amx / 127.0)
    assert not np.array_equal(oracle.quantize_act(push)[0], q)


def test_fpx_reference_within_tolerance_of_exact(oracle, golden):
    """The fp32 fallback has no bit-exact target; the reference's own fp32
    results lie within 1e-5 * sum|a*b| of the exact product, which is the
    tolerance the GPU's fp32 path is held to."""
    g = golden("fpx")
    exact, mag = oracle.gemm_f64(g["gemv_w"], g["gemv_x"][None, :])
    err = np.abs(g["gemv_y"].astype(np.float64) - exact[0])
    assert np.all(err <= 1e-5 * mag[0])
    exact, mag = oracle.gemm_f64(g["gemm_b"], g["gemm_a"])
    err = np.abs(g["gemm_dst"].astype(np.float64) - exact)
    assert np.all(err <= 1e-5 * mag)
    # a dropped term is far outside that tolerance
    bad, _ = oracle.gemm_f64(g["gemm_b"][:, :-1], g["gemm_a"][:, :-1])
    assert np.any(np.abs(g["gemm_dst"].astype(np.float64) - bad) > 1e-5 * mag)


def test_fixtures_reject_wrong_formulas(oracle, golden):
    """Plant the two likeliest restatement mistakes in the oracle (the clang
    association: inv = 1/scale and (acc*xs)*ws) and check that the gcc
    fixtures catch each of them."""
    g = golden("quantize_act")
    caught = 0
    for i, vec, q_ref, _ in split_cases(g, "q_gcc", "scale_gcc"):
        q, _ = oracle.quantize_act(vec, om.CLANG)
        caught += int(not np.array_equal(q, q_ref))
    assert caught > 0, "the quantize fixtures do not pin inv = 127/amax"
    g = golden("gemv_int8")
    y, _ = oracle.gemv_int8(g["mat"], g["matsc"], g["xq"], g["xs"], om.CLANG)
    assert not np.array_equal(bits(y), bits(g["y_gcc"])), "fixtures do not pin the rescale order"


def test_quantize_closed_form_properties(oracle):
    """Properties any correct quantizer has, independent of the fixtures."""
    rng = np.random.default_rng(7)
    for k in (1, 7, 640, 6912):
        v = (rng.standard_normal(k) * rng.uniform(0.01, 100)).astype(np.float32)
        q, s = oracle.quantize_act(v)
        amax = np.float32(np.max(np.abs(v)))
        assert bits(s) == bits(amax * np.float32(1.0 / 127.0))
        assert np.all(np.abs(q.astype(np.int32)) <= 127)
        # the element of largest magnitude maps to +-127
        assert abs(int(q[np.argmax(np.abs(v))])) == 127
        # round half away from zero of v*(127/amax), away from exact ties
        x = v.astype(np.float64) * (127.0 / np.float64(amax))
        frac = np.abs(x - np.trunc(x))
        clear = np.abs(frac - 0.5) > 1e-4
        want = np.trunc(x + np.copysign(0.5, x)).astype(np.int32)
        assert np.array_equal(q.astype(np.int32)[clear], want[clear])
        # sign symmetry
        qn, sn = oracle.quantize_act(-v)
        assert np.array_equal(qn, -q) and bits(sn) == bits(s)


def test_quantize_zero_and_subnormal_rows(oracle):
    q, s = oracle.quantize_act(np.zeros(16, np.float32))
    assert s == 1.0 and not q.any()
    v = np.zeros(16, np.float32)
    v[3] = 1e-40  # subnormal: read as zero under DAZ
    q, s = oracle.quantize_act(v)
    assert s == 1.0 and not q.any()


def test_rescale_ftz(oracle):
    lib = oracle.lib
    # a product below FLT_MIN flushes to zero, with its sign
    assert lib.oracle_rescale(1, 1e-20, 1e-20, om.GCC) == 0.0
    assert np.signbit(np.float32(lib.oracle_rescale(-1, 1e-20, 1e-20, om.GCC)))
    # an ordinary product is the IEEE result of the two multiplies
    acc, xs, ws = 123457, np.float32(0.0173), np.float32(0.00731)
    assert np.float32(lib.oracle_rescale(acc, xs, ws, om.GCC)) == np.float32(acc) * (xs * ws)


@pytest.mark.skipif(not om.RefHarness.available("gcc"), reason="oracle/_ref not built")
def test_live_against_reference_build(oracle):
    """Random shapes straight through the compiled reference."""
    ref = om.RefHarness("gcc")
    rng = np.random.default_rng(11)
    for m, n, k in ((3, 17, 48), (9, 8, 96), (16, 33, 1152)):
        A = rng.standard_normal((m, k)).astype(np.float32)
        qa, sa = oracle.quantize_acts(A)
        qr, sr = ref.quantize_acts(A)
        assert np.array_equal(qa, qr) and np.array_equal(bits(sa), bits(sr))
        B = rng.integers(-127, 128, (n, k), dtype=np.int8)
        bs = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        d, _ = oracle.gemm_int8(B, bs, qa, sa)
        dr, st = ref.gemm_int8(B, bs, qa, sa, k, np.zeros((m, n), np.float32))
        assert st == 0 and np.array_equal(bits(d), bits(dr))


def test_patch_embed_one_hot_closed_form(oracle):
    """gemma.c:4411-4448 indexing: a weight that selects one (c, py, px) per
    output channel makes the output that image pixel plus the bias, so a
    transposed channel, row or column index fails."""
    rng = np.random.default_rng(4)
    img_px, psize, dim = 28, 7, 5
    img = rng.standard_normal((img_px, img_px, 3)).astype(np.float32)
    pe = np.zeros((dim, 3, psize, psize), np.float32)
    picks = [(0, 0, 0), (2, 6, 1), (1, 3, 5), (0, 6, 6), (2, 0, 4)]
    for oc, (c, py, px) in enumerate(picks):
        pe[oc, c, py, px] = 1.0
    bias = rng.standard_normal(dim).astype(np.float32)
    out, _ = oracle.patch_embed_f64(img, pe, bias, psize)
    ppi = img_px // psize
    for pi in range(ppi * ppi):
        oy, ox = divmod(pi, ppi)
        for oc, (c, py, px) in enumerate(picks):
            want = np.float64(img[oy * psize + py, ox * psize + px, c]) + np.float64(bias[oc])
            assert out[pi, oc] == want


def test_patch_embed_linearity(oracle):
    """Linear in the image: f(a*x + y) - b = a*(f(x) - b) + (f(y) - b)."""
    rng = np.random.default_rng(5)
    img_px, psize, dim = 14, 7, 3
    # integer-valued images so that 2*x + y is exact in float32
    x = rng.integers(-8, 9, (img_px, img_px, 3)).astype(np.float32)
    y = rng.integers(-8, 9, (img_px, img_px, 3)).astype(np.float32)
    pe = rng.standard_normal((dim, 3, psize, psize)).astype(np.float32)
    b = rng.standard_normal(dim).astype(np.float32)
    fx, _ = oracle.patch_embed_f64(x, pe, b, psize)
    fy, _ = oracle.patch_embed_f64(y, pe, b, psize)
    fz, _ = oracle.patch_embed_f64((2 * x + y).astype(np.float32), pe, b, psize)
    assert np.allclose(fz - b, 2 * (fx - b) + (fy - b), rtol=1e-12, atol=1e-9)
