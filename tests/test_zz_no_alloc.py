"""gemma_hip_matmul_noalloc (the allocation-free variant of gemma_hip_matmul)
against gemma_hip_matmul itself, through the C ABI.

Bar: bit-identical fp32 outputs (both entry points run the same kernels; the
variant only takes the split-K partial tiles and tile counters from the
library's static scratch).  Two calls in a row, the second on a smaller
input, each through the split-K path, so the second reuses the scratch the
first left behind; a shape without split-K; a shape whose plan needs more
scratch than there is (rejected with an error, nothing written); and the call
captured into a HIP graph, replayed with eager work between the replays.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def operands(m, n, k, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda", generator=g)
    b = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
    asc = torch.rand(m, device="cuda", generator=g) * 9e-3 + 1e-3
    bsc = torch.rand(n, device="cuda", generator=g) * 9e-3 + 1e-3
    return a, b, asc, bsc


def both(gh, m, n, k, seed):
    a, b, asc, bsc = operands(m, n, k, seed)
    s = torch.cuda.current_stream().cuda_stream
    want = torch.full((m, n), 7.0, device="cuda")
    got = torch.full((m, n), -7.0, device="cuda")
    gh.matmul(want, n, b, k, bsc, a, k, asc, m, n, k, s)
    gh.matmul_noalloc(got, n, b, k, bsc, a, k, asc, m, n, k, s)
    torch.cuda.synchronize()
    return got, want


def test_noalloc_equals_matmul_twice_then_smaller(gh):
    # 1b prefill down (144 tiles of 64x64, K = 6912: split 3 ways), then a
    # smaller shape that also splits (40 tiles of 64x64, K = 4096: 6 ways)
    for m, n, k, seed in [(512, 1152, 6912, 1), (200, 640, 4096, 2)]:
        note(f"noalloc m={m} n={n} k={k}")
        got, want = both(gh, m, n, k, seed)
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_noalloc_without_split(gh):
    note("noalloc m=160 n=384 k=640")
    got, want = both(gh, 160, 384, 640, 3)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_noalloc_rejects_plans_beyond_scratch(gh, monkeypatch):
    from gemma_hip import GemmaHipError

    # 320 tiles forced into 8 pieces need 160 MiB of partial tiles
    monkeypatch.setenv("GEMMA_HIP_GEMM_SPLIT", "8")
    m, n, k = 2048, 2560, 2048
    a, b, asc, bsc = operands(m, n, k, 4)
    out = torch.full((m, n), 7.0, device="cuda")
    with pytest.raises(GemmaHipError, match="needs .* bytes of scratch"):
        gh.matmul_noalloc(out, n, b, k, bsc, a, k, asc, m, n, k,
                          torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_noalloc_in_a_graph(gh):
    m, n, k = 512, 1152, 6912
    note(f"noalloc graph m={m} n={n} k={k}")
    a, b, asc, bsc = operands(m, n, k, 5)
    want = torch.empty((m, n), device="cuda")
    gh.matmul(want, n, b, k, bsc, a, k, asc, m, n, k, torch.cuda.current_stream().cuda_stream)
    out = torch.empty((m, n), device="cuda")
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=side):
        out.fill_(0.0)
        gh.matmul_noalloc(out, n, b, k, bsc, a, k, asc, m, n, k, side.cuda_stream)
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), f"replay {rep}"
        # eager work on the same scratch between replays
        got, ref = both(gh, 200, 640, 4096, 6 + rep)
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
