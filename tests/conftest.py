"""Shared fixtures.  Tests marked ``gpu`` need an MI355X (gfx950); all
others run on the CPU.  The oracle (oracle/) is test infrastructure: these
tests use it only as the checker of the HIP library's results."""

from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "gemma.c_amd")
GOLDEN = os.path.join(REPO, "tests", "golden")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as om

    if not os.path.exists(om.LIB_PATH):
        subprocess.run(["make", "-C", om.ORACLE_DIR, "oracle"], check=True,
                       capture_output=True)
    return om.Oracle()


@pytest.fixture(scope="session")
def golden():
    def load(name):
        with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
            return {k: z[k] for k in z.files}

    return load


@pytest.fixture(scope="session")
def gh():
    """The HIP library on cuda:0.  Fails (never skips) when it cannot load:
    a GPU test must run the native path or report why it could not."""
    import torch

    import gemma_hip

    if not torch.cuda.is_available():
        pytest.fail("gpu test needs a HIP device (run with -m 'not gpu' on a CPU host)")
    torch.cuda.init()
    lib = gemma_hip.GemmaHip(0)
    yield lib
    lib.close()
