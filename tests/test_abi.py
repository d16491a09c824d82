"""CPU checks of the C-ABI library: it is built, loads, exports every symbol
the public header declares, and reports errors through the reference's
0/1 + message convention without a GPU.  No compute call is made here."""

from __future__ import annotations

import ctypes
import os
import subprocess

import pytest

import gemma_hip


def test_library_is_built_for_gfx950():
    assert os.path.exists(gemma_hip.LIB_PATH), "run __graft_entry__.build() first"
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list",
                          "--type=o", f"--input={gemma_hip.LIB_PATH}"],
                         capture_output=True, text=True)
    if out.returncode == 0 and out.stdout.strip():
        assert "gfx950" in out.stdout


def test_every_header_symbol_is_exported():
    lib = ctypes.CDLL(gemma_hip.LIB_PATH)
    declared = gemma_hip.header_symbols()
    assert len(declared) >= 20
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_the_header():
    assert sorted(gemma_hip._SIGS) == gemma_hip.header_symbols()


def test_library_does_not_depend_on_the_oracle():
    out = subprocess.run(["readelf", "-d", gemma_hip.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    assert "oracle" not in out and "gemma_ref" not in out


def test_calls_before_init_fail_with_message():
    lib = gemma_hip.load()
    lib.gemma_hip_shutdown()  # no-op when not initialised
    rc = lib.gemma_hip_quantize(None, None, None, 0, 1, 8, None)
    assert rc == 1
    assert b"not initialised" in lib.gemma_hip_last_error()
    rc = lib.gemma_hip_gemv_int8_host(None, None, None, None, 1.0, 4, 4)
    assert rc == 1
    assert lib.gemma_hip_device_ptr(None) is None


def test_init_without_gpu_reports_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = gemma_hip.load()
    assert lib.gemma_hip_init(0) == 1
    assert lib.gemma_hip_last_error().startswith(b"gemma_hip_init")
