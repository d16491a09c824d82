"""Python access to the CPU oracle.  TEST INFRASTRUCTURE, NOT PRODUCT.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module.  It wraps two things:

* ``Oracle``: the restatement in gemma_oracle.c (built into
  ``oracle/_build/libgemma_oracle.so``), loaded with ctypes.  Every function
  cites the reference line it restates in gemma_oracle.c.
* ``RefHarness``: the reference's own functions, compiled from
  /root/reference/gemma.c into ``oracle/_ref/gemma_ref_{gcc,clang}``
  executables (see oracle/Makefile); driven through files, one process per
  call, so the reference's FTZ/DAZ start-up state never leaks into the caller.
"""

from __future__ import annotations

import ctypes
import json
import os
import subprocess
import tempfile

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "_build", "libgemma_oracle.so")
REF_DIR = os.path.join(ORACLE_DIR, "_ref")

GCC, CLANG = 0, 1
FLAVORS = {"gcc": GCC, "clang": CLANG}

_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_int = ctypes.c_int


def _ptr(arr: np.ndarray | None, ctype):
    if arr is None:
        return ctypes.cast(None, ctype)
    assert arr.flags["C_CONTIGUOUS"]
    return arr.ctypes.data_as(ctype)


def build(quiet: bool = True) -> None:
    """Compile the restatement, and the reference harnesses when the
    reference source is present (this container only)."""
    targets = ["oracle"]
    if os.path.exists("/root/reference/gemma.c"):
        targets.append("ref")
    subprocess.run(["make", "-B", "-C", ORACLE_DIR] + targets, check=True,
                   capture_output=quiet)


class Oracle:
    """ctypes binding of gemma_oracle.c."""

    def __init__(self, path: str = LIB_PATH):
        self.margins = None  # requantization margins while tracking (track_margins)
        if not os.path.exists(path):
            raise FileNotFoundError(f"oracle library not built: {path}")
        lib = ctypes.CDLL(path)
        lib.oracle_quantize_act.restype = ctypes.c_float
        lib.oracle_quantize_act.argtypes = [_i8p, _f32p, _int, _int]
        lib.oracle_quantize_acts.restype = None
        lib.oracle_quantize_acts.argtypes = [_i8p, _f32p, _f32p, _int, _int, _int, _int]
        lib.oracle_dot_i8.restype = ctypes.c_int32
        lib.oracle_dot_i8.argtypes = [_i8p, _i8p, _int]
        lib.oracle_rescale.restype = ctypes.c_float
        lib.oracle_rescale.argtypes = [ctypes.c_int32, ctypes.c_float, ctypes.c_float, _int]
        lib.oracle_gemv_int8.restype = None
        lib.oracle_gemv_int8.argtypes = [_f32p, _i32p, _i8p, _f32p, _i8p, ctypes.c_float,
                                         _int, _int, _int]
        lib.oracle_gemm_int8.restype = None
        lib.oracle_gemm_int8.argtypes = [_f32p, _int, _i32p, _i8p, _int, _f32p, _i8p, _int,
                                         _f32p, _int, _int, _int, _int]
        lib.oracle_rescale_matrix.restype = None
        lib.oracle_rescale_matrix.argtypes = [_f32p, _i32p, _f32p, _f32p, _int, _int, _int]
        lib.oracle_gemm_f64.restype = None
        lib.oracle_gemm_f64.argtypes = [_f64p, _f64p, _f32p, _int, _f32p, _int, _int, _int, _int]
        lib.oracle_patch_embed_f64.restype = None
        lib.oracle_patch_embed_f64.argtypes = [_f64p, _f64p, _f32p, _f32p, _f32p, _int, _int, _int]
        self.lib = lib

    # -- requantization margins -------------------------------------------
    # While tracking, every quantize_act(s) call records the smallest distance,
    # over its rows' elements, of t = |v| * 127 / amax (the quantizer's
    # argument before rounding, gemma.c:2621-2646, in exact arithmetic) from a
    # rounding boundary k + 1/2.  An input that differs from the oracle's by
    # at most eps * amax moves every t by at most 254 eps (plus the fp32
    # rounding of v * inv on both sides), so a pass whose smallest margin
    # exceeds that bound quantizes every element to the oracle's int8 value.
    def track_margins(self) -> None:
        self.margins = []

    def min_margin(self) -> float:
        """Smallest margin since track_margins (inf when nothing was quantized)."""
        return min(self.margins) if self.margins else float("inf")

    @staticmethod
    def row_margins(rows: np.ndarray) -> float:
        rows = np.atleast_2d(np.asarray(rows, np.float64))
        amax = np.abs(rows).max(axis=1, keepdims=True)
        live = amax[:, 0] > 0
        if not live.any():
            return float("inf")
        t = np.abs(rows[live]) * (127.0 / amax[live])
        return float(np.abs(t - np.floor(t) - 0.5).min())

    def _record(self, rows) -> None:
        if getattr(self, "margins", None) is not None:
            self.margins.append(self.row_margins(rows))

    def quantize_act(self, vec: np.ndarray, flavor: int = GCC):
        vec = np.ascontiguousarray(vec, dtype=np.float32)
        q = np.empty(vec.shape[0], np.int8)
        s = self.lib.oracle_quantize_act(_ptr(q, _i8p), _ptr(vec, _f32p), vec.shape[0], flavor)
        self._record(vec)
        return q, np.float32(s)

    def quantize_acts(self, src: np.ndarray, n: int | None = None, flavor: int = GCC):
        """src is [m][sstr]; the first n columns of each row are quantized."""
        src = np.ascontiguousarray(src, dtype=np.float32)
        m, sstr = src.shape
        n = sstr if n is None else n
        q = np.empty((m, n), np.int8)
        s = np.empty(m, np.float32)
        self.lib.oracle_quantize_acts(_ptr(q, _i8p), _ptr(s, _f32p), _ptr(src, _f32p), sstr, m,
                                      n, flavor)
        self._record(src[:, :n])
        return q, s

    def gemv_int8(self, mat, matsc, vec, vsc, flavor: int = GCC):
        mat = np.ascontiguousarray(mat, dtype=np.int8)
        matsc = np.ascontiguousarray(matsc, dtype=np.float32)
        vec = np.ascontiguousarray(vec, dtype=np.int8)
        m, n = mat.shape
        dst = np.empty(m, np.float32)
        acc = np.empty(m, np.int32)
        self.lib.oracle_gemv_int8(_ptr(dst, _f32p), _ptr(acc, _i32p), _ptr(mat, _i8p),
                                  _ptr(matsc, _f32p), _ptr(vec, _i8p), float(vsc), m, n, flavor)
        return dst, acc

    def gemm_int8(self, mat, matsc, src, ssc, k: int | None = None, dst=None,
                  flavor: int = GCC):
        """mat [n][mstr], src [m][sstr] (the first k columns are used);
        dst [m][dstr] is updated in place when given."""
        mat = np.ascontiguousarray(mat, dtype=np.int8)
        src = np.ascontiguousarray(src, dtype=np.int8)
        matsc = np.ascontiguousarray(matsc, dtype=np.float32)
        ssc = np.ascontiguousarray(ssc, dtype=np.float32)
        n, mstr = mat.shape
        m, sstr = src.shape
        k = min(mstr, sstr) if k is None else k
        if dst is None:
            dst = np.zeros((m, n), np.float32)
        dstr = dst.shape[1]
        acc = np.empty((m, n), np.int32)
        self.lib.oracle_gemm_int8(_ptr(dst, _f32p), dstr, _ptr(acc, _i32p), _ptr(mat, _i8p), mstr,
                                  _ptr(matsc, _f32p), _ptr(src, _i8p), sstr, _ptr(ssc, _f32p), m,
                                  n, k, flavor)
        return dst, acc

    @staticmethod
    def int_sums(mat, src) -> np.ndarray:
        """Exact int32 sums src . mat^T of int8 operands, through a float64
        product: every product and partial sum is an integer of magnitude at
        most 127*127*K < 2**53, so any summation order (BLAS blocking, fused
        multiply-adds) is exact."""
        k = mat.shape[1]
        assert 127 * 127 * k < 2 ** 53
        acc = np.asarray(src, np.float64) @ np.asarray(mat, np.float64).T
        return np.ascontiguousarray(acc.astype(np.int64).astype(np.int32))

    def rescale_matrix(self, acc, ssc, matsc, flavor: int = GCC):
        """gemm_int8's flush (gemma.c:3854-3865) of precomputed int32 sums."""
        acc = np.ascontiguousarray(acc, dtype=np.int32)
        ssc = np.ascontiguousarray(ssc, dtype=np.float32)
        matsc = np.ascontiguousarray(matsc, dtype=np.float32)
        m, n = acc.shape
        dst = np.empty((m, n), np.float32)
        self.lib.oracle_rescale_matrix(_ptr(dst, _f32p), _ptr(acc, _i32p), _ptr(ssc, _f32p),
                                       _ptr(matsc, _f32p), m, n, flavor)
        return dst

    def gemm_int8_full(self, mat, matsc, src, ssc, flavor: int = GCC):
        """gemm_int8 (gemma.c:3937-4054) on dense operands at any size: the
        exact sums of int_sums, then this file's rescale of every cell."""
        return self.rescale_matrix(self.int_sums(mat, src), ssc, matsc, flavor)

    def gemm_f64(self, mat, src, k: int | None = None):
        mat = np.ascontiguousarray(mat, dtype=np.float32)
        src = np.ascontiguousarray(src, dtype=np.float32)
        n, mstr = mat.shape
        m, sstr = src.shape
        k = min(mstr, sstr) if k is None else k
        dst = np.empty((m, n), np.float64)
        mag = np.empty((m, n), np.float64)
        self.lib.oracle_gemm_f64(_ptr(dst, _f64p), _ptr(mag, _f64p), _ptr(mat, _f32p), mstr,
                                 _ptr(src, _f32p), sstr, m, n, k)
        return dst, mag


    def patch_embed_f64(self, img, pe, pe_b, psize: int):
        """img [img_px][img_px][3], pe [dim][3][psize][psize], pe_b [dim]"""
        img = np.ascontiguousarray(img, dtype=np.float32)
        pe = np.ascontiguousarray(pe, dtype=np.float32)
        pe_b = np.ascontiguousarray(pe_b, dtype=np.float32)
        img_px, dim = img.shape[0], pe.shape[0]
        npatch = (img_px // psize) ** 2
        dst = np.empty((npatch, dim), np.float64)
        mag = np.empty((npatch, dim), np.float64)
        self.lib.oracle_patch_embed_f64(_ptr(dst, _f64p), _ptr(mag, _f64p), _ptr(img, _f32p),
                                        _ptr(pe, _f32p), _ptr(pe_b, _f32p), img_px, psize, dim)
        return dst, mag


class RefHarness:
    """The reference's own functions (oracle/_ref/gemma_ref_<compiler>)."""

    def __init__(self, compiler: str = "gcc"):
        self.path = os.path.join(REF_DIR, f"gemma_ref_{compiler}")
        if not os.path.exists(self.path):
            raise FileNotFoundError(f"reference harness not built: {self.path}")
        self.compiler = compiler

    @staticmethod
    def available(compiler: str = "gcc") -> bool:
        return os.path.exists(os.path.join(REF_DIR, f"gemma_ref_{compiler}"))

    def _run(self, op: str, arrays, params, threads: int = 1) -> bytes:
        with tempfile.TemporaryDirectory() as tmp:
            inp = os.path.join(tmp, "in.bin")
            out = os.path.join(tmp, "out.bin")
            with open(inp, "wb") as f:
                for a in arrays:
                    f.write(np.ascontiguousarray(a).tobytes())
            env = dict(os.environ, OMP_NUM_THREADS=str(threads))
            r = subprocess.run([self.path, op, inp, out] + [str(int(p)) for p in params],
                               capture_output=True, text=True, env=env)
            if r.returncode != 0:
                raise RuntimeError(f"{self.path} {op} failed: {r.stderr}")
            with open(out, "rb") as f:
                return f.read()

    def quantize_act(self, vec):
        vec = np.ascontiguousarray(vec, dtype=np.float32)
        n = vec.shape[0]
        raw = self._run("quantize_act", [vec], [n])
        return (np.frombuffer(raw[:n], np.int8).copy(),
                np.frombuffer(raw[n:n + 4], np.float32)[0])

    def quantize_acts(self, src, n: int | None = None, omp: bool = True, threads: int = 4):
        src = np.ascontiguousarray(src, dtype=np.float32)
        m, sstr = src.shape
        n = sstr if n is None else n
        raw = self._run("quantize_acts", [src], [m, n, sstr, int(omp)], threads)
        q = np.frombuffer(raw[:m * n], np.int8).reshape(m, n).copy()
        s = np.frombuffer(raw[m * n:m * n + 4 * m], np.float32).copy()
        return q, s

    def gemv_int8(self, mat, matsc, vec, vsc, omp: bool = True, threads: int = 4):
        mat = np.ascontiguousarray(mat, dtype=np.int8)
        m, n = mat.shape
        raw = self._run("gemv_int8", [mat, np.asarray(matsc, np.float32),
                                      np.asarray(vec, np.int8),
                                      np.array([vsc], np.float32)], [m, n, int(omp)], threads)
        return np.frombuffer(raw, np.float32).copy()

    def gemv_int8_multi(self, jobs, vec, vsc, threads: int = 4):
        """jobs: list of (mat [mj][n] int8, scales [mj])."""
        n = int(np.asarray(vec).shape[0])
        arrays, params = [], [n, len(jobs)]
        for mat, sc in jobs:
            arrays += [np.asarray(mat, np.int8), np.asarray(sc, np.float32)]
            params.append(np.asarray(mat).shape[0])
        arrays += [np.asarray(vec, np.int8), np.array([vsc], np.float32)]
        raw = self._run("gemv_int8_multi", arrays, params, threads)
        return np.frombuffer(raw, np.float32).copy()

    def gemm_int8(self, mat, matsc, src, ssc, k: int, dst, omp: bool = True,
                  threads: int = 4):
        """mat [n][mstr], src [m][sstr], dst [m][dstr] (initial contents)."""
        mat = np.ascontiguousarray(mat, dtype=np.int8)
        src = np.ascontiguousarray(src, dtype=np.int8)
        dst = np.ascontiguousarray(dst, dtype=np.float32)
        n, mstr = mat.shape
        m, sstr = src.shape
        dstr = dst.shape[1]
        raw = self._run("gemm_int8", [mat, np.asarray(matsc, np.float32), src,
                                      np.asarray(ssc, np.float32), dst],
                        [m, n, k, dstr, mstr, sstr, int(omp)], threads)
        out = np.frombuffer(raw[:m * dstr * 4], np.float32).reshape(m, dstr).copy()
        status = int(np.frombuffer(raw[m * dstr * 4:], np.int32)[0])
        return out, status

    def gemv_fpx(self, mat, vec, omp: bool = True, threads: int = 4):
        mat = np.ascontiguousarray(mat, dtype=np.float32)
        m, n = mat.shape
        raw = self._run("gemv_fpx", [mat, np.asarray(vec, np.float32)], [m, n, int(omp)], threads)
        return np.frombuffer(raw, np.float32).copy()

    def gemv_fpx_multi(self, mats, vec, threads: int = 4):
        n = int(np.asarray(vec).shape[0])
        arrays = [np.asarray(mt, np.float32) for mt in mats] + [np.asarray(vec, np.float32)]
        params = [n, len(mats)] + [np.asarray(mt).shape[0] for mt in mats]
        raw = self._run("gemv_fpx_multi", arrays, params, threads)
        return np.frombuffer(raw, np.float32).copy()

    def gemm_fpx(self, mat, src, k: int, dst, omp: bool = True, threads: int = 4):
        mat = np.ascontiguousarray(mat, dtype=np.float32)
        src = np.ascontiguousarray(src, dtype=np.float32)
        dst = np.ascontiguousarray(dst, dtype=np.float32)
        n, mstr = mat.shape
        m, sstr = src.shape
        dstr = dst.shape[1]
        raw = self._run("gemm_fpx", [mat, src, dst], [m, n, k, dstr, mstr, sstr, int(omp)],
                        threads)
        out = np.frombuffer(raw[:m * dstr * 4], np.float32).reshape(m, dstr).copy()
        return out, int(np.frombuffer(raw[m * dstr * 4:], np.int32)[0])

    def bench(self, args, threads: int) -> dict:
        env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="close",
                   OMP_PLACES="cores")
        r = subprocess.run([self.path, "bench"] + [str(a) for a in args], capture_output=True,
                           text=True, env=env, check=True)
        return json.loads(r.stdout.strip().splitlines()[-1])
