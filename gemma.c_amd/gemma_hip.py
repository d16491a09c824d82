"""ctypes binding of libgemma_hip.so (the C ABI in include/gemma_hip.h).

This is how Python code (the tests, bench.py, __graft_entry__) reaches the
HIP kernels: every call goes through the exported C functions, exactly as the
reference's C call sites would.  Device buffers are plain addresses; torch is
only used by callers to allocate HBM and to name a stream.

A failing call raises ``GemmaHipError`` with the library's message
(gemma_hip_last_error); the library never falls back to the CPU, so a missing
or unloadable ``.so`` is an error too.
"""

from __future__ import annotations

import ctypes
import os
import re

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "lib", "libgemma_hip.so")
HEADER_PATH = os.path.join(REPO_DIR, "include", "gemma_hip.h")
MAX_JOBS = 4


class GemmaHipError(RuntimeError):
    pass


class PerfEntry(ctypes.Structure):
    """gemma_hip_perf_entry: one (phase, op) total of GPU time."""

    _fields_ = [("op", ctypes.c_char_p), ("phase", ctypes.c_int), ("sec", ctypes.c_double),
                ("calls", ctypes.c_long)]


PERF_PHASES = ("prefill", "decode", "vision")  # the reference's PerfPhase order
# the reference's PerfOp names in report order (gemma.c:2409-2431)
PERF_OPS = ("rmsnorm", "layernorm", "quantize_act", "gemv_fpx", "gemv_int8", "gemv_fpx_nn",
            "gemm_fpx", "gemm_fpx_nn", "gemm_int8", "softmax", "gelu", "rope",
            "sample_from_logits")


def perf_table(perf) -> str:
    """perf_read()'s totals as the per-phase tables of the reference's report
    (perf_print, gemma.c:6824-6862: function, calls, total ms, avg us, share of
    the phase's recorded time)."""
    lines = []
    for ph in PERF_PHASES:
        ops = perf.get(ph)
        if not ops:
            continue
        total = sum(sec for sec, _ in ops.values())
        lines.append(f"{ph}: {total * 1e3:.3f} ms of GPU time")
        lines.append(f"  {'function':<18} {'calls':>8} {'total ms':>10} {'avg us':>9} {'share':>7}")
        lines.append("  " + "-" * 18 + " " + "-" * 8 + " " + "-" * 10 + " " + "-" * 9 + " " + "-" * 7)
        for op in PERF_OPS:
            if op not in ops:
                continue
            sec, calls = ops[op]
            share = 100.0 * sec / total if total > 0 else 0.0
            lines.append(f"  {op:<18} {calls:>8} {sec * 1e3:>10.3f} {sec * 1e6 / calls:>9.2f} "
                         f"{share:>6.1f}%")
        lines.append(f"  {'total':<18} {'':>8} {total * 1e3:>10.3f}")
    return "\n".join(lines)


class Job(ctypes.Structure):
    """gemma_hip_job: mirrors the reference's GemvJob (gemma.c:2790-2800)."""

    _fields_ = [("w", ctypes.c_void_p), ("sc", ctypes.c_void_p),
                ("dst", ctypes.c_void_p), ("m", ctypes.c_int)]


class TextConfig(ctypes.Structure):
    """gemma_hip_text_config: the reference's TextConfig (gemma.c:740-761)."""

    _fields_ = [(n, ctypes.c_int) for n in ("nl", "n_heads", "nkv", "hdim", "dim", "mlp_dim",
                                            "q_scale", "slide", "nvocab")] + \
               [(n, ctypes.c_float) for n in ("theta_l", "theta_g", "eps", "sc_att", "sc_log")] + \
               [(n, ctypes.c_int) for n in ("qk_norm", "mlp_pre", "mlp_pst")] + \
               [("swa", ctypes.c_void_p)]


class Layer(ctypes.Structure):
    """gemma_hip_layer: one TextDecoderLayer (gemma.c:1173-1195)."""

    _fields_ = [(n, ctypes.c_void_p) for n in (
        "wq", "wk", "wv", "wo", "w1", "w2", "w3",
        "wq_s", "wk_s", "wv_s", "wo_s", "w1_s", "w2_s", "w3_s",
        "nq", "nk", "n1", "n2", "n3", "n4")]


class LayerF32(ctypes.Structure):
    """gemma_hip_layer_f32: one TextDecoderLayer of an fp32 ('U') file."""

    _fields_ = [(n, ctypes.c_void_p) for n in (
        "wq", "wk", "wv", "wo", "w1", "w2", "w3", "nq", "nk", "n1", "n2", "n3", "n4")]


class VisionConfig(ctypes.Structure):
    """gemma_hip_vision_config: the reference's VisionConfig (gemma.c:713-721)
    plus TextConfig's img_tok and dim (here text_dim)."""

    _fields_ = [(n, ctypes.c_int) for n in ("nl", "n_heads", "img_px", "psize", "dim",
                                            "mlp_dim")] + \
               [("eps", ctypes.c_float), ("img_tok", ctypes.c_int), ("text_dim", ctypes.c_int)]


class VisionLayer(ctypes.Structure):
    """gemma_hip_vision_layer: one VisionEncoderLayer (gemma.c:1234-1256)."""

    _fields_ = [(n, ctypes.c_void_p) for n in (
        "wq", "wk", "wv", "wo", "w1", "w2",
        "wq_s", "wk_s", "wv_s", "wo_s", "w1_s", "w2_s",
        "bq", "bk", "bv", "bo", "b1", "b2", "n1", "n1_b", "n2", "n2_b")]


class VisionLayerF32(ctypes.Structure):
    """gemma_hip_vision_layer_f32: one VisionEncoderLayer of an fp32 ('U') file."""

    _fields_ = [(n, ctypes.c_void_p) for n in (
        "wq", "wk", "wv", "wo", "w1", "w2",
        "bq", "bk", "bv", "bo", "b1", "b2", "n1", "n1_b", "n2", "n2_b")]


_P = ctypes.c_void_p
_I = ctypes.c_int

# attention arithmetic of the prompt passes and the vision tower
# (GEMMA_HIP_ATTN_*): fp32 matrix cores (the default) or fp64 (verification)
ATTN_F64, ATTN_F32 = 0, 1
_SIGS = {
    "gemma_hip_init": (_I, [_I]),
    "gemma_hip_shutdown": (None, []),
    "gemma_hip_last_error": (ctypes.c_char_p, []),
    "gemma_hip_sync": (_I, [_P]),
    "gemma_hip_register_weights": (_I, [_P, ctypes.c_size_t]),
    "gemma_hip_release_weights": (_I, [_P]),
    "gemma_hip_device_ptr": (_P, [_P]),
    "gemma_hip_quantize": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "gemma_hip_matmul": (_I, [_P, _I, _P, _I, _P, _P, _I, _P, _I, _I, _I, _P]),
    "gemma_hip_matmul_noalloc": (_I, [_P, _I, _P, _I, _P, _P, _I, _P, _I, _I, _I, _P]),
    "gemma_hip_perf_enable": (_I, [_I]),
    "gemma_hip_perf_phase": (_I, [_I]),
    "gemma_hip_perf_read": (_I, [ctypes.POINTER(PerfEntry), _I, ctypes.POINTER(_I)]),
    "gemma_hip_matmul_heads": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "gemma_hip_matmul_cols": (_I, [_P, _I, ctypes.POINTER(Job), _I, _P, _I, _P, _I, _I, _P]),
    "gemma_hip_prefill_attention": (_I, [_P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                         ctypes.c_float, ctypes.c_float, _I, _I, _P]),
    "gemma_hip_matmul_multi": (_I, [ctypes.POINTER(Job), _I, _P, _P, _I, _P]),
    "gemma_hip_quantize_matmul": (_I, [ctypes.POINTER(Job), _I, _P, _I, _P, _P, _P]),
    "gemma_hip_matmul_f32": (_I, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _P]),
    "gemma_hip_matmul_f32_cols": (_I, [_P, _I, ctypes.POINTER(Job), _I, _P, _I, _I, _I, _P]),
    "gemma_hip_matmul_f32_multi": (_I, [ctypes.POINTER(Job), _I, _P, _I, _P]),
    "gemma_hip_quantize_act_host": (_I, [_P, _P, _P, _I]),
    "gemma_hip_quantize_acts_host": (_I, [_P, _P, _P, _I, _I, _I]),
    "gemma_hip_gemv_int8_host": (_I, [_P, _P, _P, _P, ctypes.c_float, _I, _I]),
    "gemma_hip_gemv_int8_multi_host": (_I, [ctypes.POINTER(Job), _I, _P, ctypes.c_float, _I]),
    "gemma_hip_gemm_int8_host": (_I, [_P, _I, _P, _I, _P, _P, _I, _P, _I, _I, _I]),
    "gemma_hip_gemv_fpx_host": (_I, [_P, _P, _P, _I, _I]),
    "gemma_hip_gemv_fpx_multi_host": (_I, [ctypes.POINTER(Job), _I, _P, _I]),
    "gemma_hip_gemm_fpx_host": (_I, [_P, _I, _P, _I, _P, _I, _I, _I, _I]),
    "gemma_hip_patch_embed": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _P]),
    "gemma_hip_patch_embed_host": (_I, [_P, _P, _P, _P, _I, _I, _I]),
    "gemma_hip_decoder_create": (_P, [ctypes.POINTER(TextConfig), ctypes.POINTER(Layer), _P, _P,
                                      _P, _I]),
    "gemma_hip_decoder_create_f32": (_P, [ctypes.POINTER(TextConfig), ctypes.POINTER(LayerF32),
                                          _P, _P, _I]),
    "gemma_hip_decoder_destroy": (None, [_P]),
    "gemma_hip_decoder_step": (_I, [_P, _I, _I, _P, ctypes.POINTER(_I)]),
    "gemma_hip_decoder_generate": (_I, [_P, _I, _I, _I, _P]),
    "gemma_hip_decoder_prefill": (_I, [_P, _P, _I, _I, _P, ctypes.POINTER(_I)]),
    "gemma_hip_decoder_prefill_rows": (_I, [_P, _P, _I, _I, _I, _P, ctypes.POINTER(_I)]),
    "gemma_hip_gemma_image": (_I, [_P, _P, _P, ctypes.POINTER(_I), _P, ctypes.POINTER(_I)]),
    "gemma_hip_decoder_logits": (_P, [_P]),
    "gemma_hip_decoder_set_attention": (_I, [_P, _I]),
    "gemma_hip_vision_create": (_P, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "gemma_hip_vision_create_f32": (_P, [_P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "gemma_hip_vision_destroy": (None, [_P]),
    "gemma_hip_vision_forward": (_I, [_P, _P, _P]),
    "gemma_hip_vision_set_attention": (_I, [_P, _I]),
    "gemma_hip_vision_attention": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
}


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Every function the public header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gemma_hip_\w+)\s*\(", text)))


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise GemmaHipError(f"{path} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _addr(x) -> int | None:
    """Device/host address of a torch tensor, numpy array or int (None -> NULL)."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    raise TypeError(f"cannot take the address of {type(x)}")


class GemmaHip:
    """Thin object wrapper: each method is one C call; errors raise."""

    def __init__(self, device: int = 0, path: str = LIB_PATH):
        self.lib = load(path)
        self._check(self.lib.gemma_hip_init(device))
        self.device = device

    def _check(self, rc: int) -> None:
        if rc != 0:
            raise GemmaHipError(self.lib.gemma_hip_last_error().decode())

    def close(self) -> None:
        self.lib.gemma_hip_shutdown()

    def sync(self, stream: int | None = None) -> None:
        self._check(self.lib.gemma_hip_sync(stream))

    @staticmethod
    def jobs(specs) -> tuple[ctypes.Array, int]:
        """specs: iterable of (w, sc, dst, m)."""
        specs = list(specs)
        arr = (Job * max(1, len(specs)))()
        for i, (w, sc, dst, m) in enumerate(specs):
            arr[i] = Job(_addr(w), _addr(sc), _addr(dst), int(m))
        return arr, len(specs)

    # device entry points ---------------------------------------------------
    def quantize(self, dst, dsc, src, sstr, m, n, stream=None):
        self._check(self.lib.gemma_hip_quantize(_addr(dst), _addr(dsc), _addr(src), sstr, m,
                                                n, stream))

    def matmul(self, dst, dstr, mat, mstr, matsc, src, sstr, ssc, m, n, k, stream=None):
        self._check(self.lib.gemma_hip_matmul(_addr(dst), dstr, _addr(mat), mstr, _addr(matsc),
                                              _addr(src), sstr, _addr(ssc), m, n, k, stream))

    def perf_enable(self, on=True):
        self._check(self.lib.gemma_hip_perf_enable(1 if on else 0))

    def perf_phase(self, phase):
        self._check(self.lib.gemma_hip_perf_phase(PERF_PHASES.index(phase)))

    def perf_read(self):
        """{phase: {op: (seconds, calls)}} of the timed entry points."""
        out = (PerfEntry * 64)()
        n = ctypes.c_int(0)
        self._check(self.lib.gemma_hip_perf_read(out, 64, ctypes.byref(n)))
        res = {}
        for e in out[:min(n.value, 64)]:
            res.setdefault(PERF_PHASES[e.phase], {})[e.op.decode()] = (e.sec, e.calls)
        return res

    def matmul_noalloc(self, dst, dstr, mat, mstr, matsc, src, sstr, ssc, m, n, k,
                       stream=None):
        self._check(self.lib.gemma_hip_matmul_noalloc(_addr(dst), dstr, _addr(mat), mstr,
                                                      _addr(matsc), _addr(src), sstr, _addr(ssc),
                                                      m, n, k, stream))

    def matmul_heads(self, dst, mat, matsc, src, ssc, m, heads, hdim, k, stream=None):
        self._check(self.lib.gemma_hip_matmul_heads(_addr(dst), _addr(mat), _addr(matsc),
                                                    _addr(src), _addr(ssc), m, heads, hdim, k,
                                                    stream))

    def matmul_cols(self, dst, dstr, specs, src, sstr, ssc, m, k, stream=None):
        """specs: (w, sc, rows) per job; job j fills the next rows columns."""
        arr, n = self.jobs((w, sc, None, rows) for w, sc, rows in specs)
        self._check(self.lib.gemma_hip_matmul_cols(_addr(dst), dstr, arr, n, _addr(src), sstr,
                                                   _addr(ssc), m, k, stream))

    def matmul_multi(self, specs, x, xs, k, stream=None):
        arr, n = self.jobs(specs)
        self._check(self.lib.gemma_hip_matmul_multi(arr, n, _addr(x), _addr(xs), k, stream))

    def quantize_matmul(self, specs, x, k, xq=None, xs=None, stream=None):
        arr, n = self.jobs(specs)
        self._check(self.lib.gemma_hip_quantize_matmul(arr, n, _addr(x), k, _addr(xq),
                                                       _addr(xs), stream))

    def matmul_f32(self, dst, dstr, mat, mstr, src, sstr, m, n, k, stream=None):
        self._check(self.lib.gemma_hip_matmul_f32(_addr(dst), dstr, _addr(mat), mstr,
                                                  _addr(src), sstr, m, n, k, stream))

    def matmul_f32_cols(self, dst, dstr, specs, src, sstr, m, k, stream=None):
        """specs: (w, rows) per job; job j fills the next rows columns."""
        arr, n = self.jobs((w, None, None, rows) for w, rows in specs)
        self._check(self.lib.gemma_hip_matmul_f32_cols(_addr(dst), dstr, arr, n, _addr(src),
                                                       sstr, m, k, stream))

    def matmul_f32_multi(self, specs, x, k, stream=None):
        arr, n = self.jobs(specs)
        self._check(self.lib.gemma_hip_matmul_f32_multi(arr, n, _addr(x), k, stream))

    def patch_embed(self, dst, img, pe, pe_b, img_px, psize, dim, work=None, stream=None):
        self._check(self.lib.gemma_hip_patch_embed(_addr(dst), _addr(img), _addr(pe),
                                                   _addr(pe_b), img_px, psize, dim,
                                                   _addr(work), stream))

    # weights ---------------------------------------------------------------
    def prefill_attention(self, out, q, q_stride, kc, vc, n, pos0, n_heads, nkv, hdim, clen,
                          slide, asc, sc_att, dense, mode, stream=None):
        """gemma_hip_prefill_attention on device pointers."""
        self._check(self.lib.gemma_hip_prefill_attention(
            _addr(out), _addr(q), q_stride, _addr(kc), _addr(vc), n, pos0, n_heads, nkv, hdim,
            clen, slide, float(asc), float(sc_att), 1 if dense else 0, mode, stream))

    def vision_attention(self, out, qkv, bias, n, n_heads, dim, mode=0, stream=None):
        """gemma_hip_vision_attention on device pointers."""
        self._check(self.lib.gemma_hip_vision_attention(_addr(out), _addr(qkv), _addr(bias), n,
                                                        n_heads, dim, mode,
                                                        stream))

    def register_weights(self, host, nbytes: int):
        self._check(self.lib.gemma_hip_register_weights(_addr(host), nbytes))

    def release_weights(self, host):
        self._check(self.lib.gemma_hip_release_weights(_addr(host)))

    def device_ptr(self, host) -> int | None:
        return self.lib.gemma_hip_device_ptr(_addr(host))

    # device-resident decoder -----------------------------------------------
    def vision(self, vis, attention=None) -> "Vision":
        """A vision tower over a dict of VisionEncoder weights
        (model_bin.synth_vision's layout): registers every int8 tensor.
        `attention` (ATTN_F32 or ATTN_F64) sets the attention's arithmetic;
        None keeps the library's default (ATTN_F32)."""
        return _with_mode(Vision(self, vis), attention)

    def decoder(self, model, clen: int, attention=None) -> "Decoder":
        """A decoder over a model from model_bin.read_bin(): registers every
        int8 tensor (each as its own range) and builds the step graph.
        `attention` as for vision(), for the prompt passes."""
        return _with_mode(Decoder(self, model, clen), attention)


def _with_mode(obj, attention):
    if attention is not None:
        try:
            obj.set_attention(attention)
        except Exception:
            obj.close()
            raise
    return obj


class Decoder:
    """gemma_hip_decoder_*: forward_gemma_decode (gemma.c:5456) on the GPU."""

    def __init__(self, gh: GemmaHip, model, clen: int):
        import numpy as np

        self.gh, self.lib = gh, gh.lib
        c = model["config"]
        self.nvocab = c["nvocab"]
        self._keep = []
        self._registered = []

        def reg(arr):
            arr = np.asarray(arr)
            gh.register_weights(arr, arr.nbytes)
            self._registered.append(arr)
            return arr.ctypes.data

        def host(arr):
            arr = np.ascontiguousarray(arr, np.float32)
            self._keep.append(arr)
            return arr.ctypes.data

        swa = np.asarray(c["swa"], np.uint8)
        self._keep.append(swa)
        cfg = TextConfig(c["nl"], c["n_heads"], c["nkv"], c["hdim"], c["dim"], c["mlp_dim"],
                         c["q_scale"], c["slide"], c["nvocab"], c["theta_l"], c["theta_g"],
                         c["eps"], c["sc_att"], c["sc_log"], int(c["qk_norm"]),
                         int(c["mlp_pre"]), int(c["mlp_pst"]), swa.ctypes.data)
        quant = c.get("quant", True)
        layers = ((Layer if quant else LayerF32) * c["nl"])()
        try:
            for i, ly in enumerate(model["layers"]):
                f = {}
                for w in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
                    if quant:
                        f[w] = reg(ly[w][0])
                        f[w + "_s"] = reg(ly[w][1])
                    else:  # 'U': one fp32 [out][in] array
                        f[w] = reg(ly[w])
                for n in ("nq", "nk", "n1", "n2", "n3", "n4"):
                    f[n] = host(ly[n]) if ly.get(n) is not None else None
                layers[i] = (Layer if quant else LayerF32)(**f)
            fnorm = host(model["fnorm"])
            if quant:
                emb_q, emb_s = reg(model["emb"][0]), reg(model["emb"][1])
                self.handle = self.lib.gemma_hip_decoder_create(ctypes.byref(cfg), layers,
                                                                emb_q, emb_s, fnorm, clen)
            else:
                self.handle = self.lib.gemma_hip_decoder_create_f32(
                    ctypes.byref(cfg), layers, reg(model["emb"]), fnorm, clen)
            if not self.handle:
                raise GemmaHipError(self.lib.gemma_hip_last_error().decode())
        except Exception:
            self._release()
            raise

    def _release(self):
        for arr in self._registered:
            self.gh.release_weights(arr)
        self._registered = []

    def step(self, token: int, pos: int, logits=None) -> int:
        nxt = ctypes.c_int(-1)
        self.gh._check(self.lib.gemma_hip_decoder_step(self.handle, token, pos, _addr(logits),
                                                       ctypes.byref(nxt)))
        return nxt.value

    def prefill(self, tokens, pos: int, logits=None) -> int:
        """The prompt pass (forward_gemma_prefill, gemma.c:5501) over `tokens` at
        positions pos .. pos+len-1; returns the argmax after the last one."""
        import numpy as np

        toks = np.ascontiguousarray(tokens, np.int32)
        nxt = ctypes.c_int(-1)
        self.gh._check(self.lib.gemma_hip_decoder_prefill(self.handle, toks.ctypes.data,
                                                          int(toks.size), pos, _addr(logits),
                                                          ctypes.byref(nxt)))
        return nxt.value

    def prefill_rows(self, x, pos: int, mask: bool = True, logits=None) -> int:
        """The prompt pass over embedding rows x [n][dim] (forward_text_chunk,
        gemma.c:4985, on rows a caller placed in tb->x) at positions
        pos .. pos+n-1; mask=False is the dense attention of image tokens
        (gemma.c:5258-5290).  Returns the argmax after the last row."""
        import numpy as np

        x = np.ascontiguousarray(x, np.float32)
        nxt = ctypes.c_int(-1)
        self.gh._check(self.lib.gemma_hip_decoder_prefill_rows(
            self.handle, x.ctypes.data, int(x.shape[0]), pos, int(bool(mask)), _addr(logits),
            ctypes.byref(nxt)))
        return nxt.value

    def image(self, vision: "Vision", img, pos: int, logits=None):
        """forward_gemma_image (gemma.c:5561): the vision tower on img and the
        dense prompt pass of its soft tokens at pos, device to device.
        Returns (next position, argmax after the last soft token)."""
        import numpy as np

        img = np.ascontiguousarray(img, np.float32)
        assert img.shape == vision.img_shape
        p, nxt = ctypes.c_int(pos), ctypes.c_int(-1)
        self.gh._check(self.lib.gemma_hip_gemma_image(self.handle, vision.handle, img.ctypes.data,
                                                      ctypes.byref(p), _addr(logits),
                                                      ctypes.byref(nxt)))
        return p.value, nxt.value

    def generate(self, token: int, pos: int, n: int):
        import numpy as np

        out = np.empty(max(1, n), np.int32)
        self.gh._check(self.lib.gemma_hip_decoder_generate(self.handle, token, pos, n,
                                                           out.ctypes.data))
        return out[:n]

    ATTN_F64, ATTN_F32 = ATTN_F64, ATTN_F32

    def set_attention(self, mode: int):
        """GEMMA_HIP_ATTN_F32 (1, the default) or GEMMA_HIP_ATTN_F64 (0): the
        prompt passes' attention on the fp32 or the fp64 matrix cores."""
        self.gh._check(self.lib.gemma_hip_decoder_set_attention(self.handle, int(mode)))

    def logits_ptr(self) -> int:
        return self.lib.gemma_hip_decoder_logits(self.handle)

    def close(self):
        if getattr(self, "handle", None):
            self.lib.gemma_hip_decoder_destroy(self.handle)
            self.handle = None
        self._release()



class Vision:
    """gemma_hip_vision_*: forward_vision (gemma.c:4394) on the GPU."""

    def __init__(self, gh: GemmaHip, vis):
        import numpy as np

        self.gh, self.lib = gh, gh.lib
        c = vis["config"]
        self.out_shape = (c["img_tok"], c["text_dim"])
        self.img_shape = (c["img_px"], c["img_px"], 3)
        self._keep, self._registered = [], []

        def reg(arr):
            arr = np.ascontiguousarray(arr)
            gh.register_weights(arr, arr.nbytes)
            self._registered.append(arr)
            return arr.ctypes.data

        def host(arr):
            arr = np.ascontiguousarray(arr, np.float32)
            self._keep.append(arr)
            return arr.ctypes.data

        cfg = VisionConfig(c["nl"], c["n_heads"], c["img_px"], c["psize"], c["dim"],
                           c["mlp_dim"], c["eps"], c["img_tok"], c["text_dim"])
        quant = c.get("quant", True)
        kind = VisionLayer if quant else VisionLayerF32
        layers = (kind * c["nl"])()
        try:
            for i, ly in enumerate(vis["layers"]):
                f = {}
                for w in ("wq", "wk", "wv", "wo", "w1", "w2"):
                    if quant:
                        f[w] = reg(ly[w][0])
                        f[w + "_s"] = reg(ly[w][1])
                    else:  # 'U': one fp32 [out][in] array
                        f[w] = reg(ly[w])
                for b in ("bq", "bk", "bv", "bo", "b1", "b2", "n1", "n1_b", "n2", "n2_b"):
                    f[b] = host(ly[b])
                layers[i] = kind(**f)
            if quant:
                self.handle = self.lib.gemma_hip_vision_create(
                    ctypes.byref(cfg), layers, host(vis["pe"]), host(vis["pe_b"]),
                    reg(vis["pos"][0]), reg(vis["pos"][1]), host(vis["post_n"]),
                    host(vis["post_nb"]), host(vis["norm"]), reg(vis["proj"][0]),
                    reg(vis["proj"][1]))
            else:
                self.handle = self.lib.gemma_hip_vision_create_f32(
                    ctypes.byref(cfg), layers, host(vis["pe"]), host(vis["pe_b"]),
                    reg(vis["pos"]), host(vis["post_n"]), host(vis["post_nb"]),
                    host(vis["norm"]), reg(vis["proj"]))
            if not self.handle:
                raise GemmaHipError(self.lib.gemma_hip_last_error().decode())
        except Exception:
            self._release()
            raise

    def _release(self):
        for arr in self._registered:
            self.gh.release_weights(arr)
        self._registered = []

    ATTN_F64, ATTN_F32 = ATTN_F64, ATTN_F32

    def set_attention(self, mode: int):
        """GEMMA_HIP_ATTN_F32 (1, the default) or GEMMA_HIP_ATTN_F64 (0): the
        attention's arithmetic, fp32 or fp64 matrix cores."""
        self.gh._check(self.lib.gemma_hip_vision_set_attention(self.handle, int(mode)))

    def forward(self, img):
        """img [img_px][img_px][3] float32 -> soft tokens [img_tok][text_dim]."""
        import numpy as np

        img = np.ascontiguousarray(img, np.float32)
        assert img.shape == self.img_shape
        out = np.empty(self.out_shape, np.float32)
        self.gh._check(self.lib.gemma_hip_vision_forward(self.handle, img.ctypes.data,
                                                         out.ctypes.data))
        return out

    def close(self):
        if getattr(self, "handle", None):
            self.lib.gemma_hip_vision_destroy(self.handle)
            self.handle = None
        self._release()
