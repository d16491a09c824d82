"""Random-init Gemma.c model files (.bin) in the reference's layout.

The reference loads models exported from Hugging Face checkpoints
(export.py); none can be downloaded here, so the end-to-end runs at the
gemma-3-270m / 1b / 4b shapes use random weights written in exactly the
layout the reference's loader reads (gemma.c:1913-2138):

  "GEMA" + "f32" + 'Q'                       header (gemma.c:1915-1939)
  text config, big-endian: u8 nl, n_heads, nkv; u16 hdim, dim, mlp_dim,
    q_scale, slide, img_tok; u32 max_seq, nvocab; f32 theta_l, theta_g,
    eps, sc_att, sc_log                      (gemma.c:770-784)
  u8 n_bytes + sliding-window bits, MSB first (gemma.c:786-805)
  u8 flags: 4 qk_norm, 2 pre-FFN norm, 1 post-FFN norm (gemma.c:807-816)
  vocabulary: nvocab Pascal strings; u32 BE merge count; 2 strings per
    merge                                    (gemma.c:905-985)
  tensors, little-endian, back to back (gemma.c:1386-1469): emb, then per
    layer wq wk wv wo [nq nk] w1(up) w2(gate) w3(down) n1 n2 [n3] [n4],
    then fnorm.  A quantized tensor is int8 [out][in] followed by fp32 [out]
    row scales (gemma.c:1125-1156).

Weights are N(0, 0.02), quantized per output row as export.py's
Linear.quantize does (model.py:151-161): s = max(amax, 1e-8) / 127,
q = round-half-even(w / s) clamped to [-127, 127].  Norm weights are 0 (the
reference applies them as w + 1, gemma.c:2508-2521).
"""

from __future__ import annotations

import os
import struct

import numpy as np

# text-model shapes of the gemma-3 270m, 1b and 4b checkpoints
CONFIGS = {
    "gemma-3-270m": dict(nl=18, n_heads=4, nkv=1, hdim=256, dim=640, mlp=2048, slide=512),
    "gemma-3-1b": dict(nl=26, n_heads=4, nkv=1, hdim=256, dim=1152, mlp=6912, slide=512),
    "gemma-3-4b": dict(nl=34, n_heads=8, nkv=4, hdim=256, dim=2560, mlp=10240, slide=1024),
}
NVOCAB = 262144
SPECIALS = ["<pad>", "<eos>", "<bos>", "<unk>", "<start_of_turn>", "<end_of_turn>"]


def quantize_rows(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8 (model.py:151-161)."""
    amax = np.max(np.abs(w), axis=1)
    scale = (np.maximum(amax, np.float32(1e-8)) / np.float32(127.0)).astype(np.float32)
    q = np.rint(w / scale[:, None])
    return np.clip(q, -127, 127).astype(np.int8), scale


def _write_qtensor(f, rng, rows: int, cols: int, chunk_rows: int = 32768) -> None:
    scales = np.empty(rows, np.float32)
    for r0 in range(0, rows, chunk_rows):
        r1 = min(rows, r0 + chunk_rows)
        w = rng.standard_normal((r1 - r0, cols), dtype=np.float32) * np.float32(0.02)
        q, s = quantize_rows(w)
        f.write(q.tobytes())
        scales[r0:r1] = s
    f.write(scales.tobytes())


def _pascal(s: str) -> bytes:
    b = s.encode()
    assert len(b) <= 255
    return bytes([len(b)]) + b


def write_bin(path: str, name: str, seed: int = 1234, nvocab: int = NVOCAB,
              layers: int | None = None) -> str:
    """Write a random-init W8A8 (f32 build) text model of shape `name`;
    `nvocab` and `layers` shrink it for quick tests."""
    c = CONFIGS[name]
    nl, dim, hdim, mlp = c["nl"], c["dim"], c["hdim"], c["mlp"]
    if layers is not None:
        nl = layers
    q_sz, kv_sz = c["n_heads"] * hdim, c["nkv"] * hdim
    rng = np.random.default_rng(seed)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(b"GEMA" + b"f32" + b"Q")
        f.write(struct.pack(">BBBHHHHHHIIfffff", nl, c["n_heads"], c["nkv"], hdim, dim, mlp,
                            hdim, c["slide"], 256, 32768, nvocab, 10000.0, 1000000.0, 1e-6,
                            0.0, 0.0))
        nbytes = (nl + 7) // 8
        bits = bytearray(nbytes)
        for i in range(nl):
            if (i + 1) % 6 != 0:  # gemma 3: five sliding-window layers per global one
                bits[i // 8] |= 1 << (7 - i % 8)
        f.write(bytes([nbytes]) + bytes(bits))
        f.write(bytes([4 | 2 | 1]))  # qk_norm, pre- and post-FFN norms; text only
        vocab = SPECIALS + [f"t{i}" for i in range(len(SPECIALS), nvocab)]
        f.write(b"".join(_pascal(s) for s in vocab))
        f.write(struct.pack(">I", 1) + _pascal("t") + _pascal("0"))
        zeros_dim = np.zeros(dim, np.float32).tobytes()
        _write_qtensor(f, rng, nvocab, dim)  # emb, also the tied LM head
        for _ in range(nl):
            _write_qtensor(f, rng, q_sz, dim)    # wq
            _write_qtensor(f, rng, kv_sz, dim)   # wk
            _write_qtensor(f, rng, kv_sz, dim)   # wv
            _write_qtensor(f, rng, dim, q_sz)    # wo
            f.write(np.zeros(hdim, np.float32).tobytes() * 2)  # nq, nk
            _write_qtensor(f, rng, mlp, dim)     # w1 (up)
            _write_qtensor(f, rng, mlp, dim)     # w2 (gate)
            _write_qtensor(f, rng, dim, mlp)     # w3 (down)
            f.write(zeros_dim * 4)               # n1, n2, n3, n4
        f.write(zeros_dim)                       # fnorm
    os.replace(tmp, path)
    return path


def ensure_bin(directory: str, name: str, seed: int = 1234) -> str:
    """Path of the random-init model `name`, written on first use."""
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, f"{name}-w8a8-seed{seed}.bin")
    if not os.path.exists(path):
        write_bin(path, name, seed)
    return path


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="write a random-init Gemma.c .bin")
    ap.add_argument("name", choices=sorted(CONFIGS))
    ap.add_argument("path")
    ap.add_argument("--seed", type=int, default=1234)
    a = ap.parse_args()
    print(write_bin(a.path, a.name, a.seed))
