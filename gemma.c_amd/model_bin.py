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
    # the head dim of the larger checkpoints (128, gemma-3-27b) at test size
    "test-hd128": dict(nl=2, n_heads=4, nkv=2, hdim=128, dim=256, mlp=512, slide=512),
    # widths that are multiples of 16 but not of the GEMM tile (64/128) or of
    # 256-thread vectors: dim 208, mlp 1040, one q head per kv head
    "test-odd": dict(nl=2, n_heads=2, nkv=2, hdim=128, dim=208, mlp=1040, slide=512),
    # rows of 176 and 352 16-byte chunks (dim 704, mlp 1408): the fp32 GEMVs
    # take one pass of 12 chunks per lane at 16 and 32 lanes
    "test-cpl12": dict(nl=2, n_heads=2, nkv=1, hdim=128, dim=704, mlp=1408, slide=512),
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


def _write_ftensor(f, rng, rows: int, cols: int, chunk_rows: int = 32768) -> None:
    """An unquantized linear layer ('U' files): fp32 [rows][cols], N(0, 0.02)."""
    for r0 in range(0, rows, chunk_rows):
        r1 = min(rows, r0 + chunk_rows)
        f.write((rng.standard_normal((r1 - r0, cols), dtype=np.float32)
                 * np.float32(0.02)).tobytes())


def _pascal(s: str) -> bytes:
    b = s.encode()
    assert len(b) <= 255
    return bytes([len(b)]) + b


def write_bin(path: str, name: str, seed: int = 1234, nvocab: int = NVOCAB,
              layers: int | None = None, slide: int | None = None, sc_att: float = 0.0,
              sc_log: float = 0.0, flags: int = 4 | 2 | 1, norm_std: float = 0.0,
              vision: dict | None = None, swa: list | None = None, quant: bool = True) -> str:
    """Write a random-init W8A8 (f32 build) text model of shape `name`;
    `nvocab` and `layers` shrink it for quick tests, `slide`, the softcaps
    and the flags byte (4 qk-norm, 2 pre-FFN norm, 1 post-FFN norm) select
    the other code paths of the reference's decoder (`swa`, one flag per
    layer, overrides gemma 3's five sliding layers per global one); norm_std > 0 draws the
    norm weights from N(0, norm_std) instead of zeros.  `vision`, a
    synth_vision() dict whose text_dim is this model's dim, makes the file
    multimodal (flag 8): its VisionConfig follows the flags byte (gemma.c:
    723-733), the vocabulary gains the image soft token (905-913) and the
    tower's tensors follow the text decoder's in read_vision_encoder's order
    (1688-1762).  quant=False writes an unquantized ('U') file: every linear
    layer fp32 [out][in] with no scales (qtensor_size, gemma.c:1125-1131),
    the path the reference's gemv_fpx / gemm_fpx call sites take."""
    c = dict(CONFIGS[name])
    nl, dim, hdim, mlp = c["nl"], c["dim"], c["hdim"], c["mlp"]
    if layers is not None:
        nl = layers
    if slide is not None:
        c["slide"] = slide
    q_sz, kv_sz = c["n_heads"] * hdim, c["nkv"] * hdim
    rng = np.random.default_rng(seed)
    if vision is not None and vision["config"].get("quant", True) != quant:
        raise ValueError("the vision tower and the decoder must both be W8A8 or both fp32")
    linear = _write_qtensor if quant else _write_ftensor
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(b"GEMA" + b"f32" + (b"Q" if quant else b"U"))
        vc = vision["config"] if vision is not None else None
        if vc is not None and vc["text_dim"] != dim:
            raise ValueError("the vision tower's text_dim must be the model's dim")
        img_tok = vc["img_tok"] if vc is not None else 256
        f.write(struct.pack(">BBBHHHHHHIIfffff", nl, c["n_heads"], c["nkv"], hdim, dim, mlp,
                            hdim, c["slide"], img_tok, 32768, nvocab, 10000.0, 1000000.0, 1e-6,
                            sc_att, sc_log))
        nbytes = (nl + 7) // 8
        bits = bytearray(nbytes)
        for i in range(nl):
            sliding = swa[i] if swa is not None else (i + 1) % 6 != 0
            if sliding:  # gemma 3: five sliding-window layers per global one
                bits[i // 8] |= 1 << (7 - i % 8)
        f.write(bytes([nbytes]) + bytes(bits))
        f.write(bytes([(flags & 7) | (8 if vc is not None else 0)]))
        if vc is not None:
            f.write(struct.pack(">BBHHHHf", vc["nl"], vc["n_heads"], vc["mlp_dim"], vc["dim"],
                                vc["img_px"], vc["psize"], vc["eps"]))
        vocab = SPECIALS + [f"t{i}" for i in range(len(SPECIALS), nvocab)]
        if vc is not None:
            vocab.append("<image_soft_token>")
        f.write(b"".join(_pascal(s) for s in vocab))
        f.write(struct.pack(">I", 1) + _pascal("t") + _pascal("0"))

        def norm(n: int) -> bytes:
            if norm_std <= 0.0:
                return np.zeros(n, np.float32).tobytes()
            return (rng.standard_normal(n, dtype=np.float32) * np.float32(norm_std)).tobytes()

        linear(f, rng, nvocab, dim)  # emb, also the tied LM head
        for _ in range(nl):
            linear(f, rng, q_sz, dim)    # wq
            linear(f, rng, kv_sz, dim)   # wk
            linear(f, rng, kv_sz, dim)   # wv
            linear(f, rng, dim, q_sz)    # wo
            if flags & 4:
                f.write(norm(hdim) + norm(hdim))  # nq, nk
            linear(f, rng, mlp, dim)     # w1 (up)
            linear(f, rng, mlp, dim)     # w2 (gate)
            linear(f, rng, dim, mlp)     # w3 (down)
            for _ in range(2 + ((flags & 2) != 0) + ((flags & 1) != 0)):
                f.write(norm(dim))               # n1 n2 [n3] [n4]
        f.write(norm(dim))                       # fnorm
        if vision is not None:
            _write_vision(f, vision)
    os.replace(tmp, path)
    return path


def _write_vision(f, v: dict) -> None:
    """The VisionEncoder's tensors in read_vision_encoder's order (gemma.c:
    1688-1762): pe, pe_b, pos_emb, per layer n1 n1_b wq wk wv wo bq bk bv bo n2
    n2_b w1 w2 b1 b2, then post_n post_nb norm proj; int8 tensors as int8 rows
    then their fp32 row scales."""
    def t(a):
        f.write(np.ascontiguousarray(a, np.float32).tobytes())

    def q(w):
        if isinstance(w, np.ndarray):  # 'U': fp32 [rows][cols]
            t(w)
            return
        f.write(np.ascontiguousarray(w[0], np.int8).tobytes())
        t(w[1])

    t(v["pe"])
    t(v["pe_b"])
    q(v["pos"])
    for ly in v["layers"]:
        t(ly["n1"]); t(ly["n1_b"])
        for w in ("wq", "wk", "wv", "wo"):
            q(ly[w])
        for b in ("bq", "bk", "bv", "bo", "n2", "n2_b"):
            t(ly[b])
        q(ly["w1"]); q(ly["w2"]); t(ly["b1"]); t(ly["b2"])
    t(v["post_n"]); t(v["post_nb"]); t(v["norm"])
    q(v["proj"])


def read_bin(path: str) -> dict:
    """Map an f32 .bin (text decoder) into numpy views, as the reference's
    mmap loader does (gemma.c:1942-2055, tensor order 1386-1469).  Returns
    {"config": {...}, "emb": (q, s), "layers": [{"wq": (q, s), ..., "n1": ...}],
    "fnorm": ...}; tensors are read-only views of the file.  In an fp32 ('U')
    file (config["quant"] False) each linear layer is one fp32 [out][in]
    array instead of the (int8, scales) pair."""
    data = np.memmap(path, dtype=np.uint8, mode="r")
    if bytes(data[:4]) != b"GEMA" or bytes(data[4:7]) != b"f32":
        raise ValueError(f"{path}: not an f32 Gemma.c model")
    if bytes(data[7:8]) not in (b"Q", b"U"):
        raise ValueError(f"{path}: neither a W8A8 ('Q') nor an fp32 ('U') model")
    quant = bytes(data[7:8]) == b"Q"
    at = 8
    (nl, n_heads, nkv, hdim, dim, mlp, q_scale, slide, img_tok, max_seq, nvocab, theta_l,
     theta_g, eps, sc_att, sc_log) = struct.unpack(">BBBHHHHHHIIfffff", bytes(data[at:at + 43]))
    at += 43
    nbytes = int(data[at])
    bits = bytes(data[at + 1:at + 1 + nbytes])
    at += 1 + nbytes
    swa = [(bits[i // 8] >> (7 - i % 8)) & 1 for i in range(nl)]
    flags = int(data[at])
    at += 1
    multimodal = bool(flags & 8)
    vcfg = None
    if multimodal:  # vision config (gemma.c:723-733)
        vnl, vheads, vmlp, vdim, img_px, psize, veps = struct.unpack(
            ">BBHHHHf", bytes(data[at:at + 14]))
        vcfg = dict(nl=vnl, n_heads=vheads, img_px=img_px, psize=psize, dim=vdim,
                    mlp_dim=vmlp, img_tok=img_tok, eps=veps)
        at += 14
    for _ in range(nvocab + (1 if multimodal else 0)):
        at += 1 + int(data[at])
    (nmerges,) = struct.unpack(">I", bytes(data[at:at + 4]))
    at += 4
    for _ in range(2 * nmerges):
        at += 1 + int(data[at])

    def f32(n):
        nonlocal at
        v = np.frombuffer(data, np.float32, n, at)
        at += 4 * n
        return v

    def qt(rows, cols):
        nonlocal at
        if not quant:  # 'U': fp32 [rows][cols]
            return f32(rows * cols).reshape(rows, cols)
        q = np.frombuffer(data, np.int8, rows * cols, at).reshape(rows, cols)
        at += rows * cols
        return q, f32(rows)

    cfg = dict(nl=nl, n_heads=n_heads, nkv=nkv, hdim=hdim, dim=dim, mlp_dim=mlp,
               q_scale=q_scale, slide=slide, nvocab=nvocab, theta_l=theta_l, theta_g=theta_g,
               eps=eps, sc_att=sc_att, sc_log=sc_log, qk_norm=bool(flags & 4),
               mlp_pre=bool(flags & 2), mlp_pst=bool(flags & 1), swa=swa, max_seq=max_seq,
               quant=quant)
    q_sz, kv_sz = n_heads * hdim, nkv * hdim
    emb = qt(nvocab, dim)
    layers = []
    for _ in range(nl):
        ly = {"wq": qt(q_sz, dim), "wk": qt(kv_sz, dim), "wv": qt(kv_sz, dim),
              "wo": qt(dim, q_sz)}
        ly["nq"], ly["nk"] = (f32(hdim), f32(hdim)) if cfg["qk_norm"] else (None, None)
        ly["w1"], ly["w2"], ly["w3"] = qt(mlp, dim), qt(mlp, dim), qt(dim, mlp)
        ly["n1"], ly["n2"] = f32(dim), f32(dim)
        ly["n3"] = f32(dim) if cfg["mlp_pre"] else None
        ly["n4"] = f32(dim) if cfg["mlp_pst"] else None
        layers.append(ly)
    fnorm = f32(dim)
    out = {"config": cfg, "emb": emb, "layers": layers, "fnorm": fnorm}
    if vcfg is not None:
        vd, vm, p = vcfg["dim"], vcfg["mlp_dim"], vcfg["psize"]
        npatch = (vcfg["img_px"] // p) ** 2
        vis = {"config": dict(vcfg, text_dim=dim, quant=quant)}
        vis["pe"] = f32(vd * 3 * p * p).reshape(vd, 3 * p * p)
        vis["pe_b"] = f32(vd)
        vis["pos"] = qt(npatch, vd)
        vis["layers"] = []
        for _ in range(vcfg["nl"]):
            ly = {"n1": f32(vd), "n1_b": f32(vd)}
            for w in ("wq", "wk", "wv", "wo"):
                ly[w] = qt(vd, vd)
            for b in ("bq", "bk", "bv", "bo", "n2", "n2_b"):
                ly[b] = f32(vd)
            ly["w1"], ly["w2"] = qt(vm, vd), qt(vd, vm)
            ly["b1"], ly["b2"] = f32(vm), f32(vd)
            vis["layers"].append(ly)
        vis["post_n"], vis["post_nb"], vis["norm"] = f32(vd), f32(vd), f32(vd)
        vis["proj"] = qt(dim, vd)
        out["vision"] = vis
    out["end"] = at
    return out


def synth_model(name: str, seed: int = 1234, nvocab: int = NVOCAB, quant: bool = True) -> dict:
    """A random W8A8 model of shape `name` in memory, in read_bin()'s layout,
    for throughput runs where writing a multi-GB file would dominate: int8
    weights are tiles of one 64 MB random block (each tensor starting at its
    own offset), row scales U(4e-4, 8e-4) (the scale of N(0, 0.02) weights
    quantized per row), norm weights 0.  quant=False: an fp32 ('U') model,
    weights tiles of one 64 MB block of N(0, 0.02) floats."""
    c = CONFIGS[name]
    nl, dim, hdim, mlp = c["nl"], c["dim"], c["hdim"], c["mlp"]
    q_sz, kv_sz = c["n_heads"] * hdim, c["nkv"] * hdim
    rng = np.random.default_rng(seed)
    if quant:
        block = np.frombuffer(rng.bytes(64 << 20), np.int8)
        block = np.where(block == -128, np.int8(127), block).astype(np.int8)
    else:
        block = (rng.standard_normal(16 << 20) * 0.02).astype(np.float32)
    twice = np.concatenate([block, block])

    def qt(rows, cols):
        n = rows * cols
        q = np.empty(n, block.dtype)
        start, done = int(rng.integers(0, len(block))), 0
        while done < n:
            take = min(n - done, len(block))
            q[done:done + take] = twice[start:start + take]
            done += take
        if not quant:
            return q.reshape(rows, cols)
        return q.reshape(rows, cols), rng.uniform(4e-4, 8e-4, rows).astype(np.float32)

    zeros = lambda n: np.zeros(n, np.float32)  # noqa: E731
    cfg = dict(nl=nl, n_heads=c["n_heads"], nkv=c["nkv"], hdim=hdim, dim=dim, mlp_dim=mlp,
               q_scale=hdim, slide=c["slide"], nvocab=nvocab, theta_l=10000.0,
               theta_g=1000000.0, eps=float(np.float32(1e-6)), sc_att=0.0, sc_log=0.0,
               qk_norm=True, mlp_pre=True, mlp_pst=True,
               swa=[int((i + 1) % 6 != 0) for i in range(nl)], max_seq=32768, quant=quant)
    layers = [{"wq": qt(q_sz, dim), "wk": qt(kv_sz, dim), "wv": qt(kv_sz, dim),
               "wo": qt(dim, q_sz), "nq": zeros(hdim), "nk": zeros(hdim),
               "w1": qt(mlp, dim), "w2": qt(mlp, dim), "w3": qt(dim, mlp),
               "n1": zeros(dim), "n2": zeros(dim), "n3": zeros(dim), "n4": zeros(dim)}
              for _ in range(nl)]
    return {"config": cfg, "emb": qt(nvocab, dim), "layers": layers, "fnorm": zeros(dim)}


# SigLIP (the Gemma 3 vision tower): VisionConfig
# (gemma.c:713-721) plus the pooled token count TextConfig carries
VISION_CONFIGS = {
    "siglip": dict(nl=27, n_heads=16, img_px=896, psize=14, dim=1152, mlp_dim=4304, img_tok=256),
}


def synth_vision(seed: int = 1234, text_dim: int = 2560, eps: float = 1e-6, quant: bool = True,
                 **shape) -> dict:
    """Random W8A8 VisionEncoder weights (gemma.c:1565-1585) in memory: int8
    tensors uniform in [-127, 127] with row scales U(4e-4, 8e-4), the fp32
    patch embedding and biases N(0, 0.02), layer-norm weights N(1, 0.05) and
    biases N(0, 0.05), the soft-embedding RMSNorm weight N(0, 0.1) (applied as
    w + 1).  quant=False: an fp32 ('U') tower, the projections, position
    embedding and output projection N(0, 0.02) fp32.  `shape` overrides
    VISION_CONFIGS["siglip"]'s fields."""
    c = dict(VISION_CONFIGS["siglip"], **shape)
    rng = np.random.default_rng(seed)
    dim, mlp, p = c["dim"], c["mlp_dim"], c["psize"]
    npatch = (c["img_px"] // p) ** 2

    def qt(rows, cols):
        if not quant:
            return (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
        q = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
        return q, rng.uniform(4e-4, 8e-4, rows).astype(np.float32)

    def nrm(n, mean, std):
        return (mean + std * rng.standard_normal(n)).astype(np.float32)

    layers = [{"wq": qt(dim, dim), "wk": qt(dim, dim), "wv": qt(dim, dim), "wo": qt(dim, dim),
               "w1": qt(mlp, dim), "w2": qt(dim, mlp),
               "bq": nrm(dim, 0, 0.02), "bk": nrm(dim, 0, 0.02), "bv": nrm(dim, 0, 0.02),
               "bo": nrm(dim, 0, 0.02), "b1": nrm(mlp, 0, 0.02), "b2": nrm(dim, 0, 0.02),
               "n1": nrm(dim, 1, 0.05), "n1_b": nrm(dim, 0, 0.05),
               "n2": nrm(dim, 1, 0.05), "n2_b": nrm(dim, 0, 0.05)}
              for _ in range(c["nl"])]
    cfg = dict(c, eps=float(np.float32(eps)), text_dim=text_dim, quant=quant)
    return {"config": cfg, "pe": nrm(dim * 3 * p * p, 0, 0.02).reshape(dim, 3 * p * p),
            "pe_b": nrm(dim, 0, 0.02), "pos": qt(npatch, dim), "layers": layers,
            "post_n": nrm(dim, 1, 0.05), "post_nb": nrm(dim, 0, 0.05), "norm": nrm(dim, 0, 0.1),
            "proj": qt(text_dim, dim)}


def synth_image(img_px: int, seed: int = 1234) -> np.ndarray:
    """An image ~U(0, 255) per channel, normalized as gemma.c:4271-4273
    ((p / 255 - 0.5) / 0.5), HWC float32."""
    rng = np.random.default_rng(seed)
    pix = rng.integers(0, 256, (img_px, img_px, 3)).astype(np.float32)
    return ((pix / np.float32(255.0) - np.float32(0.5)) / np.float32(0.5)).astype(np.float32)


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
