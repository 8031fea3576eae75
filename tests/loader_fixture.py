"""Synthetic int4-mode weights for the loader tests: a layout manifest (load_int4's line format,
qwen_infer.c:551-553) over a blob built from the oracle's packers."""
import os

import numpy as np

from golden.fixtures import seeded_normal


def _align(buf, a=64):
    pad = (-len(buf)) % a
    buf.extend(b"\0" * pad)
    return len(buf)


def build(oracle, d, tensors=None):
    """Writes d/layout_int4.txt and d/weights.bin; returns (layout, blob, refs) where refs[name] holds
    the reference-layout arrays (kind, packed, scales, sub) or the f32 values."""
    tensors = tensors or [("q.proj", "q4g64", 200, 512), ("k.proj", "q8g64", 136, 256), ("mlp.down", "q4g256sf", 96, 1024),
                          ("norm", "f32", 512, 0), ("emb", "f32", 8, 16)]
    blob = bytearray()
    lines, refs = [], {}
    for i, (name, kind, out, inn) in enumerate(tensors):
        if kind == "f32":
            v = seeded_normal(900 + i, (out * max(inn, 1),))
            doff = _align(blob)
            blob.extend(v.tobytes())
            lines.append(f"{name} f32 {doff} {out} {inn} 0 0")
            refs[name] = ("f32", v)
            continue
        w = seeded_normal(900 + i, (out, inn), 0.02)
        if kind == "q4g64":
            pk, sc = oracle.quantize_q4g64(w)
            sub = None
        elif kind == "q8g64":
            pk, sc = oracle.quantize_q8g64(w)
            sub = None
        else:
            pk, sc, sub = oracle.quantize_g256sf(w)
        doff = _align(blob); blob.extend(pk.tobytes())
        soff = _align(blob); blob.extend(sc.tobytes())
        ng = inn // (256 if kind == "q4g256sf" else 64)
        line = f"{name} {kind} {doff} {out} {inn} {ng} {soff}"
        if sub is not None:
            soff2 = _align(blob); blob.extend(sub.tobytes())
            line += f" {soff2}"
        lines.append(line)
        refs[name] = (kind, pk, sc, sub)
    _align(blob)
    layout, path = os.path.join(d, "layout_int4.txt"), os.path.join(d, "weights.bin")
    with open(layout, "w") as f:
        f.write("\n".join(lines) + "\n")
    with open(path, "wb") as f:
        f.write(bytes(blob))
    return layout, path, refs


def build_af(d, tensors=None, seed=7):
    """Writes d/layout_af.txt (moe_load_layout_af's record format, qwen_infer.c:2496-2515) over an AF
    blob of int4 affine tensors: per tensor E x [out][in/2] code bytes, fp32 scales and biases
    [E][out][in/64], each at a 64-byte aligned offset.  Returns (layout, blob uint8 array, records),
    records[name] = (E, out, in, codes, scales, biases)."""
    tensors = tensors or [("layers.0.mlp.experts.gate", 4, 64, 128), ("layers.0.mlp.experts.up", 4, 64, 128),
                          ("layers.0.mlp.experts.down", 4, 128, 64), ("lm_head", 1, 96, 128)]
    rng = np.random.default_rng(seed)
    blob = bytearray()
    lines, recs = [], {}
    for name, E, out, inn in tensors:
        ng = inn // 64
        codes = rng.integers(0, 256, (E, out, inn // 2), dtype=np.uint8)
        sc = (rng.random((E, out, ng), dtype=np.float32) * np.float32(0.01)).astype(np.float32)
        bi = (rng.standard_normal((E, out, ng), dtype=np.float32) * np.float32(0.04)).astype(np.float32)
        po = _align(blob); blob.extend(codes.tobytes())
        so = _align(blob); blob.extend(sc.tobytes())
        bo = _align(blob); blob.extend(bi.tobytes())
        lines.append(f"{name} {E} {out} {inn} {ng} {po} {codes.nbytes} {so} {bo}")
        recs[name] = (E, out, inn, codes, sc, bi)
    _align(blob)
    layout = os.path.join(d, "layout_af.txt")
    with open(layout, "w") as f:
        f.write("\n".join(lines) + "\n")
    return layout, np.frombuffer(bytes(blob), np.uint8), recs
