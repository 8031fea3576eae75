"""Deterministic inputs that the reference's own tests use for this path, regenerated from
their published recipes (the recipes are restated here; no reference file is imported or run).

* tiny_st():   tests/regression/mk_tiny_st.py:18-44 -- three F32 [16,128] tensors
               (L0.e0.w, L0.e1.w, dense.w), random.seed(20261019), N(0, 0.05) with ~1% x8
               outliers, stored little-endian float32.
* reg_probe(): tests/regression/reg_common.h:55 -- x[c] = ((c*37)%17 - 8)/8.
* kat_qng64(): tools/qng64_dense_test.c:13-16 -- 3x64 weights ((i*37)%101-50)/23,
               x ((i*13)%31-15)/19, n=5.
* gate9():     qwen_infer.c:10811-10834 -- E=4, out=8, in=128, n=7, 6 explicit (x, expert)
               pairs with idx {0,3,1,2,0,3}; LCG seed 12345 (a=1103515245, c=12345 mod 2^32).
"""
import random

import numpy as np

TINY_OUT, TINY_IN = 16, 128


def tiny_st():
    rng = random.Random(20261019)
    out = {}
    for name in ("L0.e0.w", "L0.e1.w", "dense.w"):
        vals = []
        for _ in range(TINY_OUT * TINY_IN):
            v = rng.gauss(0.0, 0.05)
            if rng.random() < 0.01:
                v *= 8
            vals.append(v)
        out[name] = np.array(vals, dtype=np.float64).astype(np.float32).reshape(TINY_OUT, TINY_IN)
    return out


def reg_probe(n=TINY_IN):
    return np.array([((c * 37) % 17 - 8) / 8.0 for c in range(n)], dtype=np.float32)


def kat_qng64():
    out, inn = 3, 64
    src = np.array([((i * 37) % 101 - 50) / 23.0 for i in range(out * inn)], np.float32).reshape(out, inn)
    x = np.array([((i * 13) % 31 - 15) / 19.0 for i in range(inn)], np.float32)
    return src, x


def _lcg(seed):
    s = seed
    while True:
        s = (s * 1103515245 + 12345) & 0xFFFFFFFF
        yield s


def gate9():
    E, OUT, IN, N, PAIRS = 4, 8, 128, 7, 6
    idx = np.array([0, 3, 1, 2, 0, 3], np.int32)
    g = _lcg(12345)
    w = np.empty(E * OUT * IN, np.float32)
    for i in range(E * OUT * IN):
        s = next(g)
        w[i] = np.float32((np.float32(s % 20000) / np.float32(10000.0) - np.float32(1.0)) * np.float32(0.5))
    x = np.empty(PAIRS * IN, np.float32)
    for i in range(PAIRS * IN):
        s = next(g)
        x[i] = np.float32(np.float32(s % 20000) / np.float32(10000.0) - np.float32(1.0))
    return dict(E=E, out=OUT, inn=IN, n=N, idx=idx, w=w.reshape(E, OUT, IN), x=x.reshape(PAIRS, IN))


def seeded_normal(seed, shape, sigma=1.0):
    """Synthetic inputs of the BASELINE configs: N(0, sigma) from a seeded numpy Generator."""
    return (np.random.default_rng(seed).standard_normal(shape) * sigma).astype(np.float32)
