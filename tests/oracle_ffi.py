"""ctypes bindings for the CPU oracle (oracle/liboracle.so) and the reference build
(oracle/_ref/libbeglin_ref.so).  Test infrastructure: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg use this module."""
import concurrent.futures
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libbeglin_ref.so")

_P = C.c_void_p


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data_as(_P)


def load_oracle():
    if not os.path.exists(ORACLE_SO):
        raise FileNotFoundError(f"{ORACLE_SO} missing: run `make -C oracle` (or __graft_entry__.build())")
    lib = C.CDLL(ORACLE_SO)
    lib.or_f32_to_f16.restype = C.c_uint16
    lib.or_f32_to_f16.argtypes = [C.c_float]
    lib.or_f16_to_f32.restype = C.c_float
    lib.or_f16_to_f32.argtypes = [C.c_uint16]
    lib.or_quantize_qng64_dense.restype = C.c_int
    lib.or_moe_row.restype = C.c_double
    lib.or_moe_decode.restype = C.c_float
    lib.or_qng64_decode_code.restype = C.c_float
    lib.or_qng64_decode_code.argtypes = [_P, C.c_int, C.c_int]
    lib.or_pool_create.restype = _P
    lib.or_pool_create.argtypes = [C.c_int, C.c_int]
    lib.or_pool_destroy.argtypes = [_P]
    lib.or_pool_threads.argtypes = [_P]
    lib.or_pool_gemv_g256sf_sdot.argtypes = [_P] * 7 + [C.c_int, C.c_int]
    lib.or_pool_gemv_q4g64_sdot.argtypes = [_P] * 6 + [C.c_int, C.c_int]
    lib.or_pool_gemv_f32.argtypes = [_P, C.c_int, C.c_int] + [_P] * 5 + [C.c_int, C.c_int]
    return lib


def load_ref():
    """The reference's own C sources for this path, compiled in place by oracle/Makefile.
    Returns None where it was not built (e.g. a box without the reference tree and no
    prebuilt copy)."""
    if not os.path.exists(REF_SO):
        return None
    lib = C.CDLL(REF_SO)
    lib.qng64_group_bytes.restype = C.c_size_t
    lib.qng64_group_bytes.argtypes = [C.c_int]
    lib.qng64_packed_bytes.restype = C.c_size_t
    lib.qng64_packed_bytes.argtypes = [C.c_int, C.c_int, C.c_int]
    lib.qng64_quantize_f32.restype = C.c_int
    lib.qng64_quantize_f32.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P]
    lib.qng64_decode_code.restype = C.c_float
    lib.qng64_decode_code.argtypes = [_P, C.c_int, C.c_int]
    lib.qng64_matvec_f32.argtypes = [_P, _P, C.c_int, _P, _P, _P, C.c_int, C.c_int]
    lib.qng64_matmul_f32.argtypes = [_P, _P, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int]
    lib.gguf_quantize_q4g64_error_feedback.argtypes = [_P, C.c_int, C.c_int, _P, _P]
    lib.gguf_quantize_q8g64.argtypes = [_P, C.c_int, C.c_int, _P, _P]
    lib.gguf_quantize_qNg64.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P]
    lib.gguf_w_quantize_q4_0.argtypes = [_P, C.c_int64, _P]
    lib.gguf_dequant_row.argtypes = [C.c_int, _P, _P, C.c_int64]
    return lib


class Oracle:
    """numpy-facing wrappers over liboracle.so."""

    def __init__(self):
        self.lib = load_oracle()

    # ---- the dense MLP's SwiGLU (or_swiglu) ----
    def swiglu(self, g, u):
        g = np.ascontiguousarray(g, np.float32); u = np.ascontiguousarray(u, np.float32)
        h = np.zeros_like(g)
        self.lib.or_swiglu(_ptr(g), _ptr(u), _ptr(h), g.size)
        return h

    # ---- fp16 ----
    def f32_to_f16(self, f):
        return self.lib.or_f32_to_f16(C.c_float(f))

    # ---- packers (weights w: float32 [out][in]) ----
    def quantize_q4g64(self, w):
        out, inn = w.shape
        packed = np.zeros((out, inn // 2), np.uint8)
        scales = np.zeros((out, inn // 64), np.float32)
        self.lib.or_quantize_q4g64_ef(_ptr(w), out, inn, _ptr(packed), _ptr(scales))
        return packed, scales

    def quantize_q8g64(self, w):
        out, inn = w.shape
        codes = np.zeros((out, inn), np.int8)
        scales = np.zeros((out, inn // 64), np.float32)
        self.lib.or_quantize_q8g64(_ptr(w), out, inn, _ptr(codes), _ptr(scales))
        return codes, scales

    def quantize_qng64_gguf(self, w, n):
        out, inn = w.shape
        planes = np.zeros((out, inn // 64 * n * 8), np.uint8)
        scales = np.zeros((out, inn // 64), np.float32)
        self.lib.or_quantize_qng64_gguf(_ptr(w), out, inn, n, _ptr(planes), _ptr(scales))
        return planes, scales

    def quantize_qng64_dense(self, w, n):
        out, inn = w.shape
        planes = np.zeros((out, inn // 64 * n * 8), np.uint8)
        scales = np.zeros((out, inn // 64), np.float32)
        rc = self.lib.or_quantize_qng64_dense(_ptr(w), out, inn, n, _ptr(planes), _ptr(scales))
        if rc != 0:
            raise ValueError(f"qng64_quantize_f32 rejects n={n}")
        return planes, scales

    def quantize_qng64(self, w, n):
        """The config's 'reference qng64 encoder' (qng64_quantize_f32); n=4, which it rejects,
        goes through gguf_quantize_qNg64 (no n gate)."""
        return self.quantize_qng64_gguf(w, 4) if n == 4 else self.quantize_qng64_dense(w, n)

    def quantize_q4_0(self, w):
        n = w.size
        blocks = np.zeros(n // 32 * 18, np.uint8)
        self.lib.or_quantize_q4_0(_ptr(np.ascontiguousarray(w, np.float32)), C.c_int64(n), _ptr(blocks))
        return blocks

    def quantize_q4g32h(self, w):
        out, inn = w.shape
        packed = np.zeros((out, inn // 2), np.uint8)
        s16 = np.zeros((out, inn // 32), np.uint16)
        self.lib.or_quantize_q4g32h(_ptr(w), out, inn, _ptr(packed), _ptr(s16))
        return packed, s16

    def q4_0_to_q4g32h(self, blocks, out, inn):
        packed = np.zeros((out, inn // 2), np.uint8)
        s16 = np.zeros((out, inn // 32), np.uint16)
        self.lib.or_q4_0_to_q4g32h(_ptr(blocks), out, inn, _ptr(packed), _ptr(s16))
        return packed, s16

    def quantize_g256sf(self, w):
        out, inn = w.shape
        packed = np.zeros((out, inn // 2), np.uint8)
        wsuper = np.zeros((out, inn // 256), np.float32)
        sub = np.zeros((out, inn // 64), np.uint8)
        self.lib.or_quantize_g256sf(_ptr(w), out, inn, _ptr(packed), _ptr(wsuper), _ptr(sub))
        return packed, wsuper, sub

    # ---- decoders ----
    def decode(self, kind, packed, scales, out, inn, bits=0, sub=None):
        w = np.zeros((out, inn), np.float32)
        if kind == 1:
            self.lib.or_decode_q4g64(_ptr(packed), _ptr(scales), out, inn, _ptr(w))
        elif kind == 2:
            self.lib.or_decode_q8g64(_ptr(packed), _ptr(scales), out, inn, _ptr(w))
        elif kind == 3:
            self.lib.or_decode_g256sf(_ptr(packed), _ptr(scales), _ptr(sub), out, inn, _ptr(w))
        elif kind == 4:
            self.lib.or_decode_qng64(_ptr(packed), _ptr(scales), bits, out, inn, _ptr(w))
        elif kind == 5:
            self.lib.or_decode_q4g32h(_ptr(packed), _ptr(scales), out, inn, _ptr(w))
        else:
            raise ValueError(kind)
        return w

    def decode_q4_0(self, blocks, n):
        w = np.zeros(n, np.float32)
        self.lib.or_decode_q4_0(_ptr(blocks), C.c_int64(n), _ptr(w))
        return w

    # ---- GEMV ----
    def gemm_f32(self, kind, packed, scales, x, bias=None, bits=0):
        x = np.ascontiguousarray(x, np.float32)
        M = 1 if x.ndim == 1 else x.shape[0]
        inn = x.shape[-1]
        out = packed.shape[0]
        y = np.zeros((M, out), np.float32)
        self.lib.or_gemm_f32(kind, bits, _ptr(packed), _ptr(scales), _ptr(x), _ptr(bias), _ptr(y), out, inn, M)
        return y if x.ndim == 2 else y[0]

    def quant_act_i8(self, x, gsize):
        x = np.ascontiguousarray(x, np.float32)
        xq = np.zeros(x.shape, np.int8)
        a = np.zeros(x.shape[:-1] + (x.shape[-1] // gsize,), np.float32)
        rows = 1 if x.ndim == 1 else x.shape[0]
        inn = x.shape[-1]
        for m in range(rows):
            xs = x if x.ndim == 1 else x[m]
            xqs = xq if x.ndim == 1 else xq[m]
            as_ = a if x.ndim == 1 else a[m]
            self.lib.or_quant_act_i8(_ptr(xs), inn, gsize, _ptr(xqs), _ptr(as_))
        return xq, a

    def matmul_sdot(self, kind, packed, scales, x, bias=None, sub=None):
        x = np.ascontiguousarray(x, np.float32)
        M = 1 if x.ndim == 1 else x.shape[0]
        inn = x.shape[-1]
        out = packed.shape[0]
        y = np.zeros((M, out), np.float32)
        self.lib.or_matmul_sdot(kind, _ptr(packed), _ptr(scales), _ptr(sub), _ptr(x), _ptr(bias), _ptr(y), out, inn, M)
        return y if x.ndim == 2 else y[0]

    def gemm_sdot(self, kind, packed, scales, xq, ascale, bias=None, sub=None):
        M = 1 if xq.ndim == 1 else xq.shape[0]
        inn = xq.shape[-1]
        out = packed.shape[0]
        y = np.zeros((M, out), np.float32)
        if kind == 1:
            self.lib.or_gemm_q4g64_sdot(_ptr(packed), _ptr(scales), _ptr(xq), _ptr(ascale), _ptr(bias), _ptr(y), out, inn, M)
        elif kind == 2:
            self.lib.or_gemm_q8g64_sdot(_ptr(packed), _ptr(scales), _ptr(xq), _ptr(ascale), _ptr(bias), _ptr(y), out, inn, M)
        else:
            self.lib.or_gemm_g256sf_sdot(_ptr(packed), _ptr(scales), _ptr(sub), _ptr(xq), _ptr(ascale), _ptr(bias), _ptr(y), out, inn, M)
        return y if xq.ndim == 2 else y[0]

    # ---- MoE ----
    def route(self, logits, K, renorm=False):
        logits = np.ascontiguousarray(logits, np.float32)
        T, E = logits.shape
        idx = np.zeros((T, K), np.int32)
        w = np.zeros((T, K), np.float32)
        self.lib.or_moe_route(_ptr(logits), T, E, K, int(renorm), _ptr(idx), _ptr(w))
        return idx, w

    def decode_qng64_mixed(self, planes, offsets, bits, scales, out, inn):
        w = np.zeros((out, inn), np.float32)
        self.lib.or_decode_qng64_mixed(_ptr(planes), _ptr(offsets), _ptr(bits), _ptr(scales), out, inn, _ptr(w))
        return w

    def router_logits(self, w, x, bias=None):
        w = np.ascontiguousarray(w, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        E, H = w.shape
        T = x.shape[0]
        out = np.zeros((T, E), np.float32)
        self.lib.or_moe_router_logits(_ptr(w), _ptr(np.ascontiguousarray(bias, np.float32)) if bias is not None else None,
                                      _ptr(x), T, E, H, _ptr(out))
        return out


class OrExpert(C.Structure):
    _fields_ = [("kind", C.c_int), ("bits", C.c_int), ("packed", C.c_void_p), ("scales", C.c_void_p),
                ("bias", C.c_void_p)]


def expert_struct(kind, bits, packed, scales, bias=None):
    return OrExpert(kind, bits, packed.ctypes.data, scales.ctypes.data if scales is not None else None,
                    bias.ctypes.data if bias is not None else None)


def expert_array(descs):
    """descs: list of (kind, bits, packed, scales[, bias]) -> (OrExpert array, keep-alive list).
    scales may be None (dense kinds 7 / 8); bias only for kind 6 (int4 affine)."""
    arr = (OrExpert * len(descs))()
    keep = []
    for e, d in enumerate(descs):
        kind, bits, pk, sc = d[:4]
        bi = d[4] if len(d) > 4 else None
        pk = np.ascontiguousarray(pk)
        sc = np.ascontiguousarray(sc) if sc is not None else None
        bi = np.ascontiguousarray(bi) if bi is not None else None
        keep += [pk, sc, bi]
        arr[e] = expert_struct(kind, bits, pk, sc, bi)
    return arr, keep


def moe_decode(oracle, desc, out, inn, row, cols):
    """or_moe_decode (moe_decode_af) for columns `cols` of one row."""
    arr, keep = expert_array([desc])
    return np.array([oracle.lib.or_moe_decode(arr, inn, C.c_long(row), C.c_long(c)) for c in cols], np.float32)


def moe_matvec(oracle, desc, out, inn, x):
    """or_moe_matvec (qwen_infer.c:3223-3225) for one expert descriptor and one activation row."""
    arr, keep = expert_array([desc])
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(out, np.float32)
    oracle.lib.or_moe_matvec(arr, out, inn, _ptr(x), _ptr(y))
    return y


def moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w, naive=False):
    """or_moe_ffn_bucketed / or_moe_ffn_naive with routing given.  gate/up/down: per-expert
    descriptor lists; shared: (sg, su, sd) descriptors or None."""
    E = len(gate)
    ga, k1 = expert_array(gate)
    ua, k2 = expert_array(up)
    da, k3 = expert_array(down)
    if shared is not None:
        sa, k4 = expert_array(list(shared))
        sg, su, sd = C.byref(sa, 0), C.byref(sa, C.sizeof(OrExpert)), C.byref(sa, 2 * C.sizeof(OrExpert))
        Ish = shared[0][2].shape[0]
    else:
        sg = su = sd = None
        Ish = 0
    x = np.ascontiguousarray(x, np.float32)
    idx = np.ascontiguousarray(idx, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    T, K = idx.shape
    out = np.zeros((T, H), np.float32)
    fn = oracle.lib.or_moe_ffn_naive if naive else oracle.lib.or_moe_ffn_bucketed
    # Every token's output depends on its own routing only (each adds its experts' terms in expert
    # order, then the shared experts'), so token chunks run on threads (ctypes drops the GIL).
    nth = max(1, min(16, os.cpu_count() or 1, T // 4))
    bounds = [(T * i // nth, T * (i + 1) // nth) for i in range(nth)]

    def run(b):
        t0, t1 = b
        if t1 > t0:
            xs, ids, ws = x[t0:t1], idx[t0:t1], w[t0:t1]
            o = np.zeros((t1 - t0, H), np.float32)
            fn(ga, ua, da, E, sg, su, sd, H, I, Ish, t1 - t0, K, _ptr(xs), _ptr(ids), _ptr(ws), _ptr(o))
            out[t0:t1] = o

    if nth == 1:
        run((0, T))
    else:
        with concurrent.futures.ThreadPoolExecutor(nth) as ex:
            list(ex.map(run, bounds))
    return out


def mixed_qng64_random(rng, out, inn, widths):
    """A mixed per-cell qNg64 tensor (MixedQNg64Tensor layout): per (row, 64-group) cell a width
    drawn from `widths`, random plane bytes, positive scales; offsets[cells] = planes bytes."""
    ng = inn // 64
    bits = rng.choice(np.asarray(widths, np.uint8), size=out * ng).astype(np.uint8)
    offsets = np.zeros(out * ng + 1, np.uint32)
    offsets[1:] = np.cumsum(bits.astype(np.uint32) * 8)
    planes = rng.integers(0, 256, int(offsets[-1]), dtype=np.uint8)
    scales = (rng.random(out * ng, dtype=np.float32) * np.float32(0.01) + np.float32(1e-4)).astype(np.float32)
    return planes, offsets, bits, scales


def mixed_qng64_py_decode(planes, offsets, bits, scales, out, inn):
    """Independent decode of the mixed layout: numpy bit unpacking, LSB first within each byte, so
    plane j's bit p is element p's bit j."""
    ng = inn // 64
    w = np.zeros((out, inn), np.float32)
    for cell in range(out * ng):
        n, base = int(bits[cell]), int(offsets[cell])
        pl = np.unpackbits(planes[base: base + n * 8].reshape(n, 8), axis=1, bitorder="little").astype(np.int64)
        u = (pl << np.arange(n, dtype=np.int64)[:, None]).sum(axis=0)
        code = (u - (1 << (n - 1))).astype(np.float32)
        r, g = divmod(cell, ng)
        w[r, g * 64:(g + 1) * 64] = code * scales[cell]
    return w


def mxfp4_blocks(rng, out, inn, lo=116, hi=132):
    """Random GGUF MXFP4 blocks [out][inn/32][17]: exponent bytes in [lo, hi), random nibbles."""
    b = rng.integers(0, 256, (out, inn // 32, 17), dtype=np.uint8)
    b[:, :, 0] = rng.integers(lo, hi, (out, inn // 32), dtype=np.uint8)
    return b


MX_VALUES = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.float32)


def mxfp4_quant(w):
    """A GGUF MXFP4 encoding of float32 w [out][in] (in % 32 == 0): per 32-block the exponent byte b
    with max|w| <= 12 * 2^(b-128), each value the nearest of the 16 doubled E2M1 codes.  Any valid
    encoding serves the tests (parity is checked against the oracle's decode of the same blocks)."""
    out, inn = w.shape
    wb = w.reshape(out, inn // 32, 32).astype(np.float64)
    mx = np.max(np.abs(wb), axis=2)
    e = np.where(mx > 0, np.ceil(np.log2(np.maximum(mx, 1e-38) / 12.0)), -127).astype(np.int64) + 128
    b = np.clip(e, 2, 254).astype(np.uint8)
    scale = np.ldexp(1.0, b.astype(np.int64) - 128)[..., None]
    codes = np.argmin(np.abs(wb[..., None] / scale[..., None] - MX_VALUES[None, None, None, :]), axis=3).astype(np.uint8)
    blk = np.zeros((out, inn // 32, 17), np.uint8)
    blk[:, :, 0] = b
    blk[:, :, 1:] = codes[:, :, :16] | (codes[:, :, 16:] << 4)
    return blk
