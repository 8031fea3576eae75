"""beglin_amd -- MI355X (gfx950) backend for beglin's quantized GEMV / MoE-gather hot path.

The product is the C-ABI library libbeglin_hip.so (include/beglin_qgemv.h).  This package is a
thin Python veneer over it for tests and benchmarks: PyTorch only supplies device memory and the
stream.  Every call goes through the HIP library; if it is not built, importing `Context` fails.
"""
import ctypes as C

from . import capi
from .capi import (ACT_F32, ACT_W4A8, K_F16, K_F32, K_MXFP4, K_Q4G32H, K_Q4G64, K_Q4G64A,  # noqa: F401
                   K_Q4G256P, K_Q4G256SF, K_Q8G64, K_QNG64)

_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = capi.load()
    return _lib


# BGL_E_* codes of include/beglin_qgemv.h
E_ARG, E_UNSUPPORTED, E_HIP, E_NODEV, E_NOMEM, E_CAPTURE, E_TIMEOUT = -1, -2, -3, -4, -5, -6, -7


class BglError(RuntimeError):
    def __init__(self, msg, code=0):
        super().__init__(msg)
        self.code = code


def _check(rc, what):
    if rc != 0:
        raise BglError(f"{what} failed ({rc}): {lib().bgl_last_error().decode(errors='replace')}", rc)


def _p(t):
    """Device (or host numpy) pointer of a torch tensor / numpy array, None passes through."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        assert t.is_contiguous(), "tensor must be contiguous"
        return C.c_void_p(t.data_ptr())
    return C.c_void_p(t.ctypes.data)


class Tensor:
    """A weight tensor bound on the device (bgl_tensor*)."""

    def __init__(self, handle):
        self.h = C.c_void_p(handle) if not isinstance(handle, C.c_void_p) else handle

    def info(self):
        k, b, o, i = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        nb = C.c_size_t()
        _check(lib().bgl_tensor_info(self.h, C.byref(k), C.byref(b), C.byref(o), C.byref(i), C.byref(nb)), "bgl_tensor_info")
        return dict(kind=k.value, bits=b.value, out=o.value, inn=i.value, device_bytes=nb.value)

    def free(self):
        if self.h:
            lib().bgl_tensor_free(self.h)
            self.h = None


class Context:
    """One bgl_ctx on one device and one HIP stream (torch's current stream by default)."""

    def __init__(self, device=0, stream=None):
        import torch
        L = lib()
        if stream is None:
            stream = torch.cuda.current_stream(device).cuda_stream
        h = C.c_void_p()
        _check(L.bgl_ctx_create(device, C.c_void_p(stream), C.byref(h)), "bgl_ctx_create")
        self.h = h
        self.device = device

    def close(self):
        if self.h:
            lib().bgl_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self):
        _check(lib().bgl_synchronize(self.h), "bgl_synchronize")

    def check(self):
        """Synchronize, then raise if a bounded in-kernel wait gave up since the last check (bgl_ctx_check)."""
        _check(lib().bgl_ctx_check(self.h), "bgl_ctx_check")

    # ---- profiling (QWEN_PROF analogue) ----
    def prof_enable(self, on=True):
        _check(lib().bgl_prof_enable(self.h, int(on)), "bgl_prof_enable")

    def prof_read(self):
        """{phase: (ms, launches)} for phases prep/gemv/other, summed since the last read."""
        ms = (C.c_double * 3)()
        n = (C.c_int * 3)()
        _check(lib().bgl_prof_read(self.h, ms, n, 3), "bgl_prof_read")
        return {"prep": (ms[0], n[0]), "gemv": (ms[1], n[1]), "other": (ms[2], n[2])}

    # ---- binding ----
    def bind(self, kind, packed, scales, out, inn, bits=0, sub=None):
        """Bind host (numpy) buffers in the reference layout (sub: g256sf sub-codes or Q4G64A biases;
        scales None for the dense kinds and MXFP4, whose blocks carry their exponents)."""
        w = capi.bgl_wt(kind, bits if kind == K_QNG64 else (8 if kind == K_Q8G64 else 4), out, inn,
                        packed.ctypes.data, scales.ctypes.data if scales is not None else None,
                        sub.ctypes.data if sub is not None else None)
        h = C.c_void_p()
        _check(lib().bgl_bind(self.h, C.byref(w), C.byref(h)), "bgl_bind")
        return Tensor(h)

    def bind_qng64_mixed(self, planes, offsets, bits, scales, out, inn):
        """Bind a mixed per-cell qNg64 tensor (numpy planes u8, offsets u32 [cells+1], bits u8 [cells],
        scales f32 [cells])."""
        h = C.c_void_p()
        _check(lib().bgl_bind_qng64_mixed(self.h, planes.ctypes.data, planes.nbytes, offsets.ctypes.data, bits.ctypes.data,
                                          scales.ctypes.data, out, inn, C.byref(h)), "bgl_bind_qng64_mixed")
        return Tensor(h)

    def quantize(self, kind, w_dev, bits=0, qng64_encoder=1, want_ref=False):
        """Quantize fp32 weights already on the device (torch tensor [out][in]).  With want_ref the
        reference-layout bytes come back as numpy arrays."""
        import numpy as np
        out, inn = w_dev.shape
        ref = None
        args = [None, None, None]
        if want_ref:
            if kind in (K_Q4G64, K_Q4G256SF, K_Q4G32H):
                pk = np.zeros((out, inn // 2), np.uint8)
            elif kind == K_Q8G64:
                pk = np.zeros((out, inn), np.int8)
            else:
                pk = np.zeros((out, inn // 64 * bits * 8), np.uint8)
            if kind == K_Q4G32H:
                sc = np.zeros((out, inn // 32), np.uint16)
            elif kind == K_Q4G256SF:
                sc = np.zeros((out, inn // 256), np.float32)
            else:
                sc = np.zeros((out, inn // 64), np.float32)
            sub = np.zeros((out, inn // 64), np.uint8) if kind == K_Q4G256SF else None
            ref = (pk, sc, sub)
            args = [_p(pk), _p(sc), _p(sub)]
        h = C.c_void_p()
        _check(lib().bgl_quantize_dev(self.h, kind, bits, int(qng64_encoder), _p(w_dev), out, inn, C.byref(h), *args),
               "bgl_quantize_dev")
        return (Tensor(h), ref) if want_ref else Tensor(h)

    def dequant(self, t, row0, nrows, out_dev):
        _check(lib().bgl_dequant_dev(self.h, t.h, row0, nrows, _p(out_dev)), "bgl_dequant_dev")

    # ---- compute (device pointers) ----
    def matmul(self, t, x_dev, y_dev, act=ACT_F32, bias_dev=None):
        M = 1 if x_dev.dim() == 1 else x_dev.shape[0]
        _check(lib().bgl_matmul_dev(self.h, t.h, act, _p(x_dev), _p(bias_dev), _p(y_dev), M), "bgl_matmul_dev")

    def matmul_group(self, ts, x_dev, ys, act=ACT_F32, biases=None):
        n = len(ts)
        M = 1 if x_dev.dim() == 1 else x_dev.shape[0]
        W = (C.c_void_p * n)(*[t.h.value for t in ts])
        Y = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
        B = (C.c_void_p * n)(*[(b.data_ptr() if b is not None else None) for b in (biases or [None] * n)])
        _check(lib().bgl_matmul_group_dev(self.h, n, W, act, _p(x_dev), B, Y, M), "bgl_matmul_group_dev")

    def mlp(self, gate, up, down, x_dev, y_dev, act=ACT_F32, h_dev=None):
        """y = W_down (silu(W_gate x) * (W_up x)) on the device (bgl_mlp_dev); h_dev receives h."""
        M = 1 if x_dev.dim() == 1 else x_dev.shape[0]
        _check(lib().bgl_mlp_dev(self.h, gate.h, up.h, down.h, act, _p(x_dev), _p(y_dev), M, _p(h_dev)), "bgl_mlp_dev")

    def read_probe(self, ts, nblocks=0, nthreads=0):
        """Plain streaming read of the tensors' device bytes (the memory floor for a call)."""
        W = (C.c_void_p * len(ts))(*[t.h.value for t in ts])
        _check(lib().bgl_read_probe_dev(self.h, len(ts), W, nblocks, nthreads), "bgl_read_probe_dev")

    def prep_only(self, x_dev, act, t):
        """Prepare activation operands for tensor t's kind (kept in the context)."""
        M = 1 if x_dev.dim() == 1 else x_dev.shape[0]
        _check(lib().bgl_prep_act_dev(self.h, act, t.info()["kind"], _p(x_dev), M, x_dev.shape[-1]), "bgl_prep_act_dev")

    def matmul_prepped(self, t, y_dev, act=ACT_F32, bias_dev=None, M=1):
        _check(lib().bgl_matmul_prepped_dev(self.h, t.h, act, _p(bias_dev), _p(y_dev), M), "bgl_matmul_prepped_dev")

    def quant_act_i8(self, x_dev, gsize, xq_dev, ascale_dev):
        M = 1 if x_dev.dim() == 1 else x_dev.shape[0]
        _check(lib().bgl_quant_act_i8_dev(self.h, _p(x_dev), M, x_dev.shape[-1], gsize, _p(xq_dev), _p(ascale_dev)),
               "bgl_quant_act_i8_dev")

    # ---- MoE ----
    def bind_experts(self, descs):
        """descs: list of (kind, bits, packed, scales[, bias]) numpy tuples, one per expert; packed is
        2-D [out][row bytes or elements]; scales None for the dense kinds."""
        E = len(descs)
        arr = (capi.bgl_wt * E)()
        for e, d in enumerate(descs):
            kind, bits, pk, sc = d[:4]
            bi = d[4] if len(d) > 4 else None
            out = pk.shape[0]
            if kind in (K_F16, K_F32):
                inn = pk.shape[1]
            elif kind == K_MXFP4:                # GGUF blocks of 32 values, 17 bytes each
                inn = pk.reshape(out, -1).shape[1] // 17 * 32
            else:
                inn = sc.shape[1] * (32 if kind == K_Q4G32H else 64)
            b = bits if kind == K_QNG64 else (8 if kind == K_Q8G64 else 4)
            arr[e] = capi.bgl_wt(kind, b, out, inn, pk.ctypes.data, sc.ctypes.data if sc is not None else None,
                                 bi.ctypes.data if bi is not None else None)
        h = C.c_void_p()
        _check(lib().bgl_bind_experts(self.h, E, arr, C.byref(h)), "bgl_bind_experts")
        return Tensor(h)

    def experts_from_tensors(self, tensors):
        """Stack bound single tensors (e.g. from quantize()) into one expert tensor.  The new
        tensor owns them: their handles are cleared here and freed with the stack."""
        E = len(tensors)
        arr = (C.c_void_p * E)(*[t.h.value for t in tensors])
        h = C.c_void_p()
        _check(lib().bgl_experts_from_tensors(self.h, E, arr, C.byref(h)), "bgl_experts_from_tensors")
        for t in tensors:
            t.h = None
        return Tensor(h)

    def gather_matvec(self, experts, x_dev, idx_dev, y_dev):
        _check(lib().bgl_gather_matvec_dev(self.h, experts.h, _p(x_dev), _p(idx_dev), x_dev.shape[0], _p(y_dev)),
               "bgl_gather_matvec_dev")

    def moe_ffn(self, gate, up, down, shared, x_dev, idx_dev, w_dev, out_dev):
        sg, su, sd = (shared or (None, None, None))
        T, K = idx_dev.shape
        _check(lib().bgl_moe_ffn_dev(self.h, gate.h, up.h, down.h, sg.h if sg else None, su.h if su else None,
                                     sd.h if sd else None, _p(x_dev), _p(idx_dev), _p(w_dev), T, K, _p(out_dev)),
               "bgl_moe_ffn_dev")

    def moe_route(self, router_w, x_dev, K, idx_dev, w_dev, router_b=None, renorm=False):
        E, inn = router_w.shape
        _check(lib().bgl_moe_route_dev(self.h, _p(router_w), _p(router_b) if router_b is not None else None, E, inn, _p(x_dev),
                                       x_dev.shape[0], K, 1 if renorm else 0, _p(idx_dev), _p(w_dev)), "bgl_moe_route_dev")

    def moe_layer(self, router_w, gate, up, down, shared, x_dev, K, out_dev, router_b=None, renorm=False):
        sg, su, sd = (shared or (None, None, None))
        _check(lib().bgl_moe_layer_dev(self.h, _p(router_w), _p(router_b) if router_b is not None else None, 1 if renorm else 0,
                                       gate.h, up.h, down.h, sg.h if sg else None, su.h if su else None, sd.h if sd else None,
                                       _p(x_dev), x_dev.shape[0], K, _p(out_dev)), "bgl_moe_layer_dev")


class Model:
    """Weights loaded from the int4 layout manifest + blob (bgl_model_load_int4) or from the
    repacked-layout cache (bgl_model_load_cache)."""

    def __init__(self, ctx, layout, blob, cache=None):
        self.ctx, self.layout, self.blob = ctx, layout, blob
        h = C.c_void_p()
        if cache is not None:
            _check(lib().bgl_model_load_cache(ctx.h, cache.encode(), layout.encode(), blob.encode(), C.byref(h)),
                   "bgl_model_load_cache")
        else:
            _check(lib().bgl_model_load_int4(ctx.h, layout.encode(), blob.encode(), C.byref(h)), "bgl_model_load_int4")
        self.h = h

    def __len__(self):
        return lib().bgl_model_count(self.h)

    def find(self, name):
        """(kind, out, in, Tensor or None, address of the f32 data or None); the model owns the tensor."""
        k, o, i = C.c_int(), C.c_int(), C.c_int()
        t, f = C.c_void_p(), C.c_void_p()
        _check(lib().bgl_model_find(self.h, name.encode(), C.byref(k), C.byref(o), C.byref(i), C.byref(t), C.byref(f)),
               "bgl_model_find")
        return k.value, o.value, i.value, (Tensor(t) if t.value else None), f.value

    def save_cache(self, path):
        _check(lib().bgl_model_save_cache(self.h, path.encode(), self.layout.encode(), self.blob.encode()), "bgl_model_save_cache")

    def close(self):
        if self.h:
            lib().bgl_model_free(self.h)
            self.h = None


def layout_check(layout, blob):
    n = C.c_int()
    rc = lib().bgl_int4_layout_check(layout.encode(), blob.encode(), C.byref(n))
    return rc, n.value


def af_layout_check(layout, blob_bytes):
    n = C.c_int()
    rc = lib().bgl_af_layout_check(layout.encode(), blob_bytes, C.byref(n))
    return rc, n.value


def cache_valid(cache, layout, blob):
    return lib().bgl_model_cache_valid(cache.encode(), layout.encode(), blob.encode())


# ---- the name-keyed registry (mlx_moe.h boundary): thin wrappers, 1 = ok / 0 = failure ----
class Registry:
    """bgl_gpu_* entry points with numpy host buffers."""

    @staticmethod
    def L():
        return lib()

    def available(self):
        return lib().bgl_gpu_available()

    def bind_af(self, blob, name, E, out, inn, ng, packed_off, scale_off, bias_off, bits):
        return lib().bgl_gpu_bind_af(blob.ctypes.data, blob.nbytes, name.encode(), E, out, inn, ng, packed_off,
                                     scale_off, bias_off, bits)

    def load_layout_af(self, layout, blob):
        """Binds every tensor of an AF layout manifest over blob (uint8 array); the count or -1."""
        return lib().bgl_gpu_load_layout_af(layout.encode(), blob.ctypes.data, blob.nbytes)

    def binding_kind(self, name):
        b = C.c_int()
        k = lib().bgl_gpu_binding_kind(name.encode(), C.byref(b))
        return k, b.value

    def snapshot(self, name):
        sid = C.c_uint64()
        ok = lib().bgl_gpu_snapshot_binding(name.encode(), C.byref(sid))
        return ok, sid.value

    def dequant_probe(self, name, e, row, col0, ncols):
        import numpy as np
        out = np.zeros(ncols, np.float32)
        ok = lib().bgl_gpu_dequant_probe(name.encode(), e, row, col0, ncols, out.ctypes.data)
        return ok, out

    def matvec_probe(self, name, e, x, out):
        import numpy as np
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(out, np.float32)
        ok = lib().bgl_gpu_matvec_probe(name.encode(), e, x.ctypes.data, y.ctypes.data)
        return ok, y

    def ffn_gather(self, name, x, idx, out):
        import numpy as np
        x = np.ascontiguousarray(x, np.float32)
        idx = np.ascontiguousarray(idx, np.int32)
        y = np.zeros((x.shape[0], out), np.float32)
        ok = lib().bgl_gpu_ffn_gather(name.encode(), x.ctypes.data, x.shape[0], idx.ctypes.data, y.ctypes.data)
        return ok, y

    def bind_mixed(self, name, planes, offsets, bits, scales, out, inn):
        return lib().bgl_gpu_bind_qng64_mixed_dense_probe(planes.ctypes.data, planes.nbytes, offsets.ctypes.data,
                                                          bits.ctypes.data, scales.ctypes.data, name.encode(), out, inn)

    def mixed_probe(self, planes, offsets, bits, scales, out, inn, x):
        import numpy as np
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros((x.shape[0], out), np.float32)
        ok = lib().bgl_gpu_qng64_mixed_dense_probe(planes.ctypes.data, planes.nbytes, offsets.ctypes.data, bits.ctypes.data,
                                                   scales.ctypes.data, out, inn, x.ctypes.data, x.shape[0], y.ctypes.data)
        return ok, y

    def bind_router(self, name, w, bias=None):
        import numpy as np
        w = np.ascontiguousarray(w, np.float32)
        b = np.ascontiguousarray(bias, np.float32) if bias is not None else None
        return lib().bgl_gpu_bind_router(name.encode(), w.ctypes.data, b.ctypes.data if b is not None else None,
                                         w.shape[0], w.shape[1])

    def moe_layer(self, router, gate, up, down, shared, x, K, renorm=False):
        import numpy as np
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        idx = np.zeros((x.shape[0], K), np.int32)
        w = np.zeros((x.shape[0], K), np.float32)
        sg, su, sd = [s.encode() if s else None for s in (shared or (None, None, None))]
        ok = lib().bgl_gpu_moe_layer(router.encode(), gate.encode(), up.encode(), down.encode(), sg, su, sd, x.ctypes.data,
                                     x.shape[0], K, 1 if renorm else 0, out.ctypes.data, idx.ctypes.data, w.ctypes.data)
        return ok, out, idx, w

    def moe_ffn(self, gate, up, down, shared, x, idx, w):
        import numpy as np
        x = np.ascontiguousarray(x, np.float32)
        idx = np.ascontiguousarray(idx, np.int32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.zeros_like(x)
        sg, su, sd = [s.encode() if s else None for s in (shared or (None, None, None))]
        ok = lib().bgl_gpu_moe_ffn(gate.encode(), up.encode(), down.encode(), sg, su, sd, x.ctypes.data, x.shape[0],
                                   idx.ctypes.data, w.ctypes.data, idx.shape[1], out.ctypes.data)
        return ok, out
