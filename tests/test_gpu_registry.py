"""GPU tests of the name-keyed MoE registry (the mlx_moe.h boundary, bgl_gpu_*) and of the
caller-quantized dense drop-ins, through the C-ABI against the CPU oracle.

The AF blob is synthetic: E-stacked tensors laid out as mlx_gpu_bind_af reads them
(mlx_moe.cpp:146-367): int4 affine words + fp32 scales + fp32 biases (bits=4), raw int8 +
scales (bits=8), qNg64 planes + scales (n), dense fp16 / fp32 rows (bits=16/32).
Bar: decoded weights bit-exact; products max|y - ref| / max|ref| <= 1e-5."""
import sys

import numpy as np
import pytest

from golden.fixtures import gate9, seeded_normal
from oracle_ffi import moe_decode, moe_ffn, moe_matvec

pytestmark = pytest.mark.gpu
TOL = 1e-5


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib(oracle):
    import torch
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    import beglin_amd
    L = beglin_amd.lib()
    assert L.bgl_gpu_available() == 1
    return L


@pytest.fixture(scope="module")
def R(lib):
    import beglin_amd
    return beglin_amd.Registry()


def relerr(y, r):
    y = np.asarray(y, np.float64); r = np.asarray(r, np.float64)
    return float(np.max(np.abs(y - r)) / max(np.max(np.abs(r)), 1e-30))


class Blob:
    """Appends arrays at 64-byte aligned offsets; .bytes() is the blob."""

    def __init__(self):
        self.parts, self.size = [], 0

    def add(self, a):
        a = np.ascontiguousarray(a)
        pad = (-self.size) % 64
        if pad:
            self.parts.append(np.zeros(pad, np.uint8)); self.size += pad
        off = self.size
        self.parts.append(a.view(np.uint8).reshape(-1)); self.size += a.nbytes
        return off

    def bytes(self):
        return np.concatenate(self.parts) if self.parts else np.zeros(0, np.uint8)


def af_tensor(oracle, bits, E, out, inn, seed):
    """Per-expert reference-layout arrays and oracle descriptors for one AF width."""
    rng = np.random.default_rng(seed)
    ng = inn // 64
    experts = []
    for e in range(E):
        w = seeded_normal(seed * 31 + e, (out, inn), 0.02)
        if bits == 4:
            pk = rng.integers(0, 256, (out, inn // 2), dtype=np.uint8)
            sc = (rng.random((out, ng), dtype=np.float32) * np.float32(0.01)).astype(np.float32)
            bi = (rng.standard_normal((out, ng), dtype=np.float32) * np.float32(0.04)).astype(np.float32)
            experts.append((6, 4, pk, sc, bi))
        elif bits == 8:
            pk, sc = oracle.quantize_q8g64(w)
            experts.append((2, 8, pk, sc))
        elif bits == 16:
            experts.append((7, 16, w.astype(np.float16).view(np.uint16), None))
        elif bits == 32:
            experts.append((8, 32, w, None))
        else:
            pk, sc = oracle.quantize_qng64(w, bits)
            experts.append((4, bits, pk, sc))
    return experts


def put_af(R, blob, name, experts, out, inn):
    """Lay the experts into the blob and bind them by name; returns the bind status."""
    bits = experts[0][1]
    pk_off = blob.add(np.stack([d[2] for d in experts]))
    sc_off = blob.add(np.stack([d[3] for d in experts])) if experts[0][3] is not None else -1
    bi_off = blob.add(np.stack([d[4] for d in experts])) if len(experts[0]) > 4 else -1
    return (pk_off, sc_off, bi_off, bits)


def bind_all(R, oracle, specs, E, out, inn, seed):
    """specs: {name: bits}.  Builds one blob with every tensor, binds each; returns descs."""
    blob, offs, descs = Blob(), {}, {}
    for i, (name, bits) in enumerate(specs.items()):
        descs[name] = af_tensor(oracle, bits, E, out, inn, seed + i)
        offs[name] = put_af(R, blob, name, descs[name], out, inn)
    b = blob.bytes()
    for name, (po, so, bo, bits) in offs.items():
        ok = R.bind_af(b, name, E, out, inn, inn // 64, po, so, bo, bits)
        assert ok == 1, f"bind {name} bits={bits}: {R.L().bgl_last_error().decode()}"
    return descs


WIDTHS = [4, 8, 2, 3, 5, 6, 7, 9, 12, 15, 16, 32]


def test_bind_kinds_and_dequant_probe(R, oracle):
    E, out, inn = 3, 80, 256
    say("registry bind + dequant probe")
    specs = {f"dq.b{b}": b for b in WIDTHS}
    descs = bind_all(R, oracle, specs, E, out, inn, 100)
    for name, bits in specs.items():
        k, kb = R.binding_kind(name)
        assert kb == bits
        assert k == (3 if bits in (7, 9, 12, 15) else 2 if bits in (16, 32) else 1), name
        for e, row, col0, n in ((0, 0, 0, inn), (E - 1, out - 1, 64, 100), (1, 33, 5, 7)):
            ok, got = R.dequant_probe(name, e, row, col0, n)
            assert ok == 1
            want = moe_decode(oracle, descs[name][e], out, inn, row, range(col0, col0 + n))
            assert np.array_equal(got, want), (name, e, row)
    assert R.dequant_probe("dq.b4", E, 0, 0, 4)[0] == 0          # expert out of range
    assert R.dequant_probe("dq.b4", 0, 0, inn - 2, 4)[0] == 0    # columns past the row
    assert R.binding_kind("dq.none") == (0, 0)


def test_matvec_probe_and_named_gather(R, oracle):
    E, out, inn, N = 4, 96, 512, 9
    say("registry matvec / gather")
    specs = {f"mv.b{b}": b for b in WIDTHS}
    descs = bind_all(R, oracle, specs, E, out, inn, 200)
    x = seeded_normal(201, (N, inn))
    idx = np.random.default_rng(202).integers(0, E, N).astype(np.int32)
    for name in specs:
        ok, y = R.matvec_probe(name, 2, x[0], out)
        assert ok == 1
        assert relerr(y, moe_matvec(oracle, descs[name][2], out, inn, x[0])) <= TOL, name
        ok, Y = R.ffn_gather(name, x, idx, out)
        assert ok == 1
        ref = np.stack([moe_matvec(oracle, descs[name][idx[z]], out, inn, x[z]) for z in range(N)])
        assert relerr(Y, ref) <= TOL, name


def test_qng64_gather_probe_gate9(R, lib, oracle):
    """mlx_gpu_qng64_gather_probe with the GATE9 fixture (qwen_infer.c:10811-10875)."""
    import ctypes as C
    say("gate9 probe")
    g = gate9()
    E, out, inn, n = g["E"], g["out"], g["inn"], g["n"]
    descs = [(4, n) + oracle.quantize_qng64_gguf(g["w"][e], n) for e in range(E)]
    planes = np.ascontiguousarray(np.stack([d[2] for d in descs]))
    scales = np.ascontiguousarray(np.stack([d[3] for d in descs]))
    x = np.ascontiguousarray(g["x"]); idx = np.ascontiguousarray(g["idx"])
    y = np.zeros((len(idx), out), np.float32)
    ok = lib.bgl_gpu_qng64_gather_probe(planes.ctypes.data, E, out, inn, inn // 64, n, scales.ctypes.data,
                                        x.ctypes.data, len(idx), idx.ctypes.data, y.ctypes.data)
    assert ok == 1
    ref = np.stack([moe_matvec(oracle, descs[e], out, inn, x[z]) for z, e in enumerate(idx)])
    assert relerr(y, ref) <= TOL
    # shape misuse is refused, not run
    assert lib.bgl_gpu_qng64_gather_probe(planes.ctypes.data, E, out, inn, 1, n, scales.ctypes.data,
                                          x.ctypes.data, len(idx), idx.ctypes.data, y.ctypes.data) == 0
    del C


def test_dense_probe_bind_refusals_and_bounds(R, lib, oracle):
    say("registry refusals")
    out, inn = 64, 128
    w = seeded_normal(300, (out, inn), 0.02)
    for n, want in ((5, 1), (7, 0), (4, 0), (8, 0)):
        p, s = oracle.quantize_qng64_gguf(w, n)
        assert lib.bgl_gpu_bind_qng64_dense_probe(p.ctypes.data, s.ctypes.data, f"dp.n{n}".encode(), out, inn, n) == want
    assert R.binding_kind("dp.n5") == (1, 5)
    x = seeded_normal(301, (inn,))
    p5, s5 = oracle.quantize_qng64_gguf(w, 5)
    ok, y = R.matvec_probe("dp.n5", 0, x, out)
    assert ok == 1 and relerr(y, moe_matvec(oracle, (4, 5, p5, s5), out, inn, x)) <= TOL
    blob = np.zeros(1 << 16, np.uint8)
    assert R.bind_af(blob, "bad.bits1", 1, 8, 64, 1, 0, 1024, -1, 1) == 0         # width refused
    assert R.bind_af(blob, "bad.n8", 1, 8, 64, 1, 0, 1024, -1, 0) == 0            # qNg64 n=8: caller passes 0
    assert R.bind_af(blob, "bad.ng", 1, 8, 128, 1, 0, 1024, -1, 8) == 0            # ng != in/64
    assert R.bind_af(blob, "bad.oob", 4, 256, 256, 4, 60000, 0, -1, 8) == 0       # past the blob
    assert R.bind_af(blob, "bad.nobias", 1, 8, 64, 1, 0, 1024, -1, 4) == 0         # affine needs biases
    big = 2**31 - 64                                                                 # E * out * in past 64 bits
    assert R.bind_af(blob, "bad.huge", 2**31 - 1, 2**31 - 1, big, big // 64, 0, 0, 0, 4) == 0
    assert b"2^40" in lib.bgl_last_error()
    assert R.binding_kind("bad.oob") == (0, 0)


def test_snapshot_restore_and_uniform_guard(R, lib, oracle):
    say("registry snapshots")
    E, out, inn = 2, 64, 128
    d4 = bind_all(R, oracle, {"sn.t": 4}, E, out, inn, 400)["sn.t"]
    x = seeded_normal(401, (inn,))
    ok, y0 = R.matvec_probe("sn.t", 1, x, out)
    assert ok == 1
    n0 = lib.bgl_gpu_binding_snapshot_count()
    ok, sid = R.snapshot("sn.t")
    assert ok == 1 and sid != 0 and lib.bgl_gpu_binding_snapshot_count() == n0 + 1
    d16 = bind_all(R, oracle, {"sn.t": 16}, E, out, inn, 402)["sn.t"]          # rebind the name dense
    assert R.binding_kind("sn.t") == (2, 16)
    ok, y1 = R.matvec_probe("sn.t", 1, x, out)
    assert relerr(y1, moe_matvec(oracle, d16[1], out, inn, x)) <= TOL
    assert lib.bgl_gpu_restore_binding_snapshot(sid) == 1
    assert R.binding_kind("sn.t") == (1, 4)
    ok, y2 = R.matvec_probe("sn.t", 1, x, out)
    assert np.array_equal(y2, y0) and relerr(y2, moe_matvec(oracle, d4[1], out, inn, x)) <= TOL
    assert lib.bgl_gpu_drop_binding_snapshot(sid) == 1
    assert lib.bgl_gpu_drop_binding_snapshot(sid) == 0
    assert lib.bgl_gpu_restore_binding_snapshot(sid) == 0
    assert lib.bgl_gpu_binding_snapshot_count() == n0
    assert R.snapshot("sn.missing")[0] == 0
    bind_all(R, oracle, {"un.g": 7, "un.u": 9, "un.d": 12, "un.q": 4, "un.f": 16}, 1, 64, 128, 410)
    f = lambda a, b, c: lib.bgl_gpu_test_ffn_uniform(a.encode(), b.encode(), c.encode())
    assert f("un.g", "un.u", "un.d") == 1          # all qNg64 planes
    assert f("un.g", "un.u", "un.q") == 0          # planes + native quantized
    assert f("un.q", "un.q", "un.f") == 0          # quantized + dense
    assert f("un.g", "un.u", "un.none") == -1


def test_registry_moe_ffn_by_name(R, oracle):
    """Routed SwiGLU FFN over registry names, shared experts as E=1 bindings."""
    say("registry moe_ffn")
    E, H, I, K, T, Ish = 8, 256, 128, 3, 7, 192
    fm = {"gate": 4, "up": 4, "down": 9}
    descs = {}
    for role, bits in fm.items():
        o, i = (I, H) if role != "down" else (H, I)
        descs[role] = bind_all(R, oracle, {f"ffn.{role}": bits}, E, o, i, 500 + len(descs))[f"ffn.{role}"]
    for role, (o, i) in (("sg", (Ish, H)), ("su", (Ish, H)), ("sd", (H, Ish))):
        descs[role] = bind_all(R, oracle, {f"ffn.{role}": 8}, 1, o, i, 520 + len(descs))[f"ffn.{role}"]
    x = seeded_normal(530, (T, H))
    idx, w = oracle.route(seeded_normal(531, (T, E)), K, False)
    ok, got = R.moe_ffn("ffn.gate", "ffn.up", "ffn.down", ("ffn.sg", "ffn.su", "ffn.sd"), x, idx, w)
    assert ok == 1
    shared = (descs["sg"][0], descs["su"][0], descs["sd"][0])
    ref = moe_ffn(oracle, descs["gate"], descs["up"], descs["down"], shared, H, I, x, idx, w)
    assert relerr(got, ref) <= TOL
    ok, got2 = R.moe_ffn("ffn.gate", "ffn.up", "ffn.down", None, x, idx, w)
    ref2 = moe_ffn(oracle, descs["gate"], descs["up"], descs["down"], None, H, I, x, idx, w)
    assert ok == 1 and relerr(got2, ref2) <= TOL
    assert R.moe_ffn("ffn.gate", "ffn.up", "ffn.none", None, x, idx, w)[0] == 0


def test_registry_moe_layer_with_router(R, oracle):
    """moe_ffn_batched by names with the router registered (bgl_gpu_bind_router): the routing the
    call returns equals or_moe_router_logits + or_moe_route, the output the oracle's bucketed FFN."""
    say("registry moe_layer")
    E, H, I, K, T, Ish = 8, 256, 128, 3, 6, 192
    rw = seeded_normal(540, (E, H), 0.06)
    rb = seeded_normal(541, (E,), 0.1)
    assert R.bind_router("ffn.router", rw, rb) == 1
    x = seeded_normal(542, (T, H))
    ridx, rwt = oracle.route(oracle.router_logits(rw, x, rb), K, True)
    ok, got, idx, w = R.moe_layer("ffn.router", "ffn.gate", "ffn.up", "ffn.down", ("ffn.sg", "ffn.su", "ffn.sd"), x, K,
                                  renorm=True)
    assert ok == 1
    assert np.array_equal(idx, ridx)
    np.testing.assert_allclose(w, rwt, rtol=1e-6, atol=1e-9)
    descs = {}
    for role, bits in {"gate": 4, "up": 4, "down": 9}.items():
        o, i = (I, H) if role != "down" else (H, I)
        descs[role] = bind_all(R, oracle, {f"ffn.{role}": bits}, E, o, i, 500 + len(descs))[f"ffn.{role}"]
    for role, (o, i) in (("sg", (Ish, H)), ("su", (Ish, H)), ("sd", (H, Ish))):
        descs[role] = bind_all(R, oracle, {f"ffn.{role}": 8}, 1, o, i, 520 + len(descs))[f"ffn.{role}"]
    ok, got, idx, w = R.moe_layer("ffn.router", "ffn.gate", "ffn.up", "ffn.down", ("ffn.sg", "ffn.su", "ffn.sd"), x, K,
                                  renorm=True)
    shared = (descs["sg"][0], descs["su"][0], descs["sd"][0])
    ref = moe_ffn(oracle, descs["gate"], descs["up"], descs["down"], shared, H, I, x, ridx, rwt)
    assert ok == 1 and relerr(got, ref) <= TOL
    assert R.moe_layer("ffn.nope", "ffn.gate", "ffn.up", "ffn.down", None, x, K)[0] == 0          # unknown router
    assert R.bind_router("ffn.r5", seeded_normal(543, (5, H), 0.05)) == 1
    assert R.moe_layer("ffn.r5", "ffn.gate", "ffn.up", "ffn.down", None, x, K)[0] == 0            # E mismatch
    assert R.bind_router("ffn.bad", seeded_normal(544, (4, 6), 0.05)) == 0                        # in % 4


def test_mixed_qng64_bind_decode_and_probes(R, lib, oracle):
    """Mixed per-cell qNg64 (mlx_moe.h:104-116): device decode bit-exact against the oracle; the
    one-shot GEMV probe (batch 1 / 3 / 20, the last on the matrix-core path when every width <= 10)
    and the bound name through the matvec probe against the decoded product; kind 4 with bits 0;
    the dequant probe and experts e != 0 refused; snapshot / restore; the binders' checks."""
    import torch
    import beglin_amd
    from oracle_ffi import mixed_qng64_random
    say("mixed qNg64")
    rng = np.random.default_rng(77)
    out, inn = 200, 512
    for widths in (list(range(2, 16)), [2, 3, 4, 5, 6], [9]):
        planes, offsets, bits, scales = mixed_qng64_random(rng, out, inn, widths)
        wref = oracle.decode_qng64_mixed(planes, offsets, bits, scales, out, inn)
        ctx = beglin_amd.Context(0)
        t = ctx.bind_qng64_mixed(planes, offsets, bits, scales, out, inn)
        assert t.info()["kind"] == 4 and t.info()["bits"] == max(widths)
        dq = torch.empty((out, inn), device="cuda")
        ctx.dequant(t, 0, out, dq)
        ctx.sync()
        assert np.array_equal(dq.cpu().numpy().view(np.uint32), wref.view(np.uint32)), widths
        t.free(); ctx.close()
        for batch in (1, 3, 20):
            x = seeded_normal(600 + batch, (batch, inn))
            ok, y = R.mixed_probe(planes, offsets, bits, scales, out, inn, x)
            ref = x.astype(np.float64) @ wref.astype(np.float64).T
            assert ok == 1 and relerr(y, ref) <= TOL, (widths, batch)
    assert R.bind_mixed("mx.t", planes, offsets, bits, scales, out, inn) == 1
    assert R.binding_kind("mx.t") == (4, 0)
    x = seeded_normal(610, (inn,))
    ok, y = R.matvec_probe("mx.t", 0, x, out)
    assert ok == 1 and relerr(y, wref.astype(np.float64) @ x.astype(np.float64)) <= TOL
    assert R.matvec_probe("mx.t", 1, x, out)[0] == 0
    assert R.dequant_probe("mx.t", 0, 0, 0, 64)[0] == 0
    ok, sid = R.snapshot("mx.t")
    assert ok == 1
    bind_all(R, oracle, {"mx.t": 8}, 1, out, inn, 620)
    assert R.binding_kind("mx.t") == (1, 8)
    assert lib.bgl_gpu_restore_binding_snapshot(sid) == 1 and R.binding_kind("mx.t") == (4, 0)
    assert np.array_equal(R.matvec_probe("mx.t", 0, x, out)[1], y)
    assert lib.bgl_gpu_drop_binding_snapshot(sid) == 1
    # the binders' checks (mlx_moe.cpp:1750-1758): every refusal leaves the binding as it was
    bad = offsets.copy(); bad[0] = 8
    assert R.bind_mixed("mx.t", planes, bad, bits, scales, out, inn) == 0
    bad = offsets.copy(); bad[-1] += 8
    assert R.bind_mixed("mx.t", planes, bad, bits, scales, out, inn) == 0
    b16 = bits.copy(); b16[3] = 16
    assert R.bind_mixed("mx.t", planes, offsets, b16, scales, out, inn) == 0
    for v in (0.0, -1.0, np.inf, np.nan):
        s = scales.copy(); s[5] = v
        assert R.bind_mixed("mx.t", planes, offsets, bits, s, out, inn) == 0
        assert R.mixed_probe(planes, offsets, bits, s, out, inn, x[None])[0] == 0
    assert R.binding_kind("mx.t") == (4, 0)


def test_memory_report_epoch_and_counters(R, lib, oracle):
    import ctypes as C
    say("registry memory / epoch")
    a, p, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
    lib.bgl_gpu_report_memory(C.byref(a), C.byref(p), C.byref(c))
    assert a.value > 0 and p.value >= a.value
    zc, cp, nb = C.c_int(), C.c_int(), C.c_size_t()
    n = lib.bgl_gpu_zerocopy_count(C.byref(zc), C.byref(cp), C.byref(nb))
    assert n > 0 and zc.value == 0 and cp.value == n and nb.value > 0
    assert lib.bgl_gpu_set_batch(64) == 1 and lib.bgl_gpu_set_batch(65) == 0 and lib.bgl_gpu_set_batch(0) == 0
    assert lib.bgl_gpu_set_sort_threshold(8) == 1
    assert lib.bgl_gpu_reset_runtime_epoch() == 1
    lib.bgl_gpu_report_memory(None, None, C.byref(c))
    assert c.value == 0                               # per-call scratch released
    assert lib.bgl_gpu_synchronize() == 1
    # bindings survive the epoch reset
    assert R.binding_kind("mv.b9")[0] == 3
    x = seeded_normal(600, (512,))
    assert R.matvec_probe("mv.b9", 0, x, 96)[0] == 1


# ---------------------------------------------------------------- caller-quantized drop-ins
def split_act(xq):
    """q4_split_act's order (q4gemv.h:306-312): per 32 bytes, the even then the odd elements."""
    M, K = xq.shape
    v = xq.reshape(M, K // 32, 16, 2)
    return np.ascontiguousarray(np.concatenate([v[..., 0], v[..., 1]], axis=2).reshape(M, K))


@pytest.mark.parametrize("kind,M", [(1, 1), (1, 5), (2, 3), (3, 1), (3, 4)])
def test_caller_quantized_sdot_dropins(lib, oracle, kind, M):
    import beglin_amd
    import ctypes as C
    import torch
    say("sdot drop-in", kind, M)
    out, inn = 136, 1024
    w = seeded_normal(700 + kind, (out, inn), 0.02)
    x = seeded_normal(710 + M, (M, inn))
    bias = seeded_normal(720, (out,))
    gs = 256 if kind == 3 else 64
    xq, a = oracle.quant_act_i8(x, gs)
    xq = np.ascontiguousarray(xq.reshape(M, inn)); a = np.ascontiguousarray(a.reshape(M, -1))
    xin = xq if kind == 2 else split_act(xq)
    ctx = beglin_amd.Context(0, stream=torch.cuda.current_stream().cuda_stream)
    y = np.zeros((M, out), np.float32)
    if kind == 3:
        p, s, sub = oracle.quantize_g256sf(w)
        rc = lib.bgl_gemm_q4g256sf_sdot_mt(ctx.h, p.ctypes.data, s.ctypes.data, sub.ctypes.data, xin.ctypes.data,
                                           a.ctypes.data, bias.ctypes.data, y.ctypes.data, out, inn, M)
        ref = oracle.gemm_sdot(3, p, s, xq, a, bias=bias, sub=sub)
    else:
        p, s = oracle.quantize_q4g64(w) if kind == 1 else oracle.quantize_q8g64(w)
        rc = lib.bgl_gemm_qXg64_sdot_mt(ctx.h, 4 if kind == 1 else 8, p.ctypes.data, s.ctypes.data, xin.ctypes.data,
                                        a.ctypes.data, bias.ctypes.data, y.ctypes.data, out, inn, M)
        ref = oracle.gemm_sdot(kind, p, s, xq, a, bias=bias)
    assert rc == 0, lib.bgl_last_error().decode()
    assert relerr(y, ref) <= TOL
    if kind == 1 and M == 1:
        y1, y2 = np.zeros(out, np.float32), np.zeros(out, np.float32)
        x0 = np.ascontiguousarray(x[0])
        assert lib.bgl_gemv_q4g64_mt(ctx.h, p.ctypes.data, s.ctypes.data, x0.ctypes.data, None, y1.ctypes.data, out, inn) == 0
        assert lib.bgl_gemv_q4g64_mt_fused(ctx.h, p.ctypes.data, s.ctypes.data, x0.ctypes.data, None, y2.ctypes.data,
                                           out, inn) == 0
        assert np.array_equal(y1, y2)
    bad = lib.bgl_gemm_qXg64_sdot_mt(ctx.h, 5, p.ctypes.data, s.ctypes.data, xin.ctypes.data, a.ctypes.data, None,
                                     y.ctypes.data, out, inn, M)
    assert bad != 0
    ctx.sync()
    ctx.close()
    del C


def test_af_layout_manifest_binds_and_multiplies(R, oracle, tmp_path):
    """bgl_gpu_load_layout_af (moe_load_layout_af, qwen_infer.c:2496-2515): every record of the
    manifest is bound as an int4 affine tensor under its name; each expert's product equals the
    oracle's moe_matvec_af_row, the decode equals moe_decode_af bit for bit, and the named gather
    and the routed SwiGLU FFN run over the loaded names."""
    from loader_fixture import build_af
    say("AF layout manifest")
    layout, blob, recs = build_af(str(tmp_path), seed=11)
    assert R.load_layout_af(layout, blob) == len(recs)
    descs = {}
    for name, (E, out, inn, codes, sc, bi) in recs.items():
        assert R.binding_kind(name) == (1, 4), name
        descs[name] = [(6, 4, codes[e], sc[e], bi[e]) for e in range(E)]
        x = seeded_normal(1100 + E + out, (inn,))
        for e in range(E):
            ok, y = R.matvec_probe(name, e, x, out)
            assert ok == 1
            assert relerr(y, moe_matvec(oracle, descs[name][e], out, inn, x)) <= TOL, (name, e)
        ok, got = R.dequant_probe(name, E - 1, out - 1, 0, inn)
        assert ok == 1 and np.array_equal(got, moe_decode(oracle, descs[name][E - 1], out, inn, out - 1, range(inn)))
    g, u, d = "layers.0.mlp.experts.gate", "layers.0.mlp.experts.up", "layers.0.mlp.experts.down"
    T, K, H, I = 5, 2, 128, 64
    x = seeded_normal(1200, (T, H))
    idx, w = oracle.route(seeded_normal(1201, (T, 4)), K, True)
    out = np.zeros((T, H), np.float32)
    import ctypes as C
    ok = R.L().bgl_gpu_moe_ffn(g.encode(), u.encode(), d.encode(), None, None, None, x.ctypes.data, T,
                               np.ascontiguousarray(idx, np.int32).ctypes.data,
                               np.ascontiguousarray(w, np.float32).ctypes.data, K, out.ctypes.data)
    assert ok == 1, R.L().bgl_last_error().decode()
    ref = moe_ffn(oracle, descs[g], descs[u], descs[d], None, H, I, x, idx, w)
    assert relerr(out, ref) <= TOL
    del C
    # a manifest that fails its checks binds nothing and says why
    bad = tmp_path / "bad_af.txt"
    bad.write_text(open(layout).read().replace(" 4 64 128 2 ", " 4 64 128 3 ", 1))
    assert R.load_layout_af(str(bad), blob) == -1
    assert "ng" in R.L().bgl_last_error().decode()
