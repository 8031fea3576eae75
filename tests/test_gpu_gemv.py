"""GPU parity: the HIP library (through the C-ABI) against the CPU oracle on the same inputs.

Bar: packed bytes, decoded weights and int8 activation codes bit-exact; GEMV outputs within
max|y - ref| / max|ref| <= 1e-5 (fp32 accumulation, order-of-summation differences only)."""
import sys

import numpy as np
import pytest

from golden.fixtures import seeded_normal

pytestmark = pytest.mark.gpu
TOL = 1e-5


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    return torch


@pytest.fixture(scope="module")
def ctx(torch_dev):
    import beglin_amd
    c = beglin_amd.Context(0)
    yield c
    c.sync()
    c.close()


def relerr(y, r):
    y = np.asarray(y, np.float64); r = np.asarray(r, np.float64)
    return float(np.max(np.abs(y - r)) / max(np.max(np.abs(r)), 1e-30))


def weights(seed, out, inn, edge=True):
    w = seeded_normal(seed, (out, inn), 0.02)
    rng = np.random.default_rng(seed + 1)
    w[rng.random(w.shape) < 0.01] *= 8
    if edge and out > 3:
        w[1, :] = 0.0
        w[2, :64] = 5e-12
    return w


def ref_quant(oracle, kind, w, bits=0):
    if kind == 1:
        p, s = oracle.quantize_q4g64(w); return p, s, None
    if kind == 2:
        p, s = oracle.quantize_q8g64(w); return p, s, None
    if kind == 3:
        return oracle.quantize_g256sf(w)
    if kind == 4:
        p, s = oracle.quantize_qng64(w, bits); return p, s, None
    p, s = oracle.quantize_q4g32h(w); return p, s, None


CASES = [(1, 0), (2, 0), (3, 0), (5, 0)] + [(4, n) for n in range(2, 16)]


@pytest.mark.parametrize("kind,bits", CASES)
def test_device_packer_bytes_and_decode(ctx, torch_dev, oracle, kind, bits):
    torch = torch_dev
    out, inn = 77, 512
    say("packer", kind, bits, out, inn)
    w = weights(100 + kind * 20 + bits, out, inn)
    pk, sc, sub = ref_quant(oracle, kind, w, bits)
    t, (gpk, gsc, gsub) = ctx.quantize(kind, torch.from_numpy(w).cuda(), bits=bits, qng64_encoder=(bits != 4), want_ref=True)
    assert np.array_equal(gpk, pk), "device packer bytes differ"
    assert np.array_equal(gsc.view(np.uint8), sc.view(np.uint8)), "device packer scales differ"
    if sub is not None:
        assert np.array_equal(gsub, sub)
    want = oracle.decode(kind, pk, sc, out, inn, bits=bits, sub=sub)
    got = torch.empty((out, inn), dtype=torch.float32, device="cuda")
    ctx.dequant(t, 0, out, got)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32)), "tiled-layout decode not bit-exact"
    # host-side bind of the same reference bytes decodes identically
    t2 = ctx.bind(kind, pk, sc, out, inn, bits=bits, sub=sub)
    got2 = torch.empty_like(got)
    ctx.dequant(t2, 0, out, got2)
    torch.cuda.synchronize()
    assert torch.equal(got, got2)
    t.free(); t2.free()


@pytest.mark.parametrize("gsize", [64, 256])
def test_w4a8_activation_codes_bit_exact(ctx, torch_dev, oracle, gsize):
    torch = torch_dev
    say("quant_act", gsize)
    x = seeded_normal(7, (5, 2048))
    x[0, :gsize] = 0.0                                     # 1e-8 floor
    x[1, :4] = [127.0, 2.5 * 127 / 127, -0.5, 0.5]         # ties go away from zero
    xq, a = oracle.quant_act_i8(x, gsize)
    xd = torch.from_numpy(x).cuda()
    gq = torch.empty((5, 2048), dtype=torch.int8, device="cuda")
    ga = torch.empty((5, 2048 // gsize), dtype=torch.float32, device="cuda")
    ctx.quant_act_i8(xd, gsize, gq, ga)
    torch.cuda.synchronize()
    assert np.array_equal(gq.cpu().numpy(), xq)
    assert np.array_equal(ga.cpu().numpy().view(np.uint32), a.view(np.uint32))


def nonfinite_columns(M, K, seed):
    """M columns: column m % 4 == 0 carries a NaN, 1 a +Inf, 2 a -Inf (each in one group), 3 is
    finite; the non-finite values sit at different offsets so both gsize 64 and 256 see them."""
    x = seeded_normal(seed, (M, K))
    for m in range(M):
        j = (97 * m + 13) % K
        if m % 4 == 0:
            x[m, j] = np.nan
        elif m % 4 == 1:
            x[m, j] = np.inf
        elif m % 4 == 2:
            x[m, j] = -np.inf
    return x


def same_scales(got, want):
    """Scales bit-exact where finite, NaN where the oracle's is NaN (the NaN payload is not part
    of the reference's contract), +Inf where +Inf."""
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


@pytest.mark.parametrize("gsize", [64, 256])
def test_w4a8_activation_codes_nonfinite(ctx, torch_dev, oracle, gsize):
    """k_act_w4a8 on NaN / +-Inf groups: every code 0, scale NaN or +Inf (FMAX / FCVTZS semantics
    of q4gemv.h:182-206 and q4gemv_g256.h:76-96, restated by the oracle)."""
    torch = torch_dev
    say("quant_act nonfinite", gsize)
    x = nonfinite_columns(8, 2048, 11)
    xq, a = oracle.quant_act_i8(x, gsize)
    gq = torch.empty((8, 2048), dtype=torch.int8, device="cuda")
    ga = torch.empty((8, 2048 // gsize), dtype=torch.float32, device="cuda")
    ctx.quant_act_i8(torch.from_numpy(x).cuda(), gsize, gq, ga)
    torch.cuda.synchronize()
    assert np.array_equal(gq.cpu().numpy(), xq)
    same_scales(ga.cpu().numpy(), a)
    assert np.isnan(a[0]).any() and np.isposinf(a[1]).any() and np.isposinf(a[2]).any()


# (kind, K): q4g64, q8g64 and g256sf; M = 1 quantizes in the GEMV kernel, M = 8 over K = 8960
# quantizes every column once up front (k_act_w4a8) and copies the codes
@pytest.mark.parametrize("kind,inn,M", [(1, 1536, 1), (2, 1536, 1), (3, 1536, 1), (1, 8960, 8), (2, 8960, 8),
                                        (3, 8960, 8), (3, 8960, 4), (3, 1536, 8)])
def test_w4a8_nonfinite_outputs(ctx, torch_dev, oracle, kind, inn, M):
    """A column with a NaN or +-Inf activation: every output row NaN, as in the reference (codes 0
    times a NaN / +Inf scale); the finite columns are bit-exact."""
    torch = torch_dev
    out = 200
    say("w4a8 nonfinite", kind, inn, M)
    w = weights(700 + kind, out, inn)
    pk, sc, sub = ref_quant(oracle, kind, w)
    t = ctx.bind(kind, pk, sc, out, inn, sub=sub)
    cols = [nonfinite_columns(4, inn, 12 + kind)[i] for i in range(4)]
    for start in range(0, 4, M) if M == 1 else [0]:
        x = np.stack([cols[(start + m) % 4] for m in range(M)]).astype(np.float32)
        ref = oracle.matmul_sdot(kind, pk, sc, x, sub=sub)
        y = torch.full((M, out), 7.0, dtype=torch.float32, device="cuda")
        ctx.matmul(t, torch.from_numpy(x).cuda(), y, act=1)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(ref)), (start, np.isnan(got).sum(), np.isnan(ref).sum())
        assert not np.isinf(ref).any() and not np.isinf(got).any()
        fin = np.isfinite(ref)
        assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
        for m in range(M):
            assert np.isnan(ref[m]).all() == ((start + m) % 4 != 3)
    t.free()


GEMV_CASES = [
    (1, 0, 0, 1536), (1, 0, 1, 1536), (2, 0, 0, 1024), (2, 0, 1, 1024), (3, 0, 1, 1536), (5, 0, 0, 1536),
    (4, 2, 0, 1024), (4, 3, 0, 1024), (4, 4, 0, 1024), (4, 5, 0, 1408), (4, 7, 0, 1024), (4, 8, 0, 1024),
    (4, 12, 0, 1024), (4, 15, 0, 1024), (4, 9, 0, 192),
    # few row tiles and a long K: the K dimension is split over workgroups (deterministic tail sum)
    (1, 0, 0, 4096), (1, 0, 1, 4096), (4, 15, 0, 8192), (5, 0, 0, 8192),
    # W4A8 quantization passes of 256 values: partial last pass (K % 256 != 0), four passes per
    # wave (g256sf K=8960), and more passes than one round of loads covers (K=20480)
    (1, 0, 1, 320), (2, 0, 1, 1408), (3, 0, 1, 8960), (1, 0, 1, 20480),
]


@pytest.mark.parametrize("kind,bits,act,inn", GEMV_CASES)
@pytest.mark.parametrize("M", [1, 3, 8, 13])
def test_gemv_parity(ctx, torch_dev, oracle, kind, bits, act, inn, M):
    torch = torch_dev
    out = 200
    say("gemv", kind, bits, act, inn, M)
    w = weights(300 + kind * 20 + bits, out, inn)
    pk, sc, sub = ref_quant(oracle, kind, w, bits)
    x = seeded_normal(400 + M, (M, inn))
    bias = seeded_normal(500, (out,))
    if act == 0:
        ref = oracle.gemm_f32(kind, pk, sc, x, bias=bias, bits=bits)
    else:
        ref = oracle.matmul_sdot(kind, pk, sc, x, bias=bias, sub=sub)
    t = ctx.bind(kind, pk, sc, out, inn, bits=bits, sub=sub)
    xd = torch.from_numpy(x).cuda()
    bd = torch.from_numpy(bias).cuda()
    y = torch.full((M, out), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matmul(t, xd, y, act=act, bias_dev=bd)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    e = relerr(got, ref)
    print(f"  max-rel {e:.3e}")
    assert np.all(np.isfinite(got))
    assert e <= TOL, e
    if act == 1:
        # W4A8 runs the fused kernel (launches of 1, 4 or 8 columns), which folds each column's
        # groups in the reference's order
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "fused W4A8 fold not bit-exact"
    t.free()


def test_fused_group_equals_separate(ctx, torch_dev, oracle):
    """q/k/v in one launch == three launches (QWEN_FUSED_DISPATCH)."""
    torch = torch_dev
    say("fused group")
    shapes = [(1536, 1536), (256, 1536), (256, 1536)]
    ts, ys1, ys2 = [], [], []
    x = torch.from_numpy(seeded_normal(9, (1536,))).cuda()
    for i, (o, k) in enumerate(shapes):
        pk, ws, sub = oracle.quantize_g256sf(weights(600 + i, o, k, edge=False))
        ts.append(ctx.bind(3, pk, ws, o, k, sub=sub))
        ys1.append(torch.empty(o, device="cuda")); ys2.append(torch.empty(o, device="cuda"))
    ctx.matmul_group(ts, x, ys1, act=1)
    for t, y in zip(ts, ys2):
        ctx.matmul(t, x, y, act=1)
    torch.cuda.synchronize()
    for a, b in zip(ys1, ys2):
        assert torch.equal(a, b)
    for t in ts:
        t.free()


def test_host_pointer_dropins(ctx, torch_dev, oracle):
    """The reference-signature entry points (q4gemv.h:672-791, q4gemv_g256.h:339, qng64_dense.c:70-100)."""
    import ctypes as C
    import beglin_amd
    L = beglin_amd.lib()
    say("host drop-ins")
    out, inn = 130, 1024
    w = weights(700, out, inn)
    x = seeded_normal(701, (4, inn))
    bias = seeded_normal(702, (out,))
    P = lambda a: C.c_void_p(a.ctypes.data) if a is not None else None
    y = np.zeros((4, out), np.float32)
    pk, sc = oracle.quantize_q4g64(w)
    assert L.bgl_gemv_q4g64_mt(ctx.h, P(pk), P(sc), P(x[0]), P(bias), P(y[0]), out, inn) == 0
    assert relerr(y[0], oracle.gemm_f32(1, pk, sc, x[0], bias=bias)) <= TOL
    assert L.bgl_gemv_q4g64_sdot_mt(ctx.h, P(pk), P(sc), P(x[0]), P(bias), P(y[0]), out, inn) == 0
    assert relerr(y[0], oracle.matmul_sdot(1, pk, sc, x[0], bias=bias)) <= TOL
    assert L.bgl_gemm_qXg64_mt(ctx.h, 4, P(pk), P(sc), P(x), None, P(y), out, inn, 4) == 0
    assert relerr(y, oracle.gemm_f32(1, pk, sc, x)) <= TOL
    c8, s8 = oracle.quantize_q8g64(w)
    assert L.bgl_gemv_q8g64_mt(ctx.h, P(c8), P(s8), P(x[1]), None, P(y[1]), out, inn) == 0
    assert relerr(y[1], oracle.gemm_f32(2, c8, s8, x[1])) <= TOL
    assert L.bgl_gemv_q8g64_sdot_mt(ctx.h, P(c8), P(s8), P(x[1]), P(bias), P(y[1]), out, inn) == 0
    assert relerr(y[1], oracle.matmul_sdot(2, c8, s8, x[1], bias=bias)) <= TOL
    pg, wsu, sub = oracle.quantize_g256sf(w)
    assert L.bgl_gemv_q4g256sf_sdot_mt(ctx.h, P(pg), P(wsu), P(sub), P(x[2]), P(bias), P(y[2]), out, inn) == 0
    assert relerr(y[2], oracle.matmul_sdot(3, pg, wsu, x[2], bias=bias, sub=sub)) <= TOL
    assert L.bgl_gemm_q4g256sf_mt(ctx.h, P(pg), P(wsu), P(sub), P(x), P(bias), P(y), out, inn, 4) == 0
    assert relerr(y, oracle.matmul_sdot(3, pg, wsu, x, bias=bias, sub=sub)) <= TOL
    pq, sq = oracle.quantize_qng64(w, 5)
    assert L.bgl_qng64_matvec_f32(ctx.h, P(pq), P(sq), 5, P(x[3]), P(bias), P(y[3]), out, inn) == 0
    assert relerr(y[3], oracle.gemm_f32(4, pq, sq, x[3], bias=bias, bits=5)) <= TOL
    assert L.bgl_qng64_matmul_f32(ctx.h, P(pq), P(sq), 5, P(x), P(bias), P(y), out, inn, 4) == 0
    assert relerr(y, oracle.gemm_f32(4, pq, sq, x, bias=bias, bits=5)) <= TOL
    ph, sh = oracle.quantize_q4g32h(w)
    assert L.bgl_gemv_q4g32h_mt(ctx.h, P(ph), P(sh), P(x[0]), P(bias), P(y[0]), out, inn) == 0
    assert relerr(y[0], oracle.gemm_f32(5, ph, sh, x[0], bias=bias)) <= TOL
    for a in (pk, c8, pg, pq, ph):
        assert L.bgl_forget(ctx.h, P(a)) == 0


def test_error_paths(ctx, torch_dev, oracle):
    import ctypes as C
    import beglin_amd
    L = beglin_amd.lib()
    say("error paths")
    out, inn = 64, 512
    pg, wsu, sub = oracle.quantize_g256sf(weights(800, out, inn, edge=False))
    t = ctx.bind(3, pg, wsu, out, inn, sub=sub)
    x = __import__("torch").zeros(inn, device="cuda")
    y = __import__("torch").zeros(out, device="cuda")
    with pytest.raises(beglin_amd.BglError, match="requires W4A8"):
        ctx.matmul(t, x, y, act=0)                       # qwen_infer.c:697-702 FATAL -> error code
    t.free()
    P = lambda a: C.c_void_p(a.ctypes.data)
    z = np.zeros(100, np.float32)
    assert L.bgl_gemv_q4g64_mt(ctx.h, P(z), P(z), P(z), None, P(z), 10, 100) == -1     # in % 64
    assert L.bgl_qng64_matvec_f32(ctx.h, P(z), P(z), 16, P(z), None, P(z), 1, 64) == -1  # n out of range


FULL = [
    ("cfg1 int4 g32 fp16 gate_proj", 5, 0, 0, 8960, 1536),
    ("cfg2 g256sf W4A8 down_proj", 3, 0, 1, 1536, 8960),
    ("cfg3 qNg64 n=2 gate", 4, 2, 0, 14336, 4096),
    ("cfg3 qNg64 n=15 down", 4, 15, 0, 4096, 14336),
]


@pytest.mark.parametrize("name,kind,bits,act,out,inn", FULL)
def test_full_size_configs(ctx, torch_dev, oracle, name, kind, bits, act, out, inn):
    """BASELINE shapes at full size, weights quantized on the device and checked byte-exact
    against the oracle packer, output against the oracle GEMV."""
    torch = torch_dev
    say("full", name)
    w = seeded_normal(900 + kind + bits, (out, inn), 0.02)
    t, (gpk, gsc, gsub) = ctx.quantize(kind, torch.from_numpy(w).cuda(), bits=bits, want_ref=True)
    pk, sc, sub = ref_quant(oracle, kind, w, bits)
    assert np.array_equal(gpk, pk) and np.array_equal(gsc.view(np.uint8), sc.view(np.uint8))
    x = seeded_normal(901, (inn,))
    y = torch.empty(out, device="cuda")
    ctx.matmul(t, torch.from_numpy(x).cuda(), y, act=act)
    torch.cuda.synchronize()
    ref = oracle.gemm_f32(kind, pk, sc, x, bits=bits) if act == 0 else oracle.matmul_sdot(kind, pk, sc, x, sub=sub)
    e = relerr(y.cpu().numpy(), ref)
    print(f"  max-rel {e:.3e}")
    assert e <= TOL
    t.free()


def test_w4a8_fused_and_separate_paths_agree(torch_dev, oracle, monkeypatch):
    """M=1 W4A8 through the fused-quantization kernel vs through the separate prep kernel."""
    import beglin_amd
    torch = torch_dev
    say("fused vs separate W4A8")
    out, inn = 320, 2048
    pk, ws, sub = oracle.quantize_g256sf(weights(1000, out, inn))
    x = torch.from_numpy(seeded_normal(1001, (1, inn))).cuda()
    ys = []
    for flag in ("0", "1"):
        monkeypatch.setenv("BGL_NO_FUSED_Q", flag)
        c = beglin_amd.Context(0)
        t = c.bind(3, pk, ws, out, inn, sub=sub)
        y = torch.empty((1, out), device="cuda")
        c.matmul(t, x, y, act=1)
        torch.cuda.synchronize()
        ys.append(y.cpu().numpy())
        t.free(); c.close()
    assert relerr(ys[1], ys[0]) <= 1e-6


def test_graph_replays_match_eager(ctx, torch_dev, oracle):
    """Capture a GEMV sequence into a HIP graph, replay it several times with eager work and
    synchronisations in between; every replay must equal the eager result bit for bit."""
    torch = torch_dev
    say("graph replay")
    out, inn = 700, 4096
    tq = ctx.bind(4, *ref_quant(oracle, 4, weights(1100, out, inn), 7)[:2], out, inn, bits=7)
    pg, ws, sub = oracle.quantize_g256sf(weights(1101, out, inn))
    tg = ctx.bind(3, pg, ws, out, inn, sub=sub)
    x = torch.from_numpy(seeded_normal(1102, (4, inn))).cuda()
    y1 = torch.empty((4, out), device="cuda"); y2 = torch.empty((1, out), device="cuda")

    def step():
        ctx.matmul(tq, x, y1, act=0)
        ctx.matmul(tg, x[:1], y2, act=1)

    step(); torch.cuda.synchronize()
    e1, e2 = y1.clone(), y2.clone()
    cs = torch.cuda.Stream()
    import beglin_amd
    c2 = beglin_amd.Context(0, stream=cs.cuda_stream)
    tq2 = c2.bind(4, *ref_quant(oracle, 4, weights(1100, out, inn), 7)[:2], out, inn, bits=7)
    tg2 = c2.bind(3, pg, ws, out, inn, sub=sub)

    def step2():
        c2.matmul(tq2, x, y1, act=0)
        c2.matmul(tg2, x[:1], y2, act=1)

    with torch.cuda.stream(cs):
        step2()
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=cs):
        step2()
    for rep in range(4):
        y1.fill_(float("nan")); y2.fill_(float("nan"))
        with torch.cuda.stream(cs):
            g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(y1, e1) and torch.equal(y2, e2), f"replay {rep} differs"
        step(); torch.cuda.synchronize()                       # eager work between replays
    for t in (tq, tg, tq2, tg2):
        t.free()
    c2.close()


@pytest.mark.parametrize("nonfinite", [False, True])
def test_prepped_activation_reuse(ctx, torch_dev, oracle, nonfinite):
    """Prepare once, run two GEMVs (gemm_qXg64_sdot_mt's caller-quantized activations), for fp32
    and W4A8 activations, g256sf and plain g256 included.  The prepared operands belong to the
    context: x is overwritten (with NaN) after the prep, and the GEMVs still see the prepared x --
    also the NaN / Inf elements of x the fp32 GEMVs read again.  Operands that a GEMV call prepared
    for itself are not offered to a prepped call."""
    import beglin_amd
    torch = torch_dev
    say("prepped reuse", nonfinite)
    inn = 2048
    x = seeded_normal(1200, (3, inn))
    if nonfinite:
        x[0, 5] = np.nan
        x[1, 700] = np.inf
        x[2, 1900] = -np.inf
    for act, kind in ((0, 1), (1, 1), (0, 2), (1, 3), (1, beglin_amd.K_Q4G256P)):
        ts, refs = [], []
        for i, out in enumerate((96, 160)):
            if kind == beglin_amd.K_Q4G256P:
                rng = np.random.default_rng(1205 + i)
                pk = rng.integers(0, 256, (out, inn // 2), dtype=np.uint8)
                sc = (rng.random((out, inn // 256), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
                sub = None
            else:
                pk, sc, sub = ref_quant(oracle, kind, weights(1201 + i, out, inn), 0)
            ts.append(ctx.bind(kind, pk, sc, out, inn, sub=sub))
            refs.append(oracle.gemm_f32(kind, pk, sc, x) if act == 0 else oracle.matmul_sdot(kind, pk, sc, x, sub=sub))
        xd = torch.from_numpy(x).cuda()
        ctx.prep_only(xd, act, ts[0])
        xd.fill_(float("nan"))                                 # the caller reuses its buffer
        for t, ref in zip(ts, refs):
            y = torch.empty((3, t.info()["out"]), device="cuda")
            ctx.matmul_prepped(t, y, act=act, M=3)
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            for f in (np.isnan, np.isposinf, np.isneginf):
                assert np.array_equal(f(got), f(ref)), (act, kind, f.__name__)
            fin = np.isfinite(ref)
            if fin.any():                                  # (prepared operands run k_gemv's wave order)
                assert relerr(got[fin], ref[fin]) <= TOL
        for t in ts:
            t.free()
    # a context whose operands only a GEMV call prepared has nothing a prepped call may reuse
    c2 = beglin_amd.Context(0)
    pk, sc, _ = ref_quant(oracle, 1, weights(1209, 96, inn), 0)
    t = c2.bind(1, pk, sc, 96, inn)
    y = torch.empty((3, 96), device="cuda")
    c2.matmul(t, torch.from_numpy(seeded_normal(1208, (3, inn))).cuda(), y, act=1)
    with pytest.raises(beglin_amd.BglError):
        c2.matmul_prepped(t, y, act=1, M=3)
    c2.sync()
    t.free()
    c2.close()


@pytest.mark.parametrize("kind", [1, 2, 3])
def test_w4a8_batched_prep_equals_fused(torch_dev, oracle, monkeypatch, kind):
    """Several W4A8 columns quantized once up front (k_act_w4a8, then workgroups copying the codes)
    == every workgroup quantizing its launch's columns: both bit-identical to the oracle, at column
    counts that leave a launch of 4 or 8 partly filled."""
    import beglin_amd
    torch = torch_dev
    for inn in (320, 1408, 8960):
        if kind == 3 and inn % 256:
            continue
        out = 136
        w = weights(1200 + kind + inn, out, inn)
        pk, sc, sub = ref_quant(oracle, kind, w, 0)
        for M in (2, 5, 8, 12):
            say("w4a8 prep vs fused", kind, inn, M)
            x = seeded_normal(1210 + M, (M, inn))
            ref = oracle.matmul_sdot(kind, pk, sc, x, sub=sub)
            outs = []
            for flag in ("0", "1"):
                monkeypatch.setenv("BGL_Q_PREP", flag)
                c = beglin_amd.Context(0)
                t = c.bind(kind, pk, sc, out, inn, sub=sub)
                y = torch.full((M, out), float("nan"), dtype=torch.float32, device="cuda")
                c.matmul(t, torch.from_numpy(x).cuda(), y, act=1)
                torch.cuda.synchronize()
                outs.append(y.cpu().numpy())
                t.free(); c.close()
            assert np.array_equal(outs[0].view(np.uint32), ref.view(np.uint32)), (inn, M)
            assert np.array_equal(outs[1].view(np.uint32), ref.view(np.uint32)), (inn, M)


@pytest.mark.parametrize("kind,inn", [(1, 1536), (2, 1024), (3, 1536), (3, 8960), (1, 8960)])
def test_w4a8_matrix_cores_equal_dot4(torch_dev, oracle, monkeypatch, kind, inn):
    """W4A8 at 5..16 columns on the matrix cores (k_gemv_qm) against the dot4 kernel
    (BGL_NO_QMFMA=1) and the oracle, bit for bit: column counts that fill one launch, leave a
    partial one, and leave a 1-4 column remainder for the dot4 kernel (17, 21); a fused group of two
    tensors with biases; columns quantized in the kernel and up front (BGL_Q_PREP=1)."""
    import beglin_amd
    torch = torch_dev
    outs_n = (200, 72)
    ws = [weights(1400 + kind + inn + j, o, inn) for j, o in enumerate(outs_n)]
    refq = [ref_quant(oracle, kind, w, 0) for w in ws]
    biases = [seeded_normal(1410 + j, (o,)) for j, o in enumerate(outs_n)]
    for M in (5, 8, 16, 17, 21):
        say("w4a8 matrix cores", kind, inn, M)
        x = seeded_normal(1420 + M, (M, inn))
        refs = [oracle.matmul_sdot(kind, pk, sc, x, bias=bias, sub=sub) for (pk, sc, sub), bias in zip(refq, biases)]
        for flags in ({}, {"BGL_Q_PREP": "1"}, {"BGL_NO_QMFMA": "1"}):
            for k in ("BGL_Q_PREP", "BGL_NO_QMFMA"):
                monkeypatch.delenv(k, raising=False)
            for k, v in flags.items():
                monkeypatch.setenv(k, v)
            c = beglin_amd.Context(0)
            ts = [c.bind(kind, pk, sc, o, inn, sub=sub) for (pk, sc, sub), o in zip(refq, outs_n)]
            ys = [torch.full((M, o), float("nan"), dtype=torch.float32, device="cuda") for o in outs_n]
            c.matmul_group(ts, torch.from_numpy(x).cuda(), ys, act=beglin_amd.ACT_W4A8,
                           biases=[torch.from_numpy(b).cuda() for b in biases])
            torch.cuda.synchronize()
            for y, ref in zip(ys, refs):
                got = y.cpu().numpy()
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (kind, inn, M, flags, relerr(got, ref))
            for t in ts:
                t.free()
            c.close()


@pytest.mark.parametrize("M", [1, 3, 8, 13])
@pytest.mark.parametrize("inn", [512, 8960])
def test_g256plain_w4a8_bitexact(ctx, torch_dev, oracle, inn, M):
    """The plain-g256 diagnostic kind (q4gemv_g256.h:102-130; bound as the g256sf layout with
    sub-codes 1 and fold factor 1): W4A8 outputs bit-identical to the oracle's row at every M, the
    fused and the up-front-quantized launches alike; decode = (nib - 8) * scale; the kind reads
    back as 10; fusing it with a g256sf tensor is refused (the folds differ)."""
    import beglin_amd
    torch = torch_dev
    out = 200
    say("g256plain", inn, M)
    rng = np.random.default_rng(1300 + inn + M)
    pk = rng.integers(0, 256, (out, inn // 2), dtype=np.uint8)
    ws = (rng.random((out, inn // 256), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = seeded_normal(1310 + M, (M, inn))
    bias = seeded_normal(1320, (out,))
    ref = oracle.matmul_sdot(10, pk, ws, x, bias=bias)
    t = ctx.bind(beglin_amd.K_Q4G256P, pk, ws, out, inn)
    assert t.info()["kind"] == beglin_amd.K_Q4G256P
    y = torch.full((M, out), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matmul(t, torch.from_numpy(x).cuda(), y, act=beglin_amd.ACT_W4A8, bias_dev=torch.from_numpy(bias).cuda())
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), relerr(got, ref)
    if M == 1:
        d = torch.zeros((out, inn), dtype=torch.float32, device="cuda")
        ctx.dequant(t, 0, out, d)
        torch.cuda.synchronize()
        nib = np.empty((out, inn), np.float32)
        nib[:, 0::2] = pk & 15
        nib[:, 1::2] = pk >> 4
        want = (nib - np.float32(8)) * np.repeat(ws, 256, axis=1)
        assert np.array_equal(d.cpu().numpy().view(np.uint32), want.view(np.uint32))
        with pytest.raises(beglin_amd.BglError):
            ctx.matmul(t, torch.from_numpy(x).cuda(), y, act=beglin_amd.ACT_F32)        # W4A8 only
        p2, s2, sub2 = oracle.quantize_g256sf(weights(1330, out, inn))
        t2 = ctx.bind(3, p2, s2, out, inn, sub=sub2)
        with pytest.raises(beglin_amd.BglError):
            ctx.matmul_group([t, t2], torch.from_numpy(x).cuda(), [y, torch.zeros_like(y)], act=beglin_amd.ACT_W4A8)
        t2.free()
    t.free()


@pytest.mark.parametrize("M", [1, 5])
def test_g256plain_separate_quantization_path(torch_dev, oracle, monkeypatch, M):
    """Plain g256 through the separate quantization kernel + the prepared-activation GEMV
    (BGL_NO_FUSED_Q=1, whose fold takes the fold factor from the unit's record): bit-identical to
    the oracle, as through the fused kernel."""
    import beglin_amd
    torch = torch_dev
    say("g256plain separate", M)
    out, inn = 136, 1536
    rng = np.random.default_rng(1400 + M)
    pk = rng.integers(0, 256, (out, inn // 2), dtype=np.uint8)
    ws = (rng.random((out, inn // 256), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = seeded_normal(1410 + M, (M, inn))
    ref = oracle.matmul_sdot(10, pk, ws, x)
    monkeypatch.setenv("BGL_NO_FUSED_Q", "1")
    c = beglin_amd.Context(0)
    t = c.bind(beglin_amd.K_Q4G256P, pk, ws, out, inn)
    y = torch.full((M, out), float("nan"), dtype=torch.float32, device="cuda")
    c.matmul(t, torch.from_numpy(x).cuda(), y, act=beglin_amd.ACT_W4A8)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    t.free(); c.close()
    monkeypatch.delenv("BGL_NO_FUSED_Q", raising=False)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), relerr(got, ref)


def test_read_probe_tensor_limits(ctx, torch_dev):
    """The streaming-read probe (a measurement aid) takes 1-64 single tensors per launch, as a MoE
    gather launch's expert tensors need; more is refused before anything is launched."""
    import beglin_amd
    torch = torch_dev
    gen = torch.Generator(device="cuda").manual_seed(77)
    ts = [ctx.quantize(beglin_amd.K_Q4G32H, torch.randn((64, 256), generator=gen, device="cuda") * 0.02) for _ in range(65)]
    ctx.read_probe(ts[:64])
    ctx.read_probe(ts[:1], nblocks=8, nthreads=64)
    ctx.sync()
    with pytest.raises(beglin_amd.BglError):
        ctx.read_probe(ts)
    for t in ts:
        t.free()


@pytest.mark.parametrize("case", range(24))
def test_w4a8_random_shapes(torch_dev, oracle, case):
    """Seeded random W4A8 shapes, bit for bit against the oracle: kinds 1-3, ragged row counts
    (tiles and 16-row blocks partly filled), K of 1-40 groups, 1-20 columns (the dot4 kernel below
    5 columns, the matrix cores from 5, a dot4 remainder past 16), fused groups of 1-3 tensors
    with and without biases."""
    import beglin_amd
    torch = torch_dev
    rng = np.random.default_rng(3100 + case)
    kind = int(rng.integers(1, 4))
    gq = 256 if kind == 3 else 64
    inn = gq * int(rng.integers(1, 11 if kind == 3 else 41))
    M = int(rng.integers(1, 21))
    ntens = int(rng.integers(1, 4))
    outs = [int(rng.integers(1, 300)) for _ in range(ntens)]
    with_bias = bool(rng.integers(0, 2))
    say("w4a8 random", case, kind, inn, M, outs, with_bias)
    c = beglin_amd.Context(0)
    ts, refs, ys, bds = [], [], [], []
    x = seeded_normal(3200 + case, (M, inn))
    for j, o in enumerate(outs):
        pk, sc, sub = ref_quant(oracle, kind, weights(3300 + 7 * case + j, o, inn), 0)
        b = seeded_normal(3400 + 7 * case + j, (o,)) if with_bias else None
        ts.append(c.bind(kind, pk, sc, o, inn, sub=sub))
        refs.append(oracle.matmul_sdot(kind, pk, sc, x, bias=b, sub=sub))
        ys.append(torch.full((M, o), float("nan"), dtype=torch.float32, device="cuda"))
        bds.append(torch.from_numpy(b).cuda() if b is not None else None)
    c.matmul_group(ts, torch.from_numpy(x).cuda(), ys, act=beglin_amd.ACT_W4A8, biases=bds if with_bias else None)
    torch.cuda.synchronize()
    for y, ref in zip(ys, refs):
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (case, kind, inn, M, outs, relerr(got, ref))
    for t in ts:
        t.free()
    c.close()


@pytest.mark.parametrize("kind", [1, 2, 3])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_w4a8_extreme_columns(torch_dev, oracle, kind, M):
    """W4A8 columns at the edges of fp32, bit for bit against the oracle: all zeros (scale 0),
    negative zeros, subnormals only, values near 1e30, and a mix of 1e-38 and 1e30 in one group;
    on the dot4 kernel (1 column) and the matrix cores (5, 16)."""
    import beglin_amd
    torch = torch_dev
    inn, out = 1024, 136
    say("w4a8 extreme", kind, M)
    pk, sc, sub = ref_quant(oracle, kind, weights(3900 + kind, out, inn), 0)
    x = seeded_normal(3910 + M, (M, inn))
    pats = [np.zeros(inn, np.float32), -np.zeros(inn, np.float32),
            (seeded_normal(3920, (inn,)) * np.float32(1e-40)).astype(np.float32),
            (seeded_normal(3921, (inn,)) * np.float32(1e30)).astype(np.float32),
            np.where(np.arange(inn) % 3 == 0, np.float32(1e30), np.float32(1e-38)).astype(np.float32)]
    # one column: every pattern in turn; several: the patterns in the first columns, normal ones after
    xs = [p[None, :].copy() for p in pats] if M == 1 else [np.concatenate([np.stack(pats), x[len(pats):]])]
    c = beglin_amd.Context(0)
    t = c.bind(kind, pk, sc, out, inn, sub=sub)
    for xi in xs:
        ref = oracle.matmul_sdot(kind, pk, sc, xi, sub=sub)
        y = torch.full((M, out), float("nan"), dtype=torch.float32, device="cuda")
        c.matmul(t, torch.from_numpy(xi).cuda(), y, act=beglin_amd.ACT_W4A8)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(ref)), (kind, M)
        ok = ~np.isnan(ref)
        assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32)), (kind, M, relerr(got, ref))
    t.free()
    c.close()
