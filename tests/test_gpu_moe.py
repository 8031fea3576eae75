"""GPU parity of the expert-sorted MoE gather against the CPU oracle, through the C-ABI.

* bgl_gather_matvec_dev: explicit (x, expert) pairs (ffn_gather / mlx_gpu_qng64_gather_probe,
  mlx_moe.h:89-91) against or_moe_matvec per pair, every expert format, mixed formats, the
  GATE9 fixture (qwen_infer.c:10811-10875), ids outside [0, E) skipped.
* bgl_moe_ffn_dev: the routed SwiGLU FFN with shared experts (moe_ffn_batched,
  qwen_infer.c:5238-5350) against or_moe_ffn_bucketed, routing from or_moe_route, at small sizes
  and at DeepSeek-V2-Lite's shape; graph replay; error paths.
* bgl_moe_route_dev / bgl_moe_layer_dev: the router (double-accumulated scores, softmax, top-K
  with ties to the lowest id, renorm) against or_moe_router_logits + or_moe_route, and the whole
  layer on the device against the oracle pipeline.
Bar: max|y - ref| / max|ref| <= 1e-5 (fp32 arithmetic, summation order differs)."""
import sys

import numpy as np
import pytest

from golden.fixtures import gate9, seeded_normal
from oracle_ffi import moe_decode, moe_ffn, moe_matvec, mxfp4_blocks

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


def weights(seed, out, inn, sigma=0.02):
    w = seeded_normal(seed, (out, inn), sigma)
    w[np.random.default_rng(seed + 1).random(w.shape) < 0.01] *= 8
    return w


def desc(oracle, kind, bits, w):
    """Reference-layout expert descriptor (kind, bits, packed, scales[, bias]) from the oracle
    packers; int4 affine (6) gets seeded random nibbles / scales / biases (any bytes are valid AF
    int4), dense fp16 (7) / fp32 (8) carry the weights themselves."""
    if kind == 6:
        rng = np.random.default_rng(int(abs(w[0, 0]) * 1e9) % (2 ** 31))
        out, inn = w.shape
        pk = rng.integers(0, 256, (out, inn // 2), dtype=np.uint8)
        sc = (rng.random((out, inn // 64), dtype=np.float32) * np.float32(0.01)).astype(np.float32)
        bi = (rng.standard_normal((out, inn // 64), dtype=np.float32) * np.float32(0.04)).astype(np.float32)
        return (6, 4, pk, sc, bi)
    if kind == 7:
        return (7, 16, w.astype(np.float16).view(np.uint16), None)
    if kind == 9:                                   # GGUF MXFP4 blocks: any bytes are valid
        rng = np.random.default_rng(int(abs(w[0, 0]) * 1e9) % (2 ** 31))
        return (9, 4, mxfp4_blocks(rng, w.shape[0], w.shape[1], 118, 124), None)
    if kind == 8:
        return (8, 32, np.ascontiguousarray(w), None)
    if kind == 1:
        p, s = oracle.quantize_q4g64(w)
    elif kind == 2:
        p, s = oracle.quantize_q8g64(w)
    elif kind == 4:
        p, s = oracle.quantize_qng64(w, bits)
    else:
        p, s = oracle.quantize_q4g32h(w)
    return (kind, bits, p, s)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


FORMATS = [(5, 0), (1, 0), (2, 0), (4, 2), (4, 3), (4, 5), (4, 7), (4, 8), (4, 9), (4, 12), (4, 15), (6, 4), (7, 16),
           (8, 32), (9, 4)]


@pytest.mark.parametrize("kind,bits", FORMATS)
def test_gather_matvec_parity(ctx, torch_dev, oracle, kind, bits):
    torch = torch_dev
    E, out, inn, N = 6, 160, 512, 13
    say("gather", kind, bits, E, out, inn, N)
    ds = [desc(oracle, kind, bits, weights(1000 + 10 * e + bits, out, inn)) for e in range(E)]
    idx = np.random.default_rng(7).integers(0, E, N).astype(np.int32)
    idx[idx == 4] = 5                                   # one expert with no pair
    x = seeded_normal(8, (N, inn))
    ex = ctx.bind_experts(ds)
    y = torch.full((N, out), 7.0, dtype=torch.float32, device="cuda")
    ctx.gather_matvec(ex, dev(torch, x), dev(torch, idx), y)
    ctx.sync()
    ref = np.stack([moe_matvec(oracle, ds[idx[z]], out, inn, x[z]) for z in range(N)])
    assert relerr(y.cpu().numpy(), ref) <= TOL
    ex.free()


def test_gather_mixed_formats(ctx, torch_dev, oracle):
    torch = torch_dev
    fm = [(5, 0), (2, 0), (4, 7), (4, 15), (1, 0), (4, 2), (5, 0), (4, 10), (6, 4), (7, 16), (8, 32)]
    E, out, inn, N = len(fm), 200, 768, 41
    say("gather mixed", E, out, inn, N)
    ds = [desc(oracle, k, b, weights(2000 + e, out, inn)) for e, (k, b) in enumerate(fm)]
    idx = np.random.default_rng(9).integers(0, E, N).astype(np.int32)
    x = seeded_normal(10, (N, inn))
    ex = ctx.bind_experts(ds)
    y = torch.zeros((N, out), dtype=torch.float32, device="cuda")
    ctx.gather_matvec(ex, dev(torch, x), dev(torch, idx), y)
    ctx.sync()
    ref = np.stack([moe_matvec(oracle, ds[idx[z]], out, inn, x[z]) for z in range(N)])
    assert relerr(y.cpu().numpy(), ref) <= TOL
    info = ex.info()
    assert info["out"] == out and info["inn"] == inn and info["kind"] == 0
    ex.free()


def test_gate9_gather(ctx, torch_dev, oracle):
    """GATE9 (qwen_infer.c:10811-10875): E=4, out=8, in=128, n=7, pairs {0,3,1,2,0,3}."""
    torch = torch_dev
    g = gate9()
    say("gate9")
    ds = [(4, 7) + oracle.quantize_qng64_gguf(g["w"][e], 7) for e in range(g["E"])]
    ex = ctx.bind_experts(ds)
    y = torch.zeros((len(g["idx"]), g["out"]), dtype=torch.float32, device="cuda")
    ctx.gather_matvec(ex, dev(torch, g["x"]), dev(torch, g["idx"]), y)
    ctx.sync()
    ref = np.stack([moe_matvec(oracle, ds[e], g["out"], g["inn"], g["x"][z]) for z, e in enumerate(g["idx"])])
    assert relerr(y.cpu().numpy(), ref) <= TOL
    ex.free()


def test_gather_invalid_ids_skipped(ctx, torch_dev, oracle):
    torch = torch_dev
    E, out, inn = 3, 64, 256
    say("gather invalid ids")
    ds = [desc(oracle, 5, 0, weights(3000 + e, out, inn)) for e in range(E)]
    idx = np.array([0, -1, 2, 3, 1, 2], np.int32)
    x = seeded_normal(11, (len(idx), inn))
    ex = ctx.bind_experts(ds)
    y = torch.full((len(idx), out), 3.5, dtype=torch.float32, device="cuda")
    ctx.gather_matvec(ex, dev(torch, x), dev(torch, idx), y)
    ctx.sync()
    yh = y.cpu().numpy()
    assert np.all(yh[1] == 3.5) and np.all(yh[3] == 3.5)
    for z in (0, 2, 4, 5):
        assert relerr(yh[z], moe_matvec(oracle, ds[idx[z]], out, inn, x[z])) <= TOL
    ex.free()


def moe_setup(oracle, seed, E, H, I, Ish, fmts, down_fmts=None, sh_fmt=(5, 0)):
    gate = [desc(oracle, *fmts[e % len(fmts)], weights(seed + 3 * e, I, H)) for e in range(E)]
    up = [desc(oracle, *fmts[e % len(fmts)], weights(seed + 3 * e + 1, I, H)) for e in range(E)]
    dfm = down_fmts or fmts
    down = [desc(oracle, *dfm[e % len(dfm)], weights(seed + 3 * e + 2, H, I)) for e in range(E)]
    shared = None
    if Ish:
        shared = (desc(oracle, *sh_fmt, weights(seed + 900, Ish, H)), desc(oracle, *sh_fmt, weights(seed + 901, Ish, H)),
                  desc(oracle, *sh_fmt, weights(seed + 902, H, Ish)))
    return gate, up, down, shared


def bind_one(ctx, d):
    k, b, p, sc = d[:4]
    if k == 9:                                      # MXFP4: blocks of 32 values, 17 bytes each
        inn = p.reshape(p.shape[0], -1).shape[1] // 17 * 32
    else:
        inn = p.shape[1] if k in (7, 8) else sc.shape[1] * (32 if k == 5 else 64)
    return ctx.bind(k, p, sc, p.shape[0], inn, bits=b, sub=d[4] if len(d) > 4 else None)


def run_moe(ctx, torch, gate, up, down, shared, x, idx, w):
    g, u, d = ctx.bind_experts(gate), ctx.bind_experts(up), ctx.bind_experts(down)
    sh = None
    if shared:
        sh = tuple(bind_one(ctx, d) for d in shared)
    out = torch.zeros((x.shape[0], x.shape[1]), dtype=torch.float32, device="cuda")
    ctx.moe_ffn(g, u, d, sh, dev(torch, x), dev(torch, idx), dev(torch, w), out)
    ctx.sync()
    res = out.cpu().numpy()
    for t in (g, u, d) + (sh or ()):
        t.free()
    return res


@pytest.mark.parametrize("T,Ish,renorm", [(1, 384, False), (5, 0, True), (33, 384, True), (64, 128, False)])
def test_moe_ffn_parity(ctx, torch_dev, oracle, T, Ish, renorm):
    torch = torch_dev
    E, H, I, K = 16, 256, 192, 4
    say("moe_ffn", T, Ish, renorm)
    gate, up, down, shared = moe_setup(oracle, 4000 + T, E, H, I, Ish, [(5, 0)])
    x = seeded_normal(50 + T, (T, H))
    idx, w = oracle.route(seeded_normal(60 + T, (T, E)), K, renorm)
    got = run_moe(ctx, torch, gate, up, down, shared, x, idx, w)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    assert relerr(got, ref) <= TOL


def test_moe_ffn_mixed_precision(ctx, torch_dev, oracle):
    """Per-expert precision as the mixed-precision registration allows (q4g32h, int8, qNg64, AF
    int4 affine, dense fp16 / fp32)."""
    torch = torch_dev
    E, H, I, K, T, Ish = 12, 320, 256, 3, 9, 256
    say("moe_ffn mixed", E, H, I, K, T)
    fm = [(5, 0), (2, 0), (4, 7), (4, 9), (6, 4), (4, 15), (7, 16), (8, 32), (4, 11)]
    gate, up, down, shared = moe_setup(oracle, 5000, E, H, I, Ish, fm, down_fmts=fm[::-1], sh_fmt=(2, 0))
    x = seeded_normal(70, (T, H))
    idx, w = oracle.route(seeded_normal(71, (T, E)), K, True)
    got = run_moe(ctx, torch, gate, up, down, shared, x, idx, w)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    assert relerr(got, ref) <= TOL
    naive = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w, naive=True)
    assert relerr(got, naive) <= TOL


def test_moe_ffn_deepseek_v2_lite_shape(ctx, torch_dev, oracle):
    """DeepSeek-V2-Lite routed layer: E=64, hidden 2048, expert inter 1408, top-6, 2 shared
    experts (inter 2816); experts quantized on the device, mixed per-expert precision."""
    torch = torch_dev
    E, H, I, K, T, Ish = 64, 2048, 1408, 6, 8, 2816
    say("moe_ffn dsv2-lite", E, H, I, K, T)
    fm = [(5, 0), (2, 0), (4, 7), (4, 9), (4, 12), (4, 15)]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(123)
    descs = {"gate": [], "up": [], "down": []}
    tens = {"gate": [], "up": [], "down": []}
    for e in range(E):
        k, b = fm[e % len(fm)]
        for name, (o, i) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            wd = torch.randn((o, i), generator=gen, device="cuda") * 0.02
            t, (p, s, _) = ctx.quantize(k, wd, bits=b, want_ref=True)
            descs[name].append((k, b, p, s))
            tens[name].append(t)
            del wd
    sh_d, sh_t = [], []
    for (o, i) in ((Ish, H), (Ish, H), (H, Ish)):
        wd = torch.randn((o, i), generator=gen, device="cuda") * 0.02
        t, (p, s, _) = ctx.quantize(5, wd, want_ref=True)
        sh_d.append((5, 0, p, s)); sh_t.append(t)
    g = ctx.experts_from_tensors(tens["gate"])
    u = ctx.experts_from_tensors(tens["up"])
    d = ctx.experts_from_tensors(tens["down"])
    x = seeded_normal(80, (T, H))
    idx, w = oracle.route(seeded_normal(81, (T, E)), K, False)
    out = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    ctx.moe_ffn(g, u, d, tuple(sh_t), dev(torch, x), dev(torch, idx), dev(torch, w), out)
    ctx.sync()
    ref = moe_ffn(oracle, descs["gate"], descs["up"], descs["down"], tuple(sh_d), H, I, x, idx, w)
    assert relerr(out.cpu().numpy(), ref) <= TOL
    for t in [g, u, d] + sh_t:
        t.free()


def test_moe_graph_replays_match_eager(ctx, torch_dev, oracle):
    import beglin_amd
    torch = torch_dev
    E, H, I, K, T, Ish = 8, 256, 128, 2, 6, 128
    say("moe graph")
    gate, up, down, shared = moe_setup(oracle, 6000, E, H, I, Ish, [(5, 0), (4, 9)])
    x = dev(torch, seeded_normal(90, (T, H)))
    idx_h, w_h = oracle.route(seeded_normal(91, (T, E)), K, True)
    idx, w = dev(torch, idx_h), dev(torch, w_h)
    s = torch.cuda.Stream()
    gc = beglin_amd.Context(0, stream=s.cuda_stream)
    g, u, d = gc.bind_experts(gate), gc.bind_experts(up), gc.bind_experts(down)
    sh = tuple(bind_one(gc, d) for d in shared)
    out = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    with torch.cuda.stream(s):
        gc.moe_ffn(g, u, d, sh, x, idx, w, out)          # eager call sizes every scratch buffer
    gc.sync()
    eager = out.cpu().numpy().copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        gc.moe_ffn(g, u, d, sh, x, idx, w, out)
    for r in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager), f"replay {r}"
        with torch.cuda.stream(s):
            gc.moe_ffn(g, u, d, sh, x, idx, w, out)       # eager work between replays
        gc.sync()
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x.cpu().numpy(), idx_h, w_h)
    assert relerr(eager, ref) <= TOL
    for t in (g, u, d) + sh:
        t.free()
    gc.close()


ROUTE_CASES = [(1, 64, 6, False, False), (7, 64, 6, True, True), (64, 64, 6, False, True), (5, 8, 2, True, False),
               (3, 160, 8, False, True), (2, 256, 16, True, True)]


@pytest.mark.parametrize("T,E,K,renorm,bias", ROUTE_CASES)
def test_moe_route_parity(ctx, torch_dev, oracle, T, E, K, renorm, bias):
    """Device router (bgl_moe_route_dev) against or_moe_router_logits + or_moe_route: the chosen
    experts equal in selection order, the weights within 1e-6.  Hidden sizes: 2048 (one round of
    router loads), 256 (a partly used round) and 4160 (three rounds, the last one 64 values)."""
    torch = torch_dev
    H = {64: 2048, 160: 4160}.get(E, 256)
    say("route", T, E, K, renorm, bias)
    w = seeded_normal(900 + E, (E, H), 0.05)
    x = seeded_normal(901 + T, (T, H))
    b = seeded_normal(902, (E,), 0.1) if bias else None
    ridx, rw = oracle.route(oracle.router_logits(w, x, b), K, renorm)
    idx = torch.full((T, K), -1, dtype=torch.int32, device="cuda")
    wd = torch.full((T, K), float("nan"), device="cuda")
    ctx.moe_route(dev(torch, w), dev(torch, x), K, idx, wd, router_b=dev(torch, b) if bias else None, renorm=renorm)
    ctx.sync()
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(wd.cpu().numpy(), rw, rtol=1e-6, atol=1e-9)
    if renorm:
        np.testing.assert_allclose(wd.cpu().numpy().sum(axis=1), 1.0, rtol=1e-6)


def test_moe_route_ties_go_to_lowest_id(ctx, torch_dev, oracle):
    """Identical router rows give identical probabilities; the repeated strict maximum
    (moe_top_k_select, qwen_infer.c:3514-3521) takes the lowest expert id first."""
    torch = torch_dev
    E, H, K, T = 64, 256, 6, 4
    say("route ties")
    x = seeded_normal(911, (T, H))
    w = seeded_normal(910, (E, H), 0.05)
    w[3] = x[0] * np.float32(0.02)                  # the top score of token 0
    w[40] = w[3]; w[17] = w[3]
    w[50] = w[9]; w[21] = w[9]
    ridx, rw = oracle.route(oracle.router_logits(w, x), K, False)
    assert list(ridx[0][:3]) == [3, 17, 40]
    idx = torch.full((T, K), -1, dtype=torch.int32, device="cuda")
    wd = torch.zeros((T, K), device="cuda")
    ctx.moe_route(dev(torch, w), dev(torch, x), K, idx, wd)
    ctx.sync()
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(wd.cpu().numpy(), rw, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("T,renorm", [(1, False), (9, True), (64, False)])
def test_moe_layer_parity(ctx, torch_dev, oracle, T, renorm):
    """bgl_moe_layer_dev (router + routed FFN + shared experts on the device) against the oracle's
    router logits, routing and bucketed FFN."""
    torch = torch_dev
    E, H, I, K, Ish = 16, 256, 192, 4, 128
    say("moe_layer", T, renorm)
    gate, up, down, shared = moe_setup(oracle, 6100, E, H, I, Ish, [(5, 0), (2, 0), (4, 7)])
    x = seeded_normal(6101 + T, (T, H))
    rwt = seeded_normal(6102, (E, H), 0.05)
    b = seeded_normal(6103, (E,), 0.1)
    idx, w = oracle.route(oracle.router_logits(rwt, x, b), K, renorm)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    g, u, d = ctx.bind_experts(gate), ctx.bind_experts(up), ctx.bind_experts(down)
    sh = tuple(bind_one(ctx, dd) for dd in shared)
    out = torch.full((T, H), float("nan"), device="cuda")
    ctx.moe_layer(dev(torch, rwt), g, u, d, sh, dev(torch, x), K, out, router_b=dev(torch, b), renorm=renorm)
    ctx.sync()
    assert relerr(out.cpu().numpy(), ref) <= TOL
    for t in (g, u, d) + sh:
        t.free()


def test_moe_layer_fused_router_ties_and_wide(ctx, torch_dev, oracle):
    """The whole-layer entry's router for up to 16 tokens (top-K and bucketing in one workgroup)
    over E = 160 experts (a partly
    filled third block of 64 scores per lane), K = 8, renorm, and tied router rows (identical
    probabilities: the lowest expert id is picked first) -- the outputs equal the oracle's layer,
    whose FFN differs for every expert, so a wrong pick or tie order shows."""
    torch = torch_dev
    E, H, I, K, Ish, T = 160, 256, 64, 8, 64, 3
    say("moe_layer fused router", E, K, T)
    gate, up, down, shared = moe_setup(oracle, 6200, E, H, I, Ish, [(5, 0), (2, 0), (4, 7)])
    x = seeded_normal(6201, (T, H))
    rwt = seeded_normal(6202, (E, H), 0.05)
    rwt[3] = x[0] * np.float32(0.03)                     # token 0's top scores, tied three ways
    rwt[140] = rwt[3]; rwt[77] = rwt[3]
    rwt[150] = rwt[9]; rwt[21] = rwt[9]
    idx, w = oracle.route(oracle.router_logits(rwt, x), K, True)
    assert list(idx[0][:3]) == [3, 77, 140]
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    g, u, d = ctx.bind_experts(gate), ctx.bind_experts(up), ctx.bind_experts(down)
    sh = tuple(bind_one(ctx, dd) for dd in shared)
    out = torch.full((T, H), float("nan"), device="cuda")
    ctx.moe_layer(dev(torch, rwt), g, u, d, sh, dev(torch, x), K, out, renorm=True)
    ctx.sync()
    assert relerr(out.cpu().numpy(), ref) <= TOL
    for t in (g, u, d) + sh:
        t.free()


@pytest.mark.parametrize("merge,T", [("auto", 5), ("1", 5), ("auto", 20)])
def test_moe_layer_graph_replays_match_eager(torch_dev, oracle, monkeypatch, merge, T):
    """The whole layer (router, top-K + bucketing, FFN, shared experts) replayed
    from a graph: every replay, with eager calls in between, equals the eager result bit for bit
    (merge "1": the routed and shared gate+up in one launch, k_moe_x2; T = 20: the Q4G32H shared
    experts run as the matrix-core MLP block)."""
    import beglin_amd
    torch = torch_dev
    E, H, I, K, Ish = 16, 256, 128, 4, 128
    say("moe_layer graph", merge, T)
    if merge == "auto":
        monkeypatch.delenv("BGL_MOE_MERGE", raising=False)
    else:
        monkeypatch.setenv("BGL_MOE_MERGE", merge)
    gate, up, down, shared = moe_setup(oracle, 6300, E, H, I, Ish, [(5, 0), (4, 9)])
    x = dev(torch, seeded_normal(6301, (T, H)))
    rwt = dev(torch, seeded_normal(6302, (E, H), 0.05))
    s = torch.cuda.Stream()
    gc = beglin_amd.Context(0, stream=s.cuda_stream)
    g, u, d = gc.bind_experts(gate), gc.bind_experts(up), gc.bind_experts(down)
    sh = tuple(bind_one(gc, dd) for dd in shared)
    out = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    with torch.cuda.stream(s):
        gc.moe_layer(rwt, g, u, d, sh, x, K, out)
    gc.sync()
    eager = out.cpu().numpy().copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        gc.moe_layer(rwt, g, u, d, sh, x, K, out)
    for r in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager), f"replay {r}"
        with torch.cuda.stream(s):
            gc.moe_layer(rwt, g, u, d, sh, x, K, out)
        gc.sync()
    idx, w = oracle.route(oracle.router_logits(rwt.cpu().numpy(), x.cpu().numpy()), K, False)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x.cpu().numpy(), idx, w)
    assert relerr(eager, ref) <= TOL
    for t in (g, u, d) + sh:
        t.free()
    gc.close()


def test_moe_route_error_paths(ctx, torch_dev):
    import beglin_amd
    torch = torch_dev
    x = torch.zeros((2, 256), device="cuda")
    idx = torch.zeros((2, 8), dtype=torch.int32, device="cuda")
    w = torch.zeros((2, 8), device="cuda")
    with pytest.raises(beglin_amd.BglError):
        ctx.moe_route(torch.zeros((4, 256), device="cuda"), x, 8, idx, w)        # K > E
    with pytest.raises(beglin_amd.BglError):
        ctx.moe_route(torch.zeros((300, 256), device="cuda"), x, 8, idx, w)      # E > 256
    with pytest.raises(beglin_amd.BglError):
        ctx.moe_route(torch.zeros((8, 254), device="cuda"), torch.zeros((2, 254), device="cuda"), 2, idx, w)   # in % 4
    ctx.sync()


def test_moe_error_paths(ctx, torch_dev, oracle):
    import beglin_amd
    torch = torch_dev
    E, H, I = 4, 128, 64
    gate, up, down, shared = moe_setup(oracle, 7000, E, H, I, 64, [(5, 0)])
    g, u, d = ctx.bind_experts(gate), ctx.bind_experts(up), ctx.bind_experts(down)
    x = torch.zeros((2, H), device="cuda")
    out = torch.zeros((2, H), device="cuda")
    idx17 = torch.zeros((2, 17), dtype=torch.int32, device="cuda")
    w17 = torch.zeros((2, 17), device="cuda")
    with pytest.raises(beglin_amd.BglError):
        ctx.moe_ffn(g, u, d, None, x, idx17, w17, out)                 # top-K above 16
    idx = torch.zeros((2, 2), dtype=torch.int32, device="cuda")
    w = torch.zeros((2, 2), device="cuda")
    with pytest.raises(beglin_amd.BglError):
        ctx.moe_ffn(g, d, d, None, x, idx, w, out)                     # up shaped like down
    single = ctx.bind(*gate[0][:1], gate[0][2], gate[0][3], I, H)
    with pytest.raises(beglin_amd.BglError):
        ctx.moe_ffn(single, u, d, None, x, idx, w, out)               # not an expert stack
    with pytest.raises(beglin_amd.BglError):
        ctx.moe_ffn(g, u, d, (single, None, None), x, idx, w, out)    # partial shared set
    wg = weights(7100, 64, 256)
    p, sc, sub = oracle.quantize_g256sf(wg)
    t256 = ctx.bind(3, p, sc, 64, 256, sub=sub)
    with pytest.raises(beglin_amd.BglError):
        ctx.experts_from_tensors([t256])                              # W4A8-only format
    ctx.sync()
    for t in (g, u, d, single, t256):
        t.free()


@pytest.mark.parametrize("T,tr", [(1, 0), (6, 0), (21, 0), (6, 16), (21, 16), (1, 64)])
def test_moe_x_matches_prep_path(torch_dev, oracle, monkeypatch, T, tr):
    """The gather that makes its activation records in the kernel (k_moe_x) against the prep
    kernel + k_moe_gemv path and the oracle: few experts so segments run 1..12 columns (chunks of
    4 and a single last column), hidden 320 (a partial last pass of 256 values), inter 192 (a
    partly filled slot), shared experts over T > 4 columns in segments; workgroups of whole tiles
    and of 16 rows (tr: forced width, 0 = the launch's own choice)."""
    import beglin_amd
    torch = torch_dev
    E, H, I, K, Ish = 4, 320, 192, 2, 320
    say("moe_x vs prep", T, tr)
    fm = [(5, 0), (2, 0), (4, 7), (4, 15)]
    gate, up, down, shared = moe_setup(oracle, 6000 + T, E, H, I, Ish, fm, down_fmts=fm[::-1], sh_fmt=(4, 12))
    x = seeded_normal(90 + T, (T, H))
    idx, w = oracle.route(seeded_normal(91 + T, (T, E)), K, True)
    outs = []
    for flag in ("0", "1"):
        monkeypatch.setenv("BGL_NO_MOE_X", flag)
        if tr:
            monkeypatch.setenv("BGL_FORCE_TR", str(tr))
        else:
            monkeypatch.delenv("BGL_FORCE_TR", raising=False)
        c = beglin_amd.Context(0)
        outs.append(run_moe(c, torch, gate, up, down, shared, x, idx, w))
        c.close()
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    assert relerr(outs[0], ref) <= TOL and relerr(outs[1], ref) <= TOL and relerr(outs[0], outs[1]) <= 2 * TOL


@pytest.mark.parametrize("T,sh_fmt", [(16, (2, 0)), (21, (4, 10)), (64, (5, 0)), (40, (4, 12))])
def test_moe_shared_on_matrix_cores(torch_dev, oracle, monkeypatch, T, sh_fmt):
    """From 16 tokens on, shared experts in a format the matrix cores decode exactly (int8, int4 g32,
    qNg64 n <= 10) run as a dense MLP block on the matrix cores (gate+up, SwiGLU, down) and the
    combine adds their rows; n = 12 stays in the exact-digit gathers.  Both against the oracle's FFN
    and against the gathers alone (BGL_NO_MFMA=1); hidden 320 (a partial pass of 256), shared width
    320, routed experts in mixed formats."""
    import beglin_amd
    torch = torch_dev
    E, H, I, K, Ish = 6, 320, 192, 2, 320
    say("moe shared matrix cores", T, sh_fmt)
    fm = [(5, 0), (2, 0), (4, 7), (4, 15)]
    gate, up, down, shared = moe_setup(oracle, 6300 + T, E, H, I, Ish, fm, down_fmts=fm[::-1], sh_fmt=sh_fmt)
    x = seeded_normal(6310 + T, (T, H))
    idx, w = oracle.route(seeded_normal(6320 + T, (T, E)), K, True)
    outs = []
    for flag in ("0", "1"):
        monkeypatch.setenv("BGL_NO_MFMA", flag)
        c = beglin_amd.Context(0)
        outs.append(run_moe(c, torch, gate, up, down, shared, x, idx, w))
        c.close()
    monkeypatch.delenv("BGL_NO_MFMA", raising=False)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    assert relerr(outs[0], ref) <= TOL and relerr(outs[1], ref) <= TOL and relerr(outs[0], outs[1]) <= 2 * TOL


@pytest.mark.parametrize("T", [1, 3, 6, 13])
def test_moe_merged_gate_up_equals_two_launches(torch_dev, oracle, monkeypatch, T):
    """The routed and the shared gate+up in one launch (k_moe_x2; past 4 tokens the shared columns
    run in segments of 4, the last one partial at T = 6 and 13).  With the workgroup shape pinned
    (whole tiles, 4 waves) the merged launch gives the same bits as the two separate launches, and
    both equal the oracle's FFN."""
    import beglin_amd
    torch = torch_dev
    E, H, I, K, Ish = 4, 320, 192, 2, 320
    say("moe merged gate+up", T)
    fm = [(5, 0), (2, 0), (4, 7), (4, 15)]
    gate, up, down, shared = moe_setup(oracle, 6400 + T, E, H, I, Ish, fm, down_fmts=fm[::-1], sh_fmt=(4, 12))
    x = seeded_normal(6410 + T, (T, H))
    idx, w = oracle.route(seeded_normal(6420 + T, (T, E)), K, True)
    outs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("BGL_MOE_MERGE", flag)
        monkeypatch.setenv("BGL_FORCE_TR", "64")
        monkeypatch.setenv("BGL_X_WAVES", "4")
        c = beglin_amd.Context(0)
        outs.append(run_moe(c, torch, gate, up, down, shared, x, idx, w))
        c.close()
    monkeypatch.delenv("BGL_MOE_MERGE", raising=False)
    monkeypatch.delenv("BGL_FORCE_TR", raising=False)
    monkeypatch.delenv("BGL_X_WAVES", raising=False)
    assert np.array_equal(np.asarray(outs[0]).view(np.uint32), np.asarray(outs[1]).view(np.uint32))
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    assert relerr(outs[0], ref) <= TOL


@pytest.mark.parametrize("T,tr", [(9, 64), (21, 64), (40, 64), (21, 16)])
def test_moe_x_column_groups(torch_dev, oracle, monkeypatch, T, tr):
    """Chunks of 5..8 token columns in one pass over the weights (two column groups of waves,
    record capacity 8) against chunks of at most 4 (capacity 4) and the oracle: four experts so
    segments run 2..20 columns (8-column chunks, then a 4-column or single last chunk), 4 waves
    (two per group), whole tiles and 16-row workgroups, shared experts in segments of 8."""
    import beglin_amd
    torch = torch_dev
    E, H, I, K, Ish = 4, 320, 256, 2, 256
    say("moe_x column groups", T, tr)
    fm = [(5, 0), (2, 0), (4, 7), (4, 15)]
    gate, up, down, shared = moe_setup(oracle, 6600 + T, E, H, I, Ish, fm, down_fmts=fm[::-1], sh_fmt=(4, 12))
    x = seeded_normal(6610 + T, (T, H))
    idx, w = oracle.route(seeded_normal(6620 + T, (T, E)), K, True)
    outs = []
    for cap in ("8", "4"):
        monkeypatch.setenv("BGL_MOE_CAP", cap)
        monkeypatch.setenv("BGL_FORCE_TR", str(tr))
        monkeypatch.setenv("BGL_X_WAVES", "4")
        c = beglin_amd.Context(0)
        outs.append(run_moe(c, torch, gate, up, down, shared, x, idx, w))
        c.close()
    for k in ("BGL_MOE_CAP", "BGL_FORCE_TR", "BGL_X_WAVES"):
        monkeypatch.delenv(k, raising=False)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    assert relerr(outs[0], ref) <= TOL and relerr(outs[1], ref) <= TOL and relerr(outs[0], outs[1]) <= 2 * TOL


# ---------------------------------------------------------------- MXFP4 experts (AF bits = 40)
def test_mxfp4_decode_bitexact(ctx, torch_dev, oracle):
    """moe_decode_af's MXFP4 arm (qwen_infer.c:2584-2595) from the device layout, every exponent
    byte (the subnormal 0 / 1 and the overflowing 255 included) and every code: bit for bit."""
    torch = torch_dev
    import beglin_amd
    say("mxfp4 decode")
    out, inn = 72, 512
    rng = np.random.default_rng(90)
    blk = mxfp4_blocks(rng, out, inn, 0, 256)
    blk[0, :, 0] = np.arange(16, dtype=np.uint8); blk[1, :, 0] = 255 - np.arange(16, dtype=np.uint8)
    t = ctx.bind(beglin_amd.K_MXFP4, blk, None, out, inn)
    y = torch.zeros((out, inn), dtype=torch.float32, device="cuda")
    ctx.dequant(t, 0, out, y)
    ctx.sync()
    got = y.cpu().numpy()
    desc_ = (9, 4, blk, None)
    for r in range(out):
        want = moe_decode(oracle, desc_, out, inn, r, range(inn))
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), r
    t.free()


@pytest.mark.parametrize("T", [1, 6, 21])
def test_mxfp4_moe_ffn(ctx, torch_dev, oracle, T):
    """The routed SwiGLU FFN with MXFP4 experts beside q4g32h and qNg64 ones (one gather launch
    serves every format), shared experts in MXFP4, against the oracle's bucketed FFN."""
    torch = torch_dev
    say("mxfp4 moe ffn", T)
    E, H, I, K, Ish = 6, 320, 192, 2, 128
    fm = [(9, 4), (5, 0), (9, 4), (4, 7), (9, 4), (2, 0)]
    gate, up, down, shared = moe_setup(oracle, 9100 + T, E, H, I, Ish, fm, sh_fmt=(9, 4))
    x = seeded_normal(9110 + T, (T, H))
    idx, w = oracle.route(seeded_normal(9120 + T, (T, E)), K, True)
    got = run_moe(ctx, torch, gate, up, down, shared, x, idx, w)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    assert relerr(got, ref) <= TOL


def test_mxfp4_gpt_oss_shape(ctx, torch_dev, oracle):
    """GPT-OSS-20B's expert shape (hidden 2880 = 45 groups of 64, expert width 2880), 8 experts,
    top-4 over 4 tokens."""
    torch = torch_dev
    say("mxfp4 gpt-oss shape")
    E, H, I, K, T = 8, 2880, 2880, 4, 4
    gate, up, down, _ = moe_setup(oracle, 9200, E, H, I, 0, [(9, 4)])
    x = seeded_normal(9210, (T, H))
    idx, w = oracle.route(seeded_normal(9220, (T, E)), K, True)
    got = run_moe(ctx, torch, gate, up, down, None, x, idx, w)
    ref = moe_ffn(oracle, gate, up, down, None, H, I, x, idx, w)
    assert relerr(got, ref) <= TOL


def test_mxfp4_refusals(torch_dev, oracle, monkeypatch):
    """MXFP4 runs in the in-kernel-digit gather only: a dense GEMV on it, a gather forced onto the
    prepared-digit kernel, and a launch that also holds an AF int4 expert are refused."""
    import beglin_amd
    torch = torch_dev
    say("mxfp4 refusals")
    E, H, I, K, T = 2, 256, 128, 1, 3
    c = beglin_amd.Context(0)
    blk = mxfp4_blocks(np.random.default_rng(93), 64, H, 118, 124)
    t = c.bind(beglin_amd.K_MXFP4, blk, None, 64, H)
    with pytest.raises(beglin_amd.BglError):
        c.matmul(t, dev(torch, seeded_normal(94, (1, H))), torch.zeros((1, 64), device="cuda"))
    t.free()
    x = seeded_normal(95, (T, H))
    idx, w = oracle.route(seeded_normal(96, (T, E)), K, True)
    gate, up, down, _ = moe_setup(oracle, 9300, E, H, I, 0, [(9, 4), (6, 4)])
    with pytest.raises(beglin_amd.BglError):
        run_moe(c, torch, gate, up, down, None, x, idx, w)
    c.close()
    monkeypatch.setenv("BGL_NO_MOE_X", "1")
    c = beglin_amd.Context(0)
    gate, up, down, _ = moe_setup(oracle, 9400, E, H, I, 0, [(9, 4)])
    with pytest.raises(beglin_amd.BglError):
        run_moe(c, torch, gate, up, down, None, x, idx, w)
    c.close()
    monkeypatch.delenv("BGL_NO_MOE_X", raising=False)


@pytest.mark.parametrize("case", range(12))
def test_moe_ffn_random_configs(ctx, torch_dev, oracle, case):
    """Seeded random routed FFN configurations against the oracle (<= 1e-5): expert count, top-K,
    token count (1..70: the in-kernel gathers, their 8-column chunks and the matrix-core shared
    experts from 16 tokens), hidden / expert sizes in whole 64-groups, a per-expert mix of the
    gather formats (int4 g32 / g64, int8, qNg64 n = 2..15, MXFP4), shared experts or none, with
    and without renormalised weights."""
    torch = torch_dev
    rng = np.random.default_rng(4200 + case)
    E = int(rng.integers(4, 33))
    K = int(rng.integers(1, min(E, 8) + 1))
    T = int(rng.integers(1, 71))
    H = 64 * int(rng.integers(2, 9))
    I = 64 * int(rng.integers(2, 9))
    Ish = 64 * int(rng.integers(0, 5))
    pool = [(5, 0), (1, 0), (2, 0), (9, 40)] + [(4, n) for n in range(2, 16)]
    fm = [pool[int(i)] for i in rng.integers(0, len(pool), size=int(rng.integers(1, 5)))]
    sh_fmt = pool[int(rng.integers(0, 3))]
    renorm = bool(rng.integers(0, 2))
    say("moe_ffn random", case, E, K, T, H, I, Ish, fm, sh_fmt, renorm)
    gate, up, down, shared = moe_setup(oracle, 4300 + 11 * case, E, H, I, Ish, fm, sh_fmt=sh_fmt)
    x = seeded_normal(4400 + case, (T, H))
    idx, w = oracle.route(seeded_normal(4500 + case, (T, E)), K, renorm)
    got = run_moe(ctx, torch, gate, up, down, shared, x, idx, w)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    assert relerr(got, ref) <= TOL, (case, relerr(got, ref))
