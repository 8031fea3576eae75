"""GPU: the dense MLP block on the device (bgl_mlp_dev; forward_token's gate+up -> swiglu -> down,
qwen_infer.c:1560-1573, swiglu :726-733) against the oracle chain, at Qwen2.5-1.5B (H 1536,
I 8960) and Llama-3.1-8B (H 4096, I 14336) shapes.

* W4A8 (q4g256sf for Qwen, q4g64 for Llama): gate and up are bit-exact GEMVs, the SwiGLU is the
  same float function on both sides (exp rounded once from double), so h equals the oracle's
  or_swiglu of the oracle's g and u bit for bit, and y equals the oracle's W4A8 down projection
  of that h bit for bit.
* fp32 activations (int4 g32 and qNg64 n=5 for Llama, q8g64 for Qwen): h within 1e-5 of the
  oracle's (max-normalised), y within 1e-5 of the oracle's fp32 down projection of the device's
  own h, and the whole chain within 1e-5 of the oracle's.
* One W4A8 column runs the block as a single launch (bgl_mlp_q.hip: the down-projection workgroups
  wait, bounded, for the gate+up workgroups' h): h and y bit-identical to the three-launch path
  (BGL_NO_FUSED_MLP=1) and to the oracle, call after call and across graph replays; a wait forced
  to give up is reported by bgl_ctx_check while every kernel exits normally, and the next call is
  exact again."""
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


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def qdev(ctx, torch, gen, kind, bits, out, inn):
    w = torch.randn((out, inn), generator=gen, device="cuda") * 0.02
    t, ref = ctx.quantize(kind, w, bits=bits, want_ref=True)
    del w
    return t, ref


def run(ctx, torch, ts, x, act):
    M, H = x.shape
    I = ts[0].info()["out"]
    y = torch.full((M, H), float("nan"), device="cuda")
    h = torch.full((M, I), float("nan"), device="cuda")
    ctx.mlp(ts[0], ts[1], ts[2], dev(torch, x), y, act=act, h_dev=h)
    ctx.sync()
    return y.cpu().numpy(), h.cpu().numpy()


# M = 4 and 5: the down projection quantizes its columns up front and that launch forms h too (the
# 5th column runs a one-column launch over that h)
W4A8_CASES = [("qwen", 3, 1536, 8960, 1), ("qwen", 3, 1536, 8960, 4), ("qwen", 3, 1536, 8960, 5),
              ("llama", 1, 4096, 14336, 1), ("llama", 1, 4096, 14336, 8)]


@pytest.mark.parametrize("model,kind,H,I,M", W4A8_CASES)
def test_mlp_w4a8_bitexact(ctx, torch_dev, oracle, model, kind, H, I, M):
    import beglin_amd
    torch = torch_dev
    say("mlp w4a8", model, M)
    gen = torch.Generator(device="cuda").manual_seed(700 + M + H)
    shapes = ((I, H), (I, H), (H, I))
    ts, refs = zip(*[qdev(ctx, torch, gen, kind, 4, o, i) for o, i in shapes])
    x = seeded_normal(710 + M, (M, H))
    y, h = run(ctx, torch, ts, x, beglin_amd.ACT_W4A8)
    g = oracle.matmul_sdot(kind, refs[0][0], refs[0][1], x, sub=refs[0][2])
    u = oracle.matmul_sdot(kind, refs[1][0], refs[1][1], x, sub=refs[1][2])
    hr = oracle.swiglu(g, u)
    assert np.array_equal(h.view(np.uint32), hr.view(np.uint32)), relerr(h, hr)
    yr = oracle.matmul_sdot(kind, refs[2][0], refs[2][1], hr, sub=refs[2][2])
    assert np.array_equal(y.view(np.uint32), yr.view(np.uint32)), relerr(y, yr)
    for t in ts:
        t.free()


F32_CASES = [("llama", 5, 0, 4096, 14336, 1), ("llama", 5, 0, 4096, 14336, 32), ("llama", 4, 5, 4096, 14336, 3),
             ("qwen", 2, 0, 1536, 8960, 1)]


@pytest.mark.parametrize("model,kind,bits,H,I,M", F32_CASES)
def test_mlp_f32(ctx, torch_dev, oracle, model, kind, bits, H, I, M):
    import beglin_amd
    torch = torch_dev
    say("mlp f32", model, kind, bits, M)
    gen = torch.Generator(device="cuda").manual_seed(800 + M + H + bits)
    shapes = ((I, H), (I, H), (H, I))
    ts, refs = zip(*[qdev(ctx, torch, gen, kind, bits, o, i) for o, i in shapes])
    x = seeded_normal(810 + M, (M, H))
    y, h = run(ctx, torch, ts, x, beglin_amd.ACT_F32)
    g = oracle.gemm_f32(kind, refs[0][0], refs[0][1], x, bits=bits)
    u = oracle.gemm_f32(kind, refs[1][0], refs[1][1], x, bits=bits)
    hr = oracle.swiglu(g, u)
    assert relerr(h, hr) <= TOL
    assert relerr(y, oracle.gemm_f32(kind, refs[2][0], refs[2][1], h, bits=bits)) <= TOL
    assert relerr(y, oracle.gemm_f32(kind, refs[2][0], refs[2][1], hr, bits=bits)) <= TOL
    for t in ts:
        t.free()


@pytest.mark.parametrize("H,I,M", [(512, 1024, 16), (4096, 14336, 32), (1536, 8960, 40)])
def test_mlp_matrix_core_swiglu_in_reduce(ctx, torch_dev, oracle, H, I, M):
    """From 16 fp32 columns the gate+up GEMM runs on the matrix cores and its reduce launch forms
    h = silu(g) * u itself.  h must equal SwiGLU (the oracle's, which the GPU's k_swiglu matches bit
    for bit) of the g and u that the same GEMM stores when asked for them, bit for bit: at a K that
    does not split (512: the GEMM stores g and u, the reduce reads them) and at K-split shapes
    (4096, 1536); the whole block to 1e-5 against the oracle."""
    import beglin_amd
    torch = torch_dev
    say("mlp matrix-core swiglu", H, I, M)
    gen = torch.Generator(device="cuda").manual_seed(950 + M + H)
    shapes = ((I, H), (I, H), (H, I))
    ts, refs = zip(*[qdev(ctx, torch, gen, 5, 0, o, i) for o, i in shapes])
    x = seeded_normal(960 + M, (M, H))
    y, h = run(ctx, torch, ts, x, beglin_amd.ACT_F32)
    gd = torch.empty((M, I), device="cuda")
    ud = torch.empty((M, I), device="cuda")
    ctx.matmul_group([ts[0], ts[1]], dev(torch, x), [gd, ud], act=beglin_amd.ACT_F32)
    ctx.sync()
    hs = oracle.swiglu(gd.cpu().numpy(), ud.cpu().numpy())
    assert np.array_equal(h.view(np.uint32), np.asarray(hs, np.float32).view(np.uint32))
    g = oracle.gemm_f32(5, refs[0][0], refs[0][1], x)
    u = oracle.gemm_f32(5, refs[1][0], refs[1][1], x)
    hr = oracle.swiglu(g, u)
    assert relerr(h, hr) <= TOL
    assert relerr(y, oracle.gemm_f32(5, refs[2][0], refs[2][1], hr)) <= TOL
    for t in ts:
        t.free()


def test_mlp_graph_replay_and_refusals(ctx, torch_dev, oracle):
    """The block captured in a HIP graph replays to the eager result (no host round trip inside);
    shapes that do not form an MLP are refused before anything is launched."""
    import beglin_amd
    torch = torch_dev
    say("mlp graph + refusals")
    s = torch.cuda.Stream()
    c = beglin_amd.Context(0, stream=s.cuda_stream)
    gen = torch.Generator(device="cuda").manual_seed(900)
    H, I = 512, 1024
    ts = [qdev(c, torch, gen, 5, 0, o, i)[0] for o, i in ((I, H), (I, H), (H, I))]
    x = dev(torch, seeded_normal(901, (1, H)))
    y = torch.zeros((1, H), device="cuda")
    with torch.cuda.stream(s):
        c.mlp(ts[0], ts[1], ts[2], x, y)
    c.sync()
    eager = y.cpu().numpy().copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        c.mlp(ts[0], ts[1], ts[2], x, y)
    for r in range(3):
        y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), eager), r
    with pytest.raises(beglin_amd.BglError):
        c.mlp(ts[0], ts[2], ts[2], x, y)                 # up is [H][I]: not an MLP
    with pytest.raises(beglin_amd.BglError):
        c.mlp(ts[0], ts[1], ts[0], x, y)                 # down is [I][H]
    for t in ts:
        t.free()
    c.close()


def bind_mlp(c, torch, oracle, kind, H, I, seed):
    """gate, up, down bound from the oracle's packer bytes (plain g256: random codes and scales)."""
    import beglin_amd
    ts, refs = [], []
    for i, (o, inn) in enumerate(((I, H), (I, H), (H, I))):
        if kind == beglin_amd.K_Q4G256P:
            rng = np.random.default_rng(seed + i)
            pk = rng.integers(0, 256, (o, inn // 2), dtype=np.uint8)
            sc = (rng.random((o, inn // 256), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
            sub = None
        else:
            w = seeded_normal(seed + i, (o, inn), 0.02)
            if kind == 1:
                pk, sc = oracle.quantize_q4g64(w); sub = None
            elif kind == 2:
                pk, sc = oracle.quantize_q8g64(w); sub = None
            else:
                pk, sc, sub = oracle.quantize_g256sf(w)
        ts.append(c.bind(kind, pk, sc, o, inn, sub=sub))
        refs.append((pk, sc, sub))
    return ts, refs


def mlp_ref(oracle, kind, refs, x):
    g = oracle.matmul_sdot(kind, refs[0][0], refs[0][1], x, sub=refs[0][2])
    u = oracle.matmul_sdot(kind, refs[1][0], refs[1][1], x, sub=refs[1][2])
    h = oracle.swiglu(g, u)
    return oracle.matmul_sdot(kind, refs[2][0], refs[2][1], h, sub=refs[2][2]), h


def same_bits(a, b):
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)].view(np.uint32),
                                                                       b[~np.isnan(b)].view(np.uint32))


@pytest.mark.parametrize("kind,H,I", [(3, 1536, 8960), (1, 1536, 8960), (2, 1024, 3072), (10, 512, 2816),
                                      (3, 4096, 14336)])
def test_mlp_single_launch_equals_three_launches(torch_dev, oracle, monkeypatch, kind, H, I):
    """Five calls in a row on one context (the counters return to 0 after every launch), x with a
    NaN in the fourth call: y and h bit-identical to the oracle and to the three-launch path."""
    import beglin_amd
    torch = torch_dev
    say("mlp single launch", kind, H, I)
    monkeypatch.delenv("BGL_NO_FUSED_MLP", raising=False)
    c1 = beglin_amd.Context(0)
    monkeypatch.setenv("BGL_NO_FUSED_MLP", "1")
    c3 = beglin_amd.Context(0)
    monkeypatch.delenv("BGL_NO_FUSED_MLP")
    ts1, refs = bind_mlp(c1, torch, oracle, kind, H, I, 1500 + kind)
    ts3, _ = bind_mlp(c3, torch, oracle, kind, H, I, 1500 + kind)
    for call in range(5):
        x = seeded_normal(1510 + call, (1, H))
        if call == 3:
            x[0, 17] = np.nan
        ys, hs = [], []
        for c, ts in ((c1, ts1), (c3, ts3)):
            y = torch.full((1, H), 7.0, device="cuda")
            h = torch.full((1, I), 7.0, device="cuda")
            c.mlp(ts[0], ts[1], ts[2], dev(torch, x), y, act=beglin_amd.ACT_W4A8, h_dev=h)
            c.check()
            ys.append(y.cpu().numpy()); hs.append(h.cpu().numpy())
        yr, hr = mlp_ref(oracle, kind, refs, x)
        assert same_bits(hs[0], hr) and same_bits(hs[1], hr), (call, relerr(hs[0], hr))
        assert same_bits(ys[0], yr) and same_bits(ys[1], yr), (call, relerr(ys[0], yr))
        assert np.isnan(yr).all() == (call == 3)
    for t in ts1 + ts3:
        t.free()
    c1.close(); c3.close()


@pytest.mark.parametrize("case", range(8))
def test_mlp_single_launch_random_shapes(torch_dev, oracle, case):
    """Seeded random block shapes through the single-launch MLP (q4g64, q8g64, g256sf; hidden and
    intermediate sizes in whole 256-value groups, rows that leave items and down workgroups partly
    filled), two calls in a row: y and h bit-identical to the oracle."""
    import beglin_amd
    torch = torch_dev
    rng = np.random.default_rng(1800 + case)
    kind = int(rng.integers(1, 4))
    H = 256 * int(rng.integers(1, 13))
    I = 256 * int(rng.integers(1, 41))
    say("mlp single launch random", case, kind, H, I)
    c = beglin_amd.Context(0)
    ts, refs = bind_mlp(c, torch, oracle, kind, H, I, 1810 + 3 * case)
    for call in range(2):
        x = seeded_normal(1820 + 2 * case + call, (1, H))
        y = torch.full((1, H), 7.0, device="cuda")
        h = torch.full((1, I), 7.0, device="cuda")
        c.prof_enable(True)
        c.prof_read()
        c.mlp(ts[0], ts[1], ts[2], dev(torch, x), y, act=beglin_amd.ACT_W4A8, h_dev=h)
        c.check()
        assert sum(v[1] for v in c.prof_read().values()) == 1, (case, H, I)   # the single launch ran
        c.prof_enable(False)
        yr, hr = mlp_ref(oracle, kind, refs, x)
        assert same_bits(h.cpu().numpy(), hr), (case, kind, H, I, call)
        assert same_bits(y.cpu().numpy(), yr), (case, kind, H, I, call)
    for t in ts:
        t.free()
    c.close()


def test_mlp_single_launch_graph_replay(torch_dev, oracle):
    """Three MLP blocks (three layers' weights, chained: each block's y feeds the next) captured in
    one graph: every replay, with the program's own eager work in between, equals the eager run."""
    import beglin_amd
    torch = torch_dev
    say("mlp single launch graph")
    s = torch.cuda.Stream()
    c = beglin_amd.Context(0, stream=s.cuda_stream)
    H, I = 1536, 8960
    layers = [bind_mlp(c, torch, oracle, 3, H, I, 1600 + 10 * l)[0] for l in range(3)]
    x = dev(torch, seeded_normal(1650, (1, H)))
    ys = [torch.zeros((1, H), device="cuda") for _ in range(3)]

    def step():
        src = x
        for ts, y in zip(layers, ys):
            c.mlp(ts[0], ts[1], ts[2], src, y, act=beglin_amd.ACT_W4A8)
            src = y

    with torch.cuda.stream(s):
        step()
    c.check()
    eager = [y.cpu().numpy().copy() for y in ys]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step()
    for r in range(4):
        for y in ys:
            y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        c.check()
        for y, e in zip(ys, eager):
            assert np.array_equal(y.cpu().numpy().view(np.uint32), e.view(np.uint32)), r
        with torch.cuda.stream(s):                        # eager work between the replays
            step()
        c.check()
    for ts in layers:
        for t in ts:
            t.free()
    c.close()


def test_mlp_bounded_wait_gives_up(torch_dev, oracle, monkeypatch):
    """The down-projection workgroups' wait is bounded: forced from the host to wait for a count
    that is never reached (BGL_MLP_TEST_TIMEOUT=1, a short BGL_MLP_SPIN), every workgroup still
    exits, bgl_ctx_check reports BGL_E_TIMEOUT, and the next call on the same context -- whose
    counters the timed-out launch returned to 0 -- is bit-exact again."""
    import beglin_amd
    torch = torch_dev
    say("mlp bounded wait")
    monkeypatch.setenv("BGL_MLP_TEST_TIMEOUT", "1")
    monkeypatch.setenv("BGL_MLP_SPIN", "64")
    c = beglin_amd.Context(0)
    monkeypatch.delenv("BGL_MLP_TEST_TIMEOUT")
    monkeypatch.delenv("BGL_MLP_SPIN")
    H, I = 1536, 8960
    ts, refs = bind_mlp(c, torch, oracle, 3, H, I, 1700)
    x = seeded_normal(1710, (1, H))
    y = torch.zeros((1, H), device="cuda")
    c.mlp(ts[0], ts[1], ts[2], dev(torch, x), y, act=beglin_amd.ACT_W4A8)
    with pytest.raises(beglin_amd.BglError) as ei:
        c.check()
    assert ei.value.code == beglin_amd.E_TIMEOUT
    c.check()                                             # the flag was cleared
    yr, _ = mlp_ref(oracle, 3, refs, x)
    for _ in range(2):
        y.zero_()
        c.mlp(ts[0], ts[1], ts[2], dev(torch, x), y, act=beglin_amd.ACT_W4A8)
        c.check()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), yr.view(np.uint32))
    for t in ts:
        t.free()
    c.close()
