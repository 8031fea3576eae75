"""GPU parity of the one-column fp32-activation GEMV (k_gemv_x, bgl_gemv_x.hip) against the CPU
oracle's double-accumulation product (gemm_qXg64_mt / qng64_matvec_f32 at M=1, q4gemv.h:761-769,
qng64_dense.c:70-79), and against the tile kernel (k_gemv) on the same inputs.

Bar: max|y - ref| / max|ref| <= 1e-5.  Covered: every format the kernel takes (int4 g64, int4 g32
fp16-scale, int8 g64, qNg64 n=2..15, i.e. every merge of the 4-, 2- and 1-bit fields), K of one
group, an odd number of groups (a qNg64 unit with a padded second group), slots only partly filled,
ragged N, every rows-per-workgroup width, workgroups of 1 and 2 waves over a long K (the activation
records copied in several rounds), fused groups of tensors, activation columns of extreme range and
graph replays; workgroups making the activation digits themselves (short K) against the prep
kernel's digits, bit for bit."""
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


def weights(seed, out, inn):
    w = seeded_normal(seed, (out, inn), 0.02)
    w[np.random.default_rng(seed + 1).random(w.shape) < 0.01] *= 8
    if out > 3:
        w[1, :] = 0.0
    return w


def quant(oracle, kind, w, bits):
    if kind == 1:
        return oracle.quantize_q4g64(w)
    if kind == 2:
        return oracle.quantize_q8g64(w)
    if kind == 4:
        return oracle.quantize_qng64(w, bits)
    return oracle.quantize_q4g32h(w)


def gemv(c, torch, kind, bits, pk, sc, out, inn, x, bias=None):
    t = c.bind(kind, pk, sc, out, inn, bits=bits)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    bd = torch.from_numpy(bias).cuda() if bias is not None else None
    y = torch.full((1, out), float("nan"), dtype=torch.float32, device="cuda")
    c.matmul(t, xd, y, bias_dev=bd)
    torch.cuda.synchronize()
    t.free()
    return y.cpu().numpy()[0]


def context(monkeypatch, **env):
    import beglin_amd
    for k in ("BGL_FORCE_TR", "BGL_X_WAVES", "BGL_NO_GEMV_X", "BGL_X_FUSE"):
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, str(v))
    return beglin_amd.Context(0)


FORMATS = [(1, 0), (5, 0), (2, 0)] + [(4, n) for n in range(2, 16)]
SHAPES = [(200, 64), (136, 192), (70, 1408), (264, 4160)]


@pytest.mark.parametrize("kind,bits", FORMATS)
def test_gemv_x_parity(ctx, torch_dev, oracle, kind, bits):
    torch = torch_dev
    for out, inn in SHAPES:
        say("gemv_x", kind, bits, out, inn)
        w = weights(1300 + 17 * kind + bits, out, inn)
        pk, sc = quant(oracle, kind, w, bits)
        x = seeded_normal(1400 + inn, (1, inn))
        bias = seeded_normal(1401, (out,))
        got = gemv(ctx, torch, kind, bits, pk, sc, out, inn, x, bias)
        ref = oracle.gemm_f32(kind, pk, sc, x, bias=bias, bits=bits)[0]
        e = relerr(got, ref)
        print(f"  max-rel {e:.3e}")
        assert np.all(np.isfinite(got)) and e <= TOL, (out, inn, e)


@pytest.mark.parametrize("TR", [8, 16, 32, 64])
def test_gemv_x_rows_per_workgroup(torch_dev, oracle, monkeypatch, TR):
    """Every rows-per-workgroup width against the oracle and the tile kernel."""
    torch = torch_dev
    out, inn = 330, 2112                                 # 33 groups: the last slot is partly filled
    cases = [(5, 0), (4, 3), (4, 15)]
    c = context(monkeypatch, BGL_FORCE_TR=TR)
    cref = context(monkeypatch, BGL_NO_GEMV_X=1)
    for kind, bits in cases:
        say("gemv_x TR", TR, kind, bits)
        pk, sc = quant(oracle, kind, weights(1500 + bits, out, inn), bits)
        x = seeded_normal(1501, (1, inn))
        a = gemv(c, torch, kind, bits, pk, sc, out, inn, x)
        b = gemv(cref, torch, kind, bits, pk, sc, out, inn, x)
        ref = oracle.gemm_f32(kind, pk, sc, x, bits=bits)[0]
        assert relerr(a, ref) <= TOL and relerr(b, ref) <= TOL and relerr(a, b) <= 2 * TOL
    c.close(); cref.close()


@pytest.mark.parametrize("waves", [1, 2])
def test_gemv_x_long_k_few_waves(torch_dev, oracle, monkeypatch, waves):
    """Workgroups of 1-2 waves over K = 8192 / 14336: more record pieces than one round of loads
    per thread covers, and more groups than threads (the scale copy loop)."""
    torch = torch_dev
    c = context(monkeypatch, BGL_X_WAVES=waves)
    for kind, bits, out, inn in [(4, 2, 96, 14336), (2, 0, 64, 8192), (4, 9, 128, 8192)]:
        say("gemv_x waves", waves, kind, bits, inn)
        pk, sc = quant(oracle, kind, weights(1600 + bits, out, inn), bits)
        x = seeded_normal(1601, (1, inn))
        got = gemv(c, torch, kind, bits, pk, sc, out, inn, x)
        assert relerr(got, oracle.gemm_f32(kind, pk, sc, x, bits=bits)[0]) <= TOL
    c.close()


def test_gemv_x_activation_range(ctx, torch_dev, oracle):
    """Groups spanning 1e-30..1e30, all-zero groups and a group with a single non-zero element."""
    torch = torch_dev
    out, inn = 192, 1024
    say("gemv_x activation range")
    pk, sc = quant(oracle, 4, weights(1700, out, inn), 11)
    x = seeded_normal(1701, (1, inn))
    x[0, :64] *= np.float32(1e30)
    x[0, 64:128] *= np.float32(1e-30)
    x[0, 128:256] = 0.0
    x[0, 256:320] = 0.0
    x[0, 300] = -2.5
    x[0, 320:] *= np.exp(np.linspace(-6, 6, inn - 320)).astype(np.float32)
    got = gemv(ctx, torch, 4, 11, pk, sc, out, inn, x)
    ref = oracle.gemm_f32(4, pk, sc, x, bits=11)[0]
    assert np.all(np.isfinite(got)) and relerr(got, ref) <= TOL


def test_gemv_x_fused_group(ctx, torch_dev, oracle):
    """Three tensors of one kind in one launch (different N, biases) == the oracle per tensor."""
    torch = torch_dev
    inn = 1536
    outs = [512, 136, 72]
    say("gemv_x group")
    x = seeded_normal(1800, (1, inn))
    xd = torch.from_numpy(x).cuda()
    ts, ys, bs, refs = [], [], [], []
    for i, o in enumerate(outs):
        pk, sc = oracle.quantize_qng64(weights(1801 + i, o, inn), 6)
        b = seeded_normal(1810 + i, (o,))
        ts.append(ctx.bind(4, pk, sc, o, inn, bits=6))
        ys.append(torch.full((1, o), float("nan"), device="cuda"))
        bs.append(torch.from_numpy(b).cuda())
        refs.append(oracle.gemm_f32(4, pk, sc, x, bias=b, bits=6))
    ctx.matmul_group(ts, xd, ys, biases=bs)
    torch.cuda.synchronize()
    for y, r in zip(ys, refs):
        assert relerr(y.cpu().numpy(), r) <= TOL
    for t in ts:
        t.free()


def test_gemv_x_graph_replays_match_eager(torch_dev, oracle):
    import beglin_amd
    torch = torch_dev
    out, inn = 520, 4096
    say("gemv_x graph")
    pk, sc = oracle.quantize_q4g32h(weights(1900, out, inn))
    s = torch.cuda.Stream()
    gc = beglin_amd.Context(0, stream=s.cuda_stream)
    t = gc.bind(5, pk, sc, out, inn)
    x = torch.from_numpy(seeded_normal(1901, (1, inn))).cuda()
    y = torch.zeros((1, out), device="cuda")
    with torch.cuda.stream(s):
        gc.matmul(t, x, y)
    gc.sync()
    eager = y.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        gc.matmul(t, x, y)
    for r in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), eager), r
        with torch.cuda.stream(s):
            gc.matmul(t, x, y)
        gc.sync()
    assert relerr(eager, oracle.gemm_f32(5, pk, sc, x.cpu().numpy())) <= TOL
    t.free()
    gc.close()


@pytest.mark.parametrize("kind,bits", [(5, 0), (1, 0), (2, 0), (4, 2), (4, 7), (4, 15)])
def test_gemv_x_fused_digits_equal_prepared(torch_dev, oracle, monkeypatch, kind, bits):
    """Workgroups making the activation digits themselves == the prep kernel's digits: the two
    launches give bit-identical outputs (K of one group, a partial last pass of 256 values, and a
    long K; groups of extreme range, zeros and subnormal values)."""
    torch = torch_dev
    cf = context(monkeypatch, BGL_X_FUSE=1)
    cp = context(monkeypatch, BGL_X_FUSE=0)
    for out, inn in [(72, 64), (200, 1408), (136, 4160), (64, 8192)]:
        say("gemv_x fused digits", kind, bits, out, inn)
        pk, sc = quant(oracle, kind, weights(2000 + bits + inn, out, inn), bits)
        x = seeded_normal(2001 + inn, (1, inn))
        if inn >= 1408:
            x[0, :64] *= np.float32(1e30)
            x[0, 64:128] *= np.float32(1e-30)
            x[0, 128:192] = 0.0
            x[0, 192:256] *= np.float32(1e-40)            # subnormal values
        a = gemv(cf, torch, kind, bits, pk, sc, out, inn, x)
        b = gemv(cp, torch, kind, bits, pk, sc, out, inn, x)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (out, inn)
        assert relerr(a, oracle.gemm_f32(kind, pk, sc, x, bits=bits)[0]) <= TOL
    cf.close(); cp.close()


@pytest.mark.parametrize("mode", ["fused", "prep", "tile"])
def test_gemv_x_subnormal_columns(torch_dev, oracle, monkeypatch, mode):
    """Activation columns at the bottom of fp32 through the exact-digit paths (digits made in the
    GEMV, by the prep kernel, and the tile kernel at M = 1 and M = 4): a column of subnormals only
    (every 64-group below 2^-128, where the group scale 2^(e-22) would be below fp32's range), one
    of groups just above and just below 2^-128, and one near 1e-36.  Outputs within 1e-5 of the
    oracle's relative to the column's largest, or, where they are themselves subnormal, within a
    few subnormal spacings; and never all zero."""
    torch = torch_dev
    env = {"fused": {"BGL_X_FUSE": 1}, "prep": {"BGL_X_FUSE": 0}, "tile": {"BGL_NO_GEMV_X": 1}}[mode]
    c = context(monkeypatch, **env)
    out, inn = 136, 1024
    tiny = np.float32(2.0 ** -149)
    for kind, bits in [(1, 0), (5, 0), (2, 0), (4, 7)]:
        pk, sc = quant(oracle, kind, weights(4700 + kind + bits, out, inn), bits)
        base = seeded_normal(4710, (4, inn))
        x = np.empty((4, inn), np.float32)
        x[0] = base[0] * np.float32(1e-40)                              # subnormal only
        x[1] = np.where(np.arange(inn) // 64 % 2 == 0, base[1] * np.float32(1e-38),
                        base[1] * np.float32(1e-40)).astype(np.float32)  # groups above / below 2^-128
        x[2] = base[2] * np.float32(1e-36)
        x[3] = np.round(base[3] * 1000) * tiny                           # small integer multiples of 2^-149
        for M in (1, 4):
            if mode != "tile" and M > 1:
                continue
            say("gemv_x subnormal", mode, kind, bits, M)
            t = c.bind(kind, pk, sc, out, inn, bits=bits)
            for m0 in range(0, 4, M):
                xc = np.ascontiguousarray(x[m0:m0 + M])
                y = torch.full((M, out), float("nan"), dtype=torch.float32, device="cuda")
                c.matmul(t, torch.from_numpy(xc).cuda(), y)
                torch.cuda.synchronize()
                got = y.cpu().numpy()
                ref = oracle.gemm_f32(kind, pk, sc, xc, bits=bits)
                for j in range(M):
                    g, r = got[j].astype(np.float64), ref[j]
                    err = np.abs(g - r)
                    ok = np.all((err <= TOL * np.max(np.abs(r))) | (err <= 16 * float(tiny)))
                    assert np.all(np.isfinite(g)) and ok and np.any(g != 0.0), (kind, bits, M, m0 + j, float(np.max(err)))
            t.free()
    c.close()
