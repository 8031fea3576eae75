"""GPU parity of the batched matrix-core GEMM (M >= 16 fp32-activation columns, bgl_mfma.hip)
against the CPU oracle's double-accumulation product (gemm_qXg64_mt / qng64_matmul_f32,
q4gemv.h:761-769, qng64_dense.c:70-79), and against the dot4 kernels on the same inputs.

Bar: max|y - ref| / max|ref| <= 1e-5.  Covered: every format the matrix-core path takes (int4
g64, int4 g32 fp16-scale, int8 g64, qNg64 n=2..10), ragged M (16..100: column tiles of 16 and
launches of 64 columns), K split over workgroups and not, fused groups with bias, activation
columns of extreme dynamic range and all-zero columns, graph replay."""
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


def run(ctx, torch, kind, bits, pk, sc, out, inn, x, bias=None):
    t = ctx.bind(kind, pk, sc, out, inn, bits=bits)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    bd = torch.from_numpy(bias).cuda() if bias is not None else None
    y = torch.full((x.shape[0], out), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matmul(t, xd, y, bias_dev=bd)
    torch.cuda.synchronize()
    t.free()
    return y.cpu().numpy()


FORMATS = [(1, 0), (5, 0), (2, 0), (4, 2), (4, 3), (4, 4), (4, 5), (4, 7), (4, 8), (4, 9), (4, 10)]
SHAPES = [(200, 1024), (136, 256), (600, 2048)]       # K split over 4 / 1 / several workgroups


@pytest.mark.parametrize("kind,bits", FORMATS)
@pytest.mark.parametrize("M", [16, 33, 100])
def test_mfma_parity(ctx, torch_dev, oracle, kind, bits, M):
    torch = torch_dev
    for out, inn in SHAPES:
        say("mfma", kind, bits, M, out, inn)
        w = weights(700 + 13 * kind + bits, out, inn)
        pk, sc = quant(oracle, kind, w, bits)
        x = seeded_normal(800 + M, (M, inn))
        bias = seeded_normal(801, (out,))
        got = run(ctx, torch, kind, bits, pk, sc, out, inn, x, bias)
        ref = oracle.gemm_f32(kind, pk, sc, x, bias=bias, bits=bits)
        e = relerr(got, ref)
        print(f"  max-rel {e:.3e}")
        assert np.all(np.isfinite(got)) and e <= TOL, (out, inn, e)


@pytest.mark.parametrize("kind,bits", [(2, 8), (5, 0)])
@pytest.mark.parametrize("out,inn", [(198, 1024), (130, 256), (66, 2048)])
@pytest.mark.parametrize("M", [17, 32])
def test_mfma_ragged_rows(ctx, torch_dev, oracle, kind, bits, out, inn, M):
    """Row counts that are not a multiple of 4: the last 16-byte run of each column is stored element
    by element, and with out % 4 == 2 every odd column row of y (and of the K-split partials) starts
    8 bytes off a 16-byte boundary, so the stores take the unaligned path; with and without a K
    split, with a bias.  y starts as NaN, so an element the kernel skips fails the test."""
    torch = torch_dev
    say("mfma ragged", kind, out, inn, M)
    w = weights(960 + out, out, inn)
    pk, sc = quant(oracle, kind, w, bits)
    x = seeded_normal(961 + M, (M, inn))
    bias = seeded_normal(962, (out,))
    got = run(ctx, torch, kind, bits, pk, sc, out, inn, x, bias)
    ref = oracle.gemm_f32(kind, pk, sc, x, bias=bias, bits=bits)
    assert np.all(np.isfinite(got)) and relerr(got, ref) <= TOL


@pytest.mark.parametrize("M", [16, 17, 31, 32, 48, 64, 65])
def test_mfma_column_tiles(ctx, torch_dev, oracle, M):
    """Every column-tile count 1..4 and a second 64-column launch, int8 weights."""
    torch = torch_dev
    out, inn = 264, 512
    say("mfma columns", M)
    w = weights(900, out, inn)
    pk, sc = oracle.quantize_q8g64(w)
    x = seeded_normal(901 + M, (M, inn))
    got = run(ctx, torch, 2, 8, pk, sc, out, inn, x)
    assert relerr(got, oracle.gemm_f32(2, pk, sc, x)) <= TOL


def test_mfma_matches_dot4_path(torch_dev, oracle, monkeypatch):
    import beglin_amd
    torch = torch_dev
    out, inn, M = 320, 1536, 32
    say("mfma vs dot4")
    w = weights(910, out, inn)
    pk, sc = oracle.quantize_q4g32h(w)
    x = seeded_normal(911, (M, inn))
    c1 = beglin_amd.Context(0)
    a = run(c1, torch, 5, 4, pk, sc, out, inn, x)
    c1.close()
    monkeypatch.setenv("BGL_NO_MFMA", "1")
    c2 = beglin_amd.Context(0)
    b = run(c2, torch, 5, 4, pk, sc, out, inn, x)
    c2.close()
    ref = oracle.gemm_f32(5, pk, sc, x)
    assert relerr(a, ref) <= TOL and relerr(b, ref) <= TOL and relerr(a, b) <= 2 * TOL


def test_mfma_activation_range(ctx, torch_dev, oracle):
    """Columns spanning 1e-6..1e6, a column of zeros, a column with one non-zero element."""
    torch = torch_dev
    out, inn, M = 192, 1024, 20
    say("mfma activation range")
    w = weights(920, out, inn)
    pk, sc = oracle.quantize_q4g64(w)
    x = seeded_normal(921, (M, inn))
    x[0] *= np.float32(1e6)
    x[1] *= np.float32(1e-6)
    x[2] = 0.0
    x[3] = 0.0
    x[3, 777] = 3.25
    x[4] *= np.exp(np.linspace(-8, 8, inn)).astype(np.float32)        # wide range within a column
    got = run(ctx, torch, 1, 4, pk, sc, out, inn, x)
    ref = oracle.gemm_f32(1, pk, sc, x)
    for m in range(M):
        assert relerr(got[m], ref[m]) <= TOL or np.max(np.abs(ref[m])) == 0.0, m
    assert np.all(got[2] == 0.0)


def test_mfma_group_with_bias(ctx, torch_dev, oracle):
    """Fused q/k/v-shaped group (one activation, three int8 tensors) with biases, M=32."""
    torch = torch_dev
    inn, M = 1024, 32
    outs = [512, 128, 128]
    say("mfma group")
    x = seeded_normal(930, (M, inn))
    xd = torch.from_numpy(x).cuda()
    ts, ys, bs, refs = [], [], [], []
    for i, o in enumerate(outs):
        pk, sc = oracle.quantize_q8g64(weights(931 + i, o, inn))
        b = seeded_normal(940 + i, (o,))
        ts.append(ctx.bind(2, pk, sc, o, inn, bits=8))
        ys.append(torch.full((M, o), float("nan"), device="cuda"))
        bs.append(torch.from_numpy(b).cuda())
        refs.append(oracle.gemm_f32(2, pk, sc, x, bias=b))
    ctx.matmul_group(ts, xd, ys, biases=bs)
    torch.cuda.synchronize()
    for y, r in zip(ys, refs):
        assert relerr(y.cpu().numpy(), r) <= TOL
    for t in ts:
        t.free()


def test_mfma_graph_replays_match_eager(torch_dev, oracle):
    import beglin_amd
    torch = torch_dev
    out, inn, M = 256, 2048, 32
    say("mfma graph")
    pk, sc = oracle.quantize_qng64(weights(950, out, inn), 5)
    s = torch.cuda.Stream()
    gc = beglin_amd.Context(0, stream=s.cuda_stream)
    t = gc.bind(4, pk, sc, out, inn, bits=5)
    x = torch.from_numpy(seeded_normal(951, (M, inn))).cuda()
    y = torch.zeros((M, out), device="cuda")
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
    assert relerr(eager, oracle.gemm_f32(4, pk, sc, x.cpu().numpy(), bits=5)) <= TOL
    t.free()
    gc.close()


@pytest.mark.parametrize("case", range(24))
def test_f32_random_shapes(ctx, torch_dev, oracle, case):
    """Seeded random fp32-activation shapes against the oracle (<= 1e-5): int4 g64, int8 g64,
    Q4G32H and qNg64 n = 2..15, ragged row counts, K of 1-48 groups, 1-70 columns (the one-column
    kernel, the dot4 column chunks below 16, the matrix cores from 16 where the format takes them,
    launches of 64 columns past that), with and without bias."""
    torch = torch_dev
    rng = np.random.default_rng(3500 + case)
    kind = int(rng.choice([1, 2, 4, 5]))
    bits = int(rng.integers(2, 16)) if kind == 4 else 0
    inn = 64 * int(rng.integers(1, 49))
    out = int(rng.integers(1, 400))
    M = int(rng.integers(1, 71))
    with_bias = bool(rng.integers(0, 2))
    say("f32 random", case, kind, bits, inn, out, M, with_bias)
    pk, sc = quant(oracle, kind, weights(3600 + case, out, inn), bits)
    x = seeded_normal(3700 + case, (M, inn))
    bias = seeded_normal(3800 + case, (out,)) if with_bias else None
    got = run(ctx, torch, kind, bits, pk, sc, out, inn, x, bias=bias)
    ref = oracle.gemm_f32(kind, pk, sc, x, bias=bias, bits=bits)
    assert relerr(got, ref) <= TOL, (case, kind, bits, inn, out, M, relerr(got, ref))


@pytest.mark.parametrize("kind,bits", [(5, 0), (2, 0), (4, 7)])
def test_mfma_tiny_and_huge_columns(ctx, torch_dev, oracle, kind, bits):
    """Columns whose largest |x| is far from 1 on the matrix cores: 1e-36 and 1e-39 (the column's
    power-of-two scale 2^(14-e) is then beyond fp32's range as a factor), subnormals only, 1e36,
    and all zeros; every output finite and, column by column, within 1e-5 of the oracle's (the
    subnormal column's outputs within a few subnormal spacings)."""
    torch = torch_dev
    out, inn, M = 160, 1024, 20
    say("mfma tiny / huge", kind, bits)
    pk, sc = quant(oracle, kind, weights(4600 + kind, out, inn), bits)
    x = seeded_normal(4610, (M, inn))
    x[0] *= np.float32(1e-36)
    x[1] *= np.float32(1e-39)
    x[2] = (seeded_normal(4611, (inn,)) * np.float32(1e-41)).astype(np.float32)
    x[3] *= np.float32(1e36)
    x[4] = 0.0
    got = run(ctx, torch, kind, bits, pk, sc, out, inn, x)
    ref = oracle.gemm_f32(kind, pk, sc, x, bits=bits)
    assert np.all(np.isfinite(got)), [m for m in range(M) if not np.all(np.isfinite(got[m]))]
    for m in (0, 1, 3) + tuple(range(5, M)):
        assert relerr(got[m], ref[m]) <= TOL, (m, relerr(got[m], ref[m]))
    # outputs ~1e-41 are subnormal (spacing 2^-149): a few spacings of absolute error
    assert np.max(np.abs(got[2].astype(np.float64) - ref[2])) <= 16 * 2.0 ** -149
    assert np.max(np.abs(ref[2])) > 0.0 and np.all(got[4] == 0.0)
