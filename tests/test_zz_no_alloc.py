"""bgl_matmul_group_noalloc_dev (the entry point that allocates nothing) against
bgl_matmul_group_dev, through the C-ABI: the same kernels, so every output must be bit-identical.
Two calls in a row, the second with a smaller input, per path that uses scratch: fp32 activations
over prepared digits (K > 4096) with a K-split (few tiles), the matrix-core path (M >= 16, K-split
partials), W4A8 columns quantized up front (M > 1, long K), and one with outlier / non-finite
activations (the level-1 digits).  A call beyond the fixed array is refused with BGL_E_NOMEM, and
the context's own scratch state is untouched (a prepared activation made before the call is still
served after it)."""
import ctypes as C
import sys

import numpy as np
import pytest

from golden.fixtures import seeded_normal

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    return torch


def call(fn, ctx, ts, act, x, ys):
    import beglin_amd
    n = len(ts)
    W = (C.c_void_p * n)(*[t.h.value for t in ts])
    Y = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    B = (C.c_void_p * n)(*([None] * n))
    M = x.shape[0]
    return getattr(beglin_amd.lib(), fn)(ctx.h, n, W, act, C.c_void_p(x.data_ptr()), B, Y, M)


# (name, kind, bits, act, [(N, K)...] fused tensors, M first, M second)
CASES = [
    ("fp32 prepared digits + K-split", 4, 6, 0, [(96, 8192)], 12, 3),
    ("fp32 fused group, prepared digits", 5, 0, 0, [(512, 6144), (256, 6144)], 6, 2),
    ("fp32 matrix cores, K-split", 5, 0, 0, [(1024, 14336)], 32, 17),
    # M > 64 runs as chunks of 64 columns; each chunk's 16.8 MB of K-split partials reuses one
    # slice of the fixed array (four chunks of fresh slices would exceed it)
    ("fp32 matrix cores, 64-column chunks", 5, 0, 0, [(8192, 4096)], 256, 130),
    ("W4A8 g256sf, columns quantized up front", 3, 4, 1, [(1536, 8960)], 8, 4),
]


@pytest.mark.parametrize("name,kind,bits,act,shapes,M1,M2", CASES)
def test_noalloc_equals_allocating_entry(torch_dev, oracle, name, kind, bits, act, shapes, M1, M2):
    import beglin_amd
    torch = torch_dev
    ctx = beglin_amd.Context(0)
    gen = torch.Generator(device="cuda").manual_seed(7)
    ts = []
    for (N, K) in shapes:
        w = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        ts.append(ctx.quantize(kind, w, bits=bits))
        del w
    K = shapes[0][1]
    for i, M in enumerate((M1, M2)):
        say("noalloc", name, "call", i, "M", M)
        x = seed_x(torch, K, M, 90 + i, outliers=(i == 1 and act == 0))
        ya = [torch.full((M, N), float("nan"), device="cuda") for N, _ in shapes]
        yb = [torch.full((M, N), float("nan"), device="cuda") for N, _ in shapes]
        assert call("bgl_matmul_group_noalloc_dev", ctx, ts, act, x, ya) == 0, beglin_amd.lib().bgl_last_error()
        ctx.sync()
        assert call("bgl_matmul_group_dev", ctx, ts, act, x, yb) == 0, beglin_amd.lib().bgl_last_error()
        ctx.sync()
        for a, b in zip(ya, yb):
            a, b = a.cpu().numpy(), b.cpu().numpy()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
    for t in ts:
        t.free()
    ctx.close()


def seed_x(torch, K, M, seed, outliers=False):
    x = seeded_normal(seed, (M, K))
    if outliers:
        x[0, 100] = np.float32(1e5)
        x[-1, 7] = np.inf
    return torch.from_numpy(x).cuda()


def test_noalloc_refuses_beyond_the_array_and_keeps_context_state(torch_dev, oracle):
    import beglin_amd
    torch = torch_dev
    say("noalloc limit + context state")
    ctx = beglin_amd.Context(0)
    N, K = 128, 16384
    p, sc = oracle.quantize_q4g32h(seeded_normal(95, (N, K), 0.02))
    t = ctx.bind(5, p, sc, N, K)
    # a prepared activation in the context's own scratch, before the no-alloc calls
    x3 = torch.from_numpy(seeded_normal(96, (3, K))).cuda()
    ctx.prep_only(x3, 0, t)
    # fp32 digits need ~116 KB per column at K = 16384: 512 columns exceed the 32 MiB array
    big = torch.from_numpy(seeded_normal(97, (512, K))).cuda()
    yb = torch.zeros((512, N), device="cuda")
    import os
    os.environ["BGL_NO_MFMA"] = "1"            # keep the prepared-digit path (the matrix cores need less)
    c2 = beglin_amd.Context(0)
    os.environ.pop("BGL_NO_MFMA")
    rc = call("bgl_matmul_group_noalloc_dev", c2, [t], 0, big, [yb])
    assert rc == -5                             # BGL_E_NOMEM
    assert b"fixed" in beglin_amd.lib().bgl_last_error()
    c2.close()
    # a small no-alloc call, then the context's prepared activation still serves matmul_prepped
    x1 = torch.from_numpy(seeded_normal(98, (1, K))).cuda()
    y1 = torch.zeros((1, N), device="cuda")
    assert call("bgl_matmul_group_noalloc_dev", ctx, [t], 0, x1, [y1]) == 0
    y3 = torch.zeros((3, N), device="cuda")
    ctx.matmul_prepped(t, y3, act=0, M=3)
    ctx.sync()
    ref = oracle.gemm_f32(5, p, sc, x3.cpu().numpy())
    got = y3.cpu().numpy()
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-5
    ref1 = oracle.gemm_f32(5, p, sc, x1.cpu().numpy())
    assert np.max(np.abs(y1.cpu().numpy() - ref1)) / np.max(np.abs(ref1)) <= 1e-5
    t.free()
    ctx.close()
