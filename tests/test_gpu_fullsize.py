"""GPU parity at the BASELINE configurations' full sizes, on exactly the paths bench.py times.

* cfg2 (Qwen2.5-1.5B, q4g256sf W4A8): the fused qkv (1536+256+256 rows) and fused gate+up
  (2 x 8960 rows) launches and the down projection (K = 8960), at M = 1, 4 and 8 -- every output
  bit-identical to the oracle's q4_dot_sdot_row_g256sf_v restatement (q4gemv_g256.h:134-157,
  :230-262), the launch shapes of the bench (>= 512 workgroups, the 4-wave 8-column branch).
* cfg4 (DeepSeek-V2-Lite MoE layer): bgl_moe_layer_dev -- device router, top-6, bucketing, routed
  gate+up+SwiGLU+down in the bench's mixed precision, two shared experts merged (2816), the
  combine -- at E = 64, hidden 2048, expert 1408, T = 1, 8, 64, against the oracle's router logits,
  routing and bucketed FFN (moe_ffn_batched, qwen_infer.c:5238-5350).  Bar 1e-5.
* cfg5 (Llama-3.1-8B, M = 32, matrix cores): q / k int8, gate / down int4 g32 and qNg64 n = 5 at
  K = 4096 and K = 14336 (the K-split path), against the oracle's fp32-product double sums.

Weights are made on the device (seeded torch generator) and quantized by the device packers,
which are byte-checked against the oracle elsewhere; the reference-layout bytes come back for the
oracle."""
import sys

import numpy as np
import pytest

from golden.fixtures import seeded_normal
from oracle_ffi import moe_ffn

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


# ---------------------------------------------------------------------------- cfg2
@pytest.mark.parametrize("M", [1, 4, 8])
def test_cfg2_fused_launches_bitexact(ctx, torch_dev, oracle, M):
    import beglin_amd
    torch = torch_dev
    gen = torch.Generator(device="cuda").manual_seed(20 + M)
    H, I = 1536, 8960
    groups = {"qkv": [(H, H), (256, H), (256, H)], "gate_up": [(I, H), (I, H)], "down": [(H, I)]}
    for name, shapes in groups.items():
        say("cfg2", name, M)
        ts, refs = zip(*[qdev(ctx, torch, gen, beglin_amd.K_Q4G256SF, 4, o, i) for o, i in shapes])
        inn = shapes[0][1]
        x = seeded_normal(30 + M, (M, inn))
        ys = [torch.full((M, o), float("nan"), device="cuda") for o, _ in shapes]
        bias = [seeded_normal(40 + j, (o,)) if name == "qkv" else None for j, (o, _) in enumerate(shapes)]
        ctx.matmul_group(list(ts), dev(torch, x), ys, act=beglin_amd.ACT_W4A8,
                         biases=[dev(torch, b) if b is not None else None for b in bias])
        ctx.sync()
        for j, ((pk, ws, sub), y) in enumerate(zip(refs, ys)):
            want = oracle.matmul_sdot(3, pk, ws, x, bias=bias[j], sub=sub)
            got = y.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, j, M, relerr(got, want))
        for t in ts:
            t.free()


# ---------------------------------------------------------------------------- cfg4
CFG4_FORMATS = [(5, 0), (2, 0)] + [(4, n) for n in range(7, 16)]


@pytest.mark.parametrize("T", [1, 8, 64])
def test_cfg4_layer_full_shape(ctx, torch_dev, oracle, T):
    torch = torch_dev
    E, H, I, K, Ish = 64, 2048, 1408, 6, 2816
    say("cfg4 layer", T)
    gen = torch.Generator(device="cuda").manual_seed(400 + T)
    rng = np.random.default_rng(401 + T)
    fm = [CFG4_FORMATS[i] for i in rng.integers(0, len(CFG4_FORMATS), E)]
    shf = CFG4_FORMATS[int(rng.integers(0, len(CFG4_FORMATS)))]
    descs, stacks = [], []
    for (o, i) in ((I, H), (I, H), (H, I)):
        ts, ds = [], []
        for (k, b) in fm:
            t, (p, s, _) = qdev(ctx, torch, gen, k, b, o, i)
            ts.append(t); ds.append((k, b, p, s))
        stacks.append(ctx.experts_from_tensors(ts))
        descs.append(ds)
    sh_t, sh_d = [], []
    for (o, i) in ((Ish, H), (Ish, H), (H, Ish)):
        t, (p, s, _) = qdev(ctx, torch, gen, shf[0], shf[1], o, i)
        sh_t.append(t); sh_d.append((shf[0], shf[1], p, s))
    rw = seeded_normal(402 + T, (E, H), float(1.0 / np.sqrt(H)))
    x = seeded_normal(403 + T, (T, H))
    idx, w = oracle.route(oracle.router_logits(rw, x), K, False)
    ref = moe_ffn(oracle, descs[0], descs[1], descs[2], tuple(sh_d), H, I, x, idx, w)
    out = torch.full((T, H), float("nan"), device="cuda")
    ctx.moe_layer(dev(torch, rw), stacks[0], stacks[1], stacks[2], tuple(sh_t), dev(torch, x), K, out)
    ctx.sync()
    e = relerr(out.cpu().numpy(), ref)
    print(f"  max-rel {e:.3e}")
    assert e <= TOL, e
    for t in stacks + sh_t:
        t.free()


# ---------------------------------------------------------------------------- cfg5
CFG5 = [(2, 0, 4096, 4096), (2, 0, 1024, 4096), (5, 0, 14336, 4096), (5, 0, 4096, 14336), (4, 5, 4096, 14336),
        (4, 5, 14336, 4096)]


@pytest.mark.parametrize("kind,bits,N,K", CFG5)
def test_cfg5_full_shapes_m32(ctx, torch_dev, oracle, kind, bits, N, K):
    torch = torch_dev
    M = 32
    say("cfg5", kind, bits, N, K)
    gen = torch.Generator(device="cuda").manual_seed(500 + K + N + bits)
    t, (p, s, _) = qdev(ctx, torch, gen, kind, bits, N, K)
    x = seeded_normal(501 + K, (M, K))
    y = torch.full((M, N), float("nan"), device="cuda")
    ctx.matmul(t, dev(torch, x), y)
    ctx.sync()
    ref = oracle.gemm_f32(kind, p, s, x, bits=bits)
    e = max(relerr(y.cpu().numpy()[m], ref[m]) for m in range(M))
    print(f"  max-rel {e:.3e}")
    assert e <= TOL, e
    t.free()
