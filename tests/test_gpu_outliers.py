"""GPU parity of every fp32-activation kernel on activations with outliers and non-finite values,
at the BASELINE shapes, through the C-ABI against the CPU oracle (fp32 products, double sums:
qng64_dense.c:90-98, qwen_infer.c:2731-2776; the oracle restates them).

The fp32 activations become exact integer digits per 64-group relative to the group's largest
element; a group whose other elements lie far below that element (an outlier, a "massive
activation" channel) also carries a level-1 residual, so the small elements keep their precision.
These tests put such outliers where they hurt most: channels x1e3..x1e5 whose weight columns are
x0.01 or zero (the outlier then adds little to y while its group's other elements carry the
result), clusters of 33 or 40 large channels per group with zero weight columns (y then comes
from each group's small minority), two outliers of different size in one group, all-zero and
subnormal groups.

Non-finite policy (matches the reference's IEEE arithmetic): a NaN activation makes every output of
its column NaN; +-Inf gives +-Inf where every product with it has that sign, NaN where a weight at
an Inf channel is zero or products of both signs meet.  The tests compare the NaN / +Inf / -Inf
pattern of every output with the oracle's, and the finite outputs to the 1e-5 bar.

Kernels: k_gemv_x (M=1, digits made in the kernel and prepared), k_gemv (M = 4 / 8, and M = 32 with
the matrix cores switched off), k_gemm_mfma (M = 32), k_moe_x and k_moe_gemv (routed MoE FFN at the
DeepSeek-V2-Lite expert shape).  Bar: max|y - ref| / max|ref| <= 1e-5."""
import sys

import numpy as np
import pytest

from golden.fixtures import seeded_normal
from oracle_ffi import moe_ffn, mxfp4_quant

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


def context(monkeypatch, **env):
    import beglin_amd
    for k in ("BGL_FORCE_TR", "BGL_X_WAVES", "BGL_NO_GEMV_X", "BGL_X_FUSE", "BGL_NO_MFMA", "BGL_NO_MOE_X"):
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, str(v))
    return beglin_amd.Context(0)


def relerr(y, r):
    y = np.asarray(y, np.float64); r = np.asarray(r, np.float64)
    return float(np.max(np.abs(y - r)) / max(np.max(np.abs(r)), 1e-30))


def quant(oracle, kind, w, bits):
    if kind == 1:
        return oracle.quantize_q4g64(w)
    if kind == 2:
        return oracle.quantize_q8g64(w)
    if kind == 4:
        return oracle.quantize_qng64(w, bits)
    return oracle.quantize_q4g32h(w)


# ---------------------------------------------------------------------------- activation patterns
def outlier_case(name, K, M, seed):
    """(x [M][K], column multipliers for the weights [K]) for one named pattern."""
    rng = np.random.default_rng(seed)
    x = seeded_normal(seed, (M, K))
    wmul = np.ones(K, np.float32)
    if name == "x1e3_w0.01":
        ch = rng.choice(K, 8, replace=False); x[:, ch] *= np.float32(1e3); wmul[ch] = 0.01
    elif name == "x1e4_w0.01":
        ch = rng.choice(K, 8, replace=False); x[:, ch] *= np.float32(1e4); wmul[ch] = 0.01
    elif name == "x1e5_w0":
        ch = rng.choice(K, 16, replace=False); x[:, ch] *= np.float32(1e5); wmul[ch] = 0.0
    elif name == "two_sizes_one_group":
        g = 64 * int(rng.integers(0, K // 64))
        x[:, g + 3] = np.float32(1e5); wmul[g + 3] = 0.0
        x[:, g + 40] *= np.float32(1e3)
    elif name.startswith("maj"):                                    # "maj<count>_x<mult>": a cluster of large channels
        nbig, mul = name[3:].split("_x")
        for g0 in range(0, K, 64):
            ch = g0 + rng.choice(64, int(nbig), replace=False)
            x[:, ch] *= np.float32(float(mul)); wmul[ch] = 0.0
    elif name == "zeros_subnormals":
        x[:, :64] = 0.0
        if K >= 256:
            x[:, 64:128] *= np.float32(1e-40)                       # all subnormal
            x[:, 128:192] *= np.float32(1e-39)
            x[:, 130] = np.float32(3.0)                             # one normal value among subnormals
            x[:, 192:256] = 0.0
            x[:, 200] = np.float32(-1e-3)                           # a single nonzero element
    return x.astype(np.float32), wmul


PATTERNS = ["x1e3_w0.01", "x1e4_w0.01", "x1e5_w0", "two_sizes_one_group", "zeros_subnormals"]
# Most of every group's channels large (x1e2 .. x1e4) with zero weight columns, so y comes from the
# group's small elements alone: every level-0 element then errs by up to 2^-23 of its group's large
# maximum, and the groups need their level-1 residual (bgl_x_level1: 8 or more small elements).
MAJORITY = [f"maj{n}_x{m}" for n in (33, 40) for m in ("1e2", "1e3", "1e4")]


def make_weights(oracle, kind, bits, N, K, wmul, seed):
    w = (seeded_normal(seed, (N, K), 0.02) * wmul[None, :]).astype(np.float32)
    return quant(oracle, kind, w, bits)


def run_dense(c, torch, kind, bits, pk, sc, N, K, x):
    t = c.bind(kind, pk, sc, N, K, bits=bits)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    y = torch.full((x.shape[0], N), 7.0, dtype=torch.float32, device="cuda")
    c.matmul(t, xd, y)
    torch.cuda.synchronize()
    t.free()
    return y.cpu().numpy()


def check_classes(got, ref, what):
    """NaN / +Inf / -Inf in the same places; finite values within the bar."""
    for f, nm in ((np.isnan, "nan"), (np.isposinf, "+inf"), (np.isneginf, "-inf")):
        a, b = f(got), f(ref)
        assert np.array_equal(a, b), (what, nm, int(a.sum()), int(b.sum()), np.argwhere(a != b)[:5].tolist())
    fin = np.isfinite(ref)
    if fin.any():
        e = relerr(got[fin], ref[fin])
        assert e <= TOL, (what, e)


# ---------------------------------------------------------------------------- dense GEMVs, M = 1
# (kind, bits, N, K): cfg1 (Q4G32H gate_proj), cfg3 gate and down (qNg64 n = 2 / 15), int4 g64, int8
DENSE = [(5, 0, 8960, 1536), (4, 2, 14336, 4096), (4, 15, 14336, 4096), (4, 2, 4096, 14336), (4, 7, 4096, 14336),
         (1, 0, 2048, 2048), (2, 0, 1024, 4096)]


@pytest.mark.parametrize("kind,bits,N,K", DENSE)
@pytest.mark.parametrize("fuse", [-1, 0])
def test_gemv_x_outliers(torch_dev, oracle, monkeypatch, kind, bits, N, K, fuse):
    """k_gemv_x at M = 1: digits made in the kernel (K <= 4096, fuse = -1) or by the prep kernel."""
    torch = torch_dev
    c = context(monkeypatch, **({"BGL_X_FUSE": fuse} if fuse >= 0 else {}))
    for i, pat in enumerate(PATTERNS):
        say("gemv_x outliers", kind, bits, N, K, fuse, pat)
        x, wmul = outlier_case(pat, K, 1, 100 + i)
        pk, sc = make_weights(oracle, kind, bits, N, K, wmul, 200 + i)
        got = run_dense(c, torch, kind, bits, pk, sc, N, K, x)
        ref = oracle.gemm_f32(kind, pk, sc, x, bits=bits)
        e = relerr(got, ref)
        print(f"  max-rel {e:.3e}")
        assert np.all(np.isfinite(got)) and e <= TOL, (pat, e)
    c.close()


# cfg1 (Q4G32H 8960x1536), cfg3 gate n = 2 / 15 and cfg3 down n = 7
MAJ_DENSE = [(5, 0, 8960, 1536), (4, 2, 14336, 4096), (4, 15, 14336, 4096), (4, 7, 4096, 14336)]


@pytest.mark.parametrize("kind,bits,N,K", MAJ_DENSE)
def test_dense_majority_outliers(torch_dev, oracle, monkeypatch, kind, bits, N, K):
    """33 or 40 of every group's 64 channels at x1e2 .. x1e4 with zero weight columns: k_gemv_x
    (digits made in the kernel, and by the prep kernel) at M = 1, k_gemv at M = 4 and the matrix
    cores (or, for qNg64 n > 10, k_gemv) at M = 32 on the first 2048 rows, all to the 1e-5 bar.
    The weights of a pattern are quantized once and serve every configuration."""
    torch = torch_dev
    ctxs = {"fused": context(monkeypatch), "prep": context(monkeypatch, BGL_X_FUSE=0)}
    monkeypatch.delenv("BGL_X_FUSE", raising=False)
    NR = min(N, 2048)                                   # rows of the 32-column run
    for i, pat in enumerate(MAJORITY):
        x, wmul = outlier_case(pat, K, 32, 800 + i)
        pk, sc = make_weights(oracle, kind, bits, N, K, wmul, 820 + i)
        ref14 = oracle.gemm_f32(kind, pk, sc, x[:4], bits=bits)
        ref32 = oracle.gemm_f32(kind, pk[:NR], sc[:NR], x, bits=bits)
        for name, c, M in (("fused", ctxs["fused"], 1), ("prep", ctxs["prep"], 1), ("fused", ctxs["fused"], 4)):
            say("majority outliers", kind, bits, N, K, M, name, pat)
            got = run_dense(c, torch, kind, bits, pk, sc, N, K, x[:M])
            e = max(relerr(got[m], ref14[m]) for m in range(M))
            print(f"  max-rel {e:.3e}")
            assert np.all(np.isfinite(got)) and e <= TOL, (pat, name, M, e)
        say("majority outliers", kind, bits, NR, K, 32, pat)
        got = run_dense(ctxs["fused"], torch, kind, bits, pk[:NR], sc[:NR], NR, K, x)
        e = max(relerr(got[m], ref32[m]) for m in range(32))
        print(f"  max-rel {e:.3e}")
        assert np.all(np.isfinite(got)) and e <= TOL, (pat, 32, e)
    for c in ctxs.values():
        c.close()


@pytest.mark.parametrize("kind,bits", [(5, 0), (4, 3), (2, 0), (1, 0)])
@pytest.mark.parametrize("M,env", [(4, {}), (8, {}), (32, {"BGL_NO_MFMA": 1})])
def test_gemv_columns_outliers(torch_dev, oracle, monkeypatch, kind, bits, M, env):
    """k_gemv over prepared digits: several columns, some with outliers, one plain."""
    torch = torch_dev
    c = context(monkeypatch, **env)
    N, K = 1536, 4096
    for i, pat in enumerate(PATTERNS[:3]):
        say("gemv columns outliers", kind, bits, M, env, pat)
        x, wmul = outlier_case(pat, K, M, 300 + i)
        x[M - 1] = seeded_normal(301 + i, (K,))                    # a column without outliers
        pk, sc = make_weights(oracle, kind, bits, N, K, wmul, 310 + i)
        got = run_dense(c, torch, kind, bits, pk, sc, N, K, x)
        ref = oracle.gemm_f32(kind, pk, sc, x, bits=bits)
        for m in range(M):
            e = relerr(got[m], ref[m])
            assert e <= TOL, (pat, m, e)
    c.close()


@pytest.mark.parametrize("kind,bits", [(5, 0), (2, 0), (4, 5), (1, 0)])
def test_mfma_outliers(torch_dev, oracle, monkeypatch, kind, bits):
    """k_gemm_mfma at M = 32 (cfg5's batch) on Llama-8B-width K: columns scaled per K-split and split
    into fp16 hi/lo parts keep ~22 bits down to 2^-17 of the split's largest element."""
    torch = torch_dev
    c = context(monkeypatch)
    N, K, M = 1024, 4096, 32
    for i, pat in enumerate(PATTERNS):
        say("mfma outliers", kind, bits, pat)
        x, wmul = outlier_case(pat, K, M, 400 + i)
        pk, sc = make_weights(oracle, kind, bits, N, K, wmul, 410 + i)
        got = run_dense(c, torch, kind, bits, pk, sc, N, K, x)
        ref = oracle.gemm_f32(kind, pk, sc, x, bits=bits)
        e = max(relerr(got[m], ref[m]) for m in range(M))
        print(f"  max-rel {e:.3e}")
        assert e <= TOL, (pat, e)
    c.close()


# ---------------------------------------------------------------------------- non-finite
def nonfinite_x(K, M, seed):
    """Column 0: a NaN; column 1: one +Inf; column 2: +Inf and -Inf; column 3: -Inf in a group
    with an outlier; the rest plain."""
    x = seeded_normal(seed, (M, K))
    x[0, 77] = np.nan
    x[1, 130] = np.inf
    if M > 2:
        x[2, 5] = np.inf
        x[2, K - 3] = -np.inf
    if M > 3:
        x[3, 200] = -np.inf
        x[3, 201] = np.float32(1e5)
    return x.astype(np.float32)


def nonfinite_weights(oracle, kind, bits, N, K, seed):
    w = seeded_normal(seed, (N, K), 0.02)
    w[1, :] = 0.0                                                  # a zero row: 0 * Inf = NaN
    w[2, :64] = 0.0                                                # zero weight at channels 5 / 77
    w[3, 128:192] = 0.0                                            # zero weight at the +Inf channel 130
    return quant(oracle, kind, w, bits)


@pytest.mark.parametrize("kind,bits", [(5, 0), (1, 0), (2, 0), (4, 2), (4, 9), (4, 15)])
@pytest.mark.parametrize("M,env", [(1, {}), (1, {"BGL_X_FUSE": 0}), (1, {"BGL_NO_GEMV_X": 1}), (4, {}), (32, {}),
                                   (32, {"BGL_NO_MFMA": 1})])
def test_nonfinite_activations(torch_dev, oracle, monkeypatch, kind, bits, M, env):
    torch = torch_dev
    if M == 32 and not env and kind == 4 and bits > 10:
        pytest.skip("qNg64 n > 10 has no matrix-core kernel (the dot4 path is the M=32 case above)")
    c = context(monkeypatch, **env)
    N, K = 320, 1024
    say("nonfinite", kind, bits, M, env)
    pk, sc = nonfinite_weights(oracle, kind, bits, N, K, 500 + bits)
    xs = nonfinite_x(K, max(M, 4), 501)
    cols = [xs[i:i + 1] for i in range(4)] if M == 1 else [xs[:M] if M >= 4 else xs[:4]]
    for x in cols:
        got = run_dense(c, torch, kind, bits, pk, sc, N, K, x)
        ref = oracle.gemm_f32(kind, pk, sc, x, bits=bits)
        assert np.isnan(ref).any() or np.isinf(ref).any()
        check_classes(got, ref, (kind, bits, M, env))
        if M > 4:                                                  # columns past 4 are finite and exact
            assert np.all(np.isfinite(got[4:])) and relerr(got[4:], ref[4:]) <= TOL
    c.close()


# ---------------------------------------------------------------------------- routed MoE
def moe_descs(oracle, E, H, I, fmts, seed, wmul_h, wmul_i):
    def one(kind, bits, o, i, s, wm):
        w = (seeded_normal(s, (o, i), 0.02) * wm[None, :]).astype(np.float32)
        if kind == 9:                                   # MXFP4 blocks (no scales array)
            return (9, 4, mxfp4_quant(w), None)
        p, sc = quant(oracle, kind, w, bits)
        return (kind, bits, p, sc)
    gate = [one(*fmts[e % len(fmts)], I, H, seed + 3 * e, wmul_h) for e in range(E)]
    up = [one(*fmts[e % len(fmts)], I, H, seed + 3 * e + 1, wmul_h) for e in range(E)]
    down = [one(*fmts[e % len(fmts)], H, I, seed + 3 * e + 2, wmul_i) for e in range(E)]
    return gate, up, down


def run_moe(c, torch, gate, up, down, x, idx, w):
    g, u, d = c.bind_experts(gate), c.bind_experts(up), c.bind_experts(down)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = torch.full(x.shape, 7.0, dtype=torch.float32, device="cuda")
    c.moe_ffn(g, u, d, None, dev(x), dev(idx), dev(w), out)
    c.sync()
    for t in (g, u, d):
        t.free()
    return out.cpu().numpy()


@pytest.mark.parametrize("env", [{}, {"BGL_NO_MOE_X": 1}])
@pytest.mark.parametrize("T", [1, 8])
def test_moe_outliers(torch_dev, oracle, monkeypatch, env, T):
    """Routed FFN at DeepSeek-V2-Lite's expert shape (hidden 2048, expert 1408, top-6) over 12
    experts of mixed precision; token rows with outlier channels whose gate/up columns are small."""
    torch = torch_dev
    c = context(monkeypatch, **env)
    E, H, I, K = 12, 2048, 1408, 6
    fm = [(5, 0), (2, 0), (4, 7), (4, 12), (1, 0), (4, 15)]
    for i, pat in enumerate(["x1e4_w0.01", "x1e5_w0", "two_sizes_one_group"]):
        say("moe outliers", env, T, pat)
        x, wmul = outlier_case(pat, H, T, 600 + i)
        gate, up, down = moe_descs(oracle, E, H, I, fm, 610 + 40 * i, wmul, np.ones(I, np.float32))
        idx, w = oracle.route(seeded_normal(620 + i, (T, E)), K, False)
        got = run_moe(c, torch, gate, up, down, x, idx, w)
        ref = moe_ffn(oracle, gate, up, down, None, H, I, x, idx, w)
        e = relerr(got, ref)
        print(f"  max-rel {e:.3e}")
        assert e <= TOL, (pat, e)
    c.close()


def test_moe_majority_outliers(torch_dev, oracle, monkeypatch):
    """The routed FFN at DeepSeek-V2-Lite's expert shape (k_moe_x, and k_moe_gemv over prepared
    digits) with 33 or 40 of every group's 64 hidden channels at x1e2 .. x1e4 and zero gate/up
    columns there, at T = 1 and 8.  The experts of a pattern are quantized once."""
    torch = torch_dev
    cx = context(monkeypatch)
    cg = context(monkeypatch, BGL_NO_MOE_X=1)
    monkeypatch.delenv("BGL_NO_MOE_X", raising=False)
    E, H, I, K = 12, 2048, 1408, 6
    fm = [(5, 0), (2, 0), (4, 7), (4, 12), (1, 0), (4, 15)]
    for i, pat in enumerate(MAJORITY):
        x8, wmul = outlier_case(pat, H, 8, 840 + i)
        gate, up, down = moe_descs(oracle, E, H, I, fm, 850 + 40 * i, wmul, np.ones(I, np.float32))
        for T in (1, 8):
            x = np.ascontiguousarray(x8[:T])
            idx, w = oracle.route(seeded_normal(860 + i + T, (T, E)), K, False)
            ref = moe_ffn(oracle, gate, up, down, None, H, I, x, idx, w)
            for name, c in (("moe_x", cx), ("moe_gemv", cg)):
                say("moe majority outliers", name, T, pat)
                got = run_moe(c, torch, gate, up, down, x, idx, w)
                e = relerr(got, ref)
                print(f"  max-rel {e:.3e}")
                assert e <= TOL, (pat, name, T, e)
    cx.close()
    cg.close()


@pytest.mark.parametrize("env", [{}, {"BGL_NO_MOE_X": 1}])
def test_moe_nonfinite(torch_dev, oracle, monkeypatch, env):
    """NaN / +-Inf token rows through gate+up, SwiGLU (g / (1 + exp(-g)) * u, qwen_infer.c:3475-3481)
    and the down projection: the same NaN / Inf pattern as the oracle, finite rows to the bar."""
    torch = torch_dev
    c = context(monkeypatch, **env)
    E, H, I, K, T = 8, 512, 384, 3, 5
    say("moe nonfinite", env)
    fm = [(5, 0), (2, 0), (4, 9), (1, 0)]
    gate, up, down = moe_descs(oracle, E, H, I, fm, 700, np.ones(H, np.float32), np.ones(I, np.float32))
    x = seeded_normal(701, (T, H))
    x[0, 10] = np.nan
    x[1, 300] = np.inf
    x[2, 7] = -np.inf
    idx, w = oracle.route(seeded_normal(702, (T, E)), K, False)
    got = run_moe(c, torch, gate, up, down, x, idx, w)
    ref = moe_ffn(oracle, gate, up, down, None, H, I, x, idx, w)
    check_classes(got, ref, env)
    assert np.all(np.isfinite(got[3:])) and relerr(got[3:], ref[3:]) <= TOL
    c.close()


@pytest.mark.parametrize("T", [1, 8])
def test_moe_outliers_mxfp4(torch_dev, oracle, monkeypatch, T):
    """MXFP4 experts (beside int4 g32 and qNg64 ones) under the outlier patterns: their level-1 and
    non-finite cold paths (signed codes, no -8 correction) against the oracle's MXFP4 row."""
    torch = torch_dev
    c = context(monkeypatch)
    E, H, I, K = 8, 2048, 1408, 6
    fm = [(9, 4), (5, 0), (9, 4), (4, 12)]
    for i, pat in enumerate(["x1e4_w0.01", "x1e5_w0", "two_sizes_one_group"]):
        say("moe outliers mxfp4", T, pat)
        x, wmul = outlier_case(pat, H, T, 640 + i)
        gate, up, down = moe_descs(oracle, E, H, I, fm, 650 + 40 * i, wmul, np.ones(I, np.float32))
        idx, w = oracle.route(seeded_normal(660 + i, (T, E)), K, False)
        got = run_moe(c, torch, gate, up, down, x, idx, w)
        ref = moe_ffn(oracle, gate, up, down, None, H, I, x, idx, w)
        e = relerr(got, ref)
        print(f"  max-rel {e:.3e}")
        assert e <= TOL, (pat, e)
    x = seeded_normal(670, (5, H))
    x[0, 10] = np.nan
    x[1, 300] = np.inf
    x[2, 7] = -np.inf
    gate, up, down = moe_descs(oracle, E, H, I, fm, 680, np.ones(H, np.float32), np.ones(I, np.float32))
    idx, w = oracle.route(seeded_normal(690, (5, E)), K, False)
    got = run_moe(c, torch, gate, up, down, x, idx, w)
    ref = moe_ffn(oracle, gate, up, down, None, H, I, x, idx, w)
    check_classes(got, ref, {})
    assert np.all(np.isfinite(got[3:])) and relerr(got[3:], ref[3:]) <= TOL
    c.close()
