"""GPU: the int4-mode loader (bgl_model_load_int4, load_int4 qwen_infer.c:554-615) and the cache
of the repacked device layout (the .beglin pattern, gguf_cache.c).

* every quantized tensor of a synthetic manifest + blob is bound and multiplies like the oracle
  (fp32 activations <= 1e-5; W4A8 at M=1 bit-exact);
* f32 tensors are read in place from the mapped blob;
* a saved cache reloads to the same device bytes (bit-identical decode and products), goes stale
  when the blob's mtime changes, and a truncated cache file is refused."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

from golden.fixtures import seeded_normal
from loader_fixture import build

pytestmark = pytest.mark.gpu
TOL = 1e-5
KINDS = {"q4g64": 1, "q8g64": 2, "q4g256sf": 3}


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


def products(ctx, torch, oracle, model, refs):
    """name -> (W4A8 y, fp32-activation y, decoded rows) for every bound tensor, each checked
    against the oracle."""
    res = {}
    for name, ref in refs.items():
        kind, out, inn, t, f32 = model.find(name)
        if ref[0] == "f32":
            assert kind == 0 and t is None
            v = np.ctypeslib.as_array(C.cast(f32, C.POINTER(C.c_float)), shape=(ref[1].size,))
            assert np.array_equal(v, ref[1])
            continue
        assert kind == KINDS[ref[0]] and t is not None
        _, pk, sc, sub = ref
        x = seeded_normal(31 + out, (inn,))
        xd = torch.from_numpy(x).cuda()
        y8 = torch.empty(out, device="cuda")
        ctx.matmul(t, xd, y8, act=1)
        ya = None
        if kind != 3:
            ya = torch.empty(out, device="cuda")
            ctx.matmul(t, xd, ya, act=0)
        ctx.sync()
        r8 = oracle.matmul_sdot(kind, pk, sc, x, sub=sub)
        assert np.array_equal(y8.cpu().numpy().view(np.uint32), r8.view(np.uint32)), name
        if ya is not None:
            assert relerr(ya.cpu().numpy(), oracle.gemm_f32(kind, pk, sc, x)) <= TOL, name
        dq = torch.empty((out, inn), device="cuda")
        ctx.dequant(t, 0, out, dq)
        ctx.sync()
        assert np.array_equal(dq.cpu().numpy(), oracle.decode(kind, pk, sc, out, inn, sub=sub)), name
        res[name] = (y8.cpu().numpy(), None if ya is None else ya.cpu().numpy(), dq.cpu().numpy())
    return res


def test_load_int4_and_cache_round_trip(ctx, torch_dev, oracle, tmp_path):
    import beglin_amd
    torch = torch_dev
    say("loader")
    layout, blob, refs = build(oracle, str(tmp_path))
    m = beglin_amd.Model(ctx, layout, blob)
    assert len(m) == len(refs)
    first = products(ctx, torch, oracle, m, refs)
    cache = str(tmp_path / "weights.bglc")
    m.save_cache(cache)
    m.close()
    assert beglin_amd.cache_valid(cache, layout, blob) == 1
    say("cache")
    mc = beglin_amd.Model(ctx, layout, blob, cache=cache)
    again = products(ctx, torch, oracle, mc, refs)
    for name, (a8, aa, adq) in first.items():
        b8, ba, bdq = again[name]
        assert np.array_equal(a8, b8) and np.array_equal(adq, bdq) and (aa is None or np.array_equal(aa, ba)), name
    with pytest.raises(beglin_amd.BglError):
        mc.find("nope")
    mc.close()
    st = os.stat(blob)
    os.utime(blob, ns=(st.st_atime_ns, st.st_mtime_ns + 2_000_000_000))   # the blob changed: cache stale
    assert beglin_amd.cache_valid(cache, layout, blob) == 0
    with pytest.raises(beglin_amd.BglError):
        beglin_amd.Model(ctx, layout, blob, cache=cache)
    os.utime(blob, ns=(st.st_atime_ns, st.st_mtime_ns))
    assert beglin_amd.cache_valid(cache, layout, blob) == 1
    with open(cache, "r+b") as f:                          # truncated mid-data: refused, not read past
        f.truncate(os.path.getsize(cache) // 2)
    assert beglin_amd.cache_valid(cache, layout, blob) == 1
    with pytest.raises(beglin_amd.BglError):
        beglin_amd.Model(ctx, layout, blob, cache=cache)


def test_load_refuses_a_bad_manifest(ctx, oracle, tmp_path):
    import beglin_amd
    layout, blob, _ = build(oracle, str(tmp_path))
    lines = open(layout).read().splitlines()
    lines[1] = lines[1].replace("q8g64", "q6k")
    with open(layout, "w") as f:
        f.write("\n".join(lines) + "\n")
    with pytest.raises(beglin_amd.BglError):
        beglin_amd.Model(ctx, layout, blob)
