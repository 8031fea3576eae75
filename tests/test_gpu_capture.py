"""Graph capture and the context's per-call scratch, through the C-ABI.

A graph captured from a context's stream holds the raw addresses of the scratch its calls used
(activation digits, sort buffers, routing, partial sums).  These tests pin the contract stated in
include/beglin_qgemv.h:
* a later, larger eager call that outgrows the scratch does not free what a graph uses: replays
  after it still give the captured call's result, bit for bit;
* a captured call that would need more scratch than any eager call has sized fails with
  BGL_E_CAPTURE, enqueues nothing, and the context keeps working."""
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


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def moe_stack(ctx, oracle, E, o, i, seed):
    ds = []
    for e in range(E):
        w = seeded_normal(seed + e, (o, i), 0.02)
        p, s = oracle.quantize_q4g32h(w) if e % 2 == 0 else oracle.quantize_qng64(w, 9)
        ds.append((5, 0, p, s) if e % 2 == 0 else (4, 9, p, s))
    return ctx.bind_experts(ds)


def test_moe_layer_graph_survives_larger_eager_call(torch_dev, oracle):
    import beglin_amd
    torch = torch_dev
    E, H, I, K = 16, 512, 256, 4
    say("capture moe layer T=1, eager T=64, replay")
    s = torch.cuda.Stream()
    c = beglin_amd.Context(0, stream=s.cuda_stream)
    g, u, d = moe_stack(c, oracle, E, I, H, 100), moe_stack(c, oracle, E, I, H, 200), moe_stack(c, oracle, E, H, I, 300)
    rw = dev(torch, seeded_normal(400, (E, H), 0.05))
    x1 = dev(torch, seeded_normal(401, (1, H)))
    x64 = dev(torch, seeded_normal(402, (64, H)))
    y1 = torch.zeros((1, H), device="cuda")
    y64 = torch.zeros((64, H), device="cuda")
    with torch.cuda.stream(s):
        c.moe_layer(rw, g, u, d, None, x1, K, y1)
    c.sync()
    eager = y1.cpu().numpy().copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        c.moe_layer(rw, g, u, d, None, x1, K, y1)
    for r in range(3):
        with torch.cuda.stream(s):
            c.moe_layer(rw, g, u, d, None, x64, K, y64)      # outgrows every scratch buffer the graph uses
        c.sync()
        y1.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y1.cpu().numpy(), eager), r
    for t in (g, u, d):
        t.free()
    c.close()


def test_dense_graph_survives_larger_eager_call(torch_dev, oracle):
    """fp32 activations over a prepared-digit path (K > 4096) and a K-split launch (few tiles)."""
    import beglin_amd
    torch = torch_dev
    say("capture dense M=2, eager M=12, replay")
    s = torch.cuda.Stream()
    c = beglin_amd.Context(0, stream=s.cuda_stream)
    N, K = 96, 8192                                      # 2 tiles: split K over workgroups (partials)
    p, sc = oracle.quantize_qng64(seeded_normal(500, (N, K), 0.02), 6)
    t = c.bind(4, p, sc, N, K, bits=6)
    x2 = dev(torch, seeded_normal(501, (2, K)))
    x12 = dev(torch, seeded_normal(502, (12, K)))
    y2 = torch.zeros((2, N), device="cuda")
    y12 = torch.zeros((12, N), device="cuda")
    with torch.cuda.stream(s):
        c.matmul(t, x2, y2)
    c.sync()
    eager = y2.cpu().numpy().copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        c.matmul(t, x2, y2)
    for r in range(3):
        with torch.cuda.stream(s):
            c.matmul(t, x12, y12)
        c.sync()
        y2.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y2.cpu().numpy(), eager), r
    t.free()
    c.close()


def test_capture_that_needs_more_scratch_is_refused(torch_dev, oracle):
    import beglin_amd
    torch = torch_dev
    say("capture needing growth -> BGL_E_CAPTURE")
    s = torch.cuda.Stream()
    c = beglin_amd.Context(0, stream=s.cuda_stream)
    N, K = 256, 8192
    p, sc = oracle.quantize_q4g32h(seeded_normal(600, (N, K), 0.02))
    t = c.bind(5, p, sc, N, K)
    x1 = dev(torch, seeded_normal(601, (1, K)))
    x8 = dev(torch, seeded_normal(602, (8, K)))
    y1 = torch.zeros((1, N), device="cuda")
    y8 = torch.zeros((8, N), device="cuda")
    with torch.cuda.stream(s):
        c.matmul(t, x1, y1)                               # sizes the scratch for one column
    c.sync()
    graph = torch.cuda.CUDAGraph()
    refused = None
    with torch.cuda.stream(s):
        graph.capture_begin()
        try:
            c.matmul(t, x8, y8)                           # eight columns' digits: more scratch
        except beglin_amd.BglError as e:
            refused = e
        graph.capture_end()
    assert refused is not None and "capture" in str(refused), refused
    with torch.cuda.stream(s):
        c.matmul(t, x8, y8)                               # eager: grows the scratch and runs
    c.sync()
    ref = oracle.gemm_f32(5, p, sc, x8.cpu().numpy())
    got = y8.cpu().numpy()
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-5
    t.free()
    c.close()
