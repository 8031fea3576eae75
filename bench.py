"""bench.py -- quantized GEMV / MoE-gather throughput on one MI355X.

Default workload: a Qwen2.5-1.5B decode layer, all seven projections as
q4g256sf W4A8 GEMVs (q 1536x1536, k/v 256x1536, o 1536x1536, gate/up 8960x1536, down 1536x8960),
28 layers of distinct weights (696 MB, > 2x the 256 MB MALL), M=1.  One "step" = one pass over the
28 layers, issued the way the engine issues it: fused q/k/v, o, fused gate+up, down
(QWEN_FUSED_DISPATCH, qwen_infer.c:1276-1306); each call = activation quantization + GEMV.  The
step is captured once into a HIP graph and replayed.  Weights are seeded N(0, 0.02), quantized on
the device by the build's g256sf packer; activations seeded N(0, 1).

Prints ONE JSON line.  `value` = algorithmic bytes per step / step time (GB/s), with
algorithmic bytes = packed + scale + sub-code bytes + 4*M*K (x) + 4*M*N (y) per call.
`roofline.achieved` = the same bytes over the summed duration of the GEMV kernel launches alone
(HIP event-record nodes around every launch, captured into the replayed graph on the context's
stream), i.e. without the inter-launch gaps that `value` includes.  `cpu_baseline` = the reference's threaded CPU
path (portable-C restatement, q4pool row-block split) timed on this host on a bounded sample.

Other workloads for the per-config numbers: --workload cfg1 | cfg3 | cfg4 | cfg5 (see --help).
cfg5 = Llama-3.1-8B projections (q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096, down
4096x14336) at M=32 fp32 activation rows on the matrix-core path: attention int8 (q8g64), MLP
int4 g32 (Q4G32H), a seeded 20% of the tensors qNg64 n=5; one step = --layers layers.
cfg4 = DeepSeek-V2-Lite routed MoE FFN (E=64 + 2 shared experts, hidden 2048, expert inter 1408,
top-6), the whole layer on the device: fp32 router [64 x 2048] with N(0, 1/2048) entries (N(0,1)
logits), softmax, top-6, sort, SwiGLU experts, combine, shared experts; T=--M tokens, per-expert
precision drawn from the seed over {q4g32h, q8g64, qNg64 n=7..15}; one step = --layers distinct
MoE layers; algorithmic bytes = the packed + scale bytes of every expert the step's routing
touches (+ shared experts, router weights, x, out)."""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "quantized GEMV / MoE-gather achieved HBM GB/s (% of peak) + µs per call at M=1"
# the arithmetic each path computes in
DT_W4A8 = "int8 (W4A8: int4 codes x int8 activations, exact int32 dot4 sums, fp32 fold)"
DT_F32ACT = "fp32 activations as exact integer digits (int32 dot4 sums over int8 digits, fp32 fold)"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def qwen_layer_shapes():
    """(name, [(out, in), ...]) per call, in forward_token's issue order (qwen_infer.c:1276-1306,
    1560-1573): the fused q/k/v projection, o, and the MLP block (gate, up, down)."""
    return [("qkv", [(1536, 1536), (256, 1536), (256, 1536)]), ("o", [(1536, 1536)]),
            ("mlp", [(8960, 1536), (8960, 1536), (1536, 8960)])]


def alg_bytes(kind, out, inn, bits, M):
    w = {1: out * inn / 2 + 4 * out * inn / 64, 2: out * inn + 4 * out * inn / 64,
         3: out * inn / 2 + 4 * out * inn / 256 + out * inn / 64, 4: out * inn * bits / 8 + 4 * out * inn / 64,
         5: out * inn / 2 + 2 * out * inn / 32}[kind]
    return w + 4 * M * inn + 4 * M * out


def host_nproc():
    try:
        return len(os.sched_getaffinity(0))
    except Exception:
        return os.cpu_count() or 1


# The GPU box allots 16 host cores to a one-GPU job (its worker pools are to be sized to that
# share, whatever nproc shows); the CPU leg uses all of them and records nproc beside.
HOST_SHARE = 16


def host_threads():
    return max(1, min(HOST_SHARE, host_nproc()))


ROTATE_BYTES = 512 << 20       # CPU legs cycle through weight copies of at least this footprint (2x the MALL)


# ------------------------------------------------------------------------------------- GPU side
class Workload:
    """A list of calls; each call = (tensors, x, ys, act, bytes, tag).  Tag "mlp": the tensors are
    (gate, up, down) of one MLP block (bgl_mlp_dev), ys its one output."""

    def __init__(self, ctx, torch):
        self.ctx, self.torch = ctx, torch
        self.calls = []
        self.tensors = []

    def add(self, group, x, act, nbytes, tag):
        outs = [group[2]] if tag == "mlp" else group
        ys = [self.torch.empty((x.shape[0], t.info()["out"]), device="cuda") for t in outs]
        self.calls.append((group, x, ys, act, nbytes, tag))
        self.tensors += group

    def run(self, tags=None):
        for group, x, ys, act, _, tag in self.calls:
            if tags is None or tag in tags:
                if tag == "mlp":
                    self.ctx.mlp(group[0], group[1], group[2], x, ys[0], act=act)
                elif len(group) == 1:
                    self.ctx.matmul(group[0], x, ys[0], act=act)
                else:
                    self.ctx.matmul_group(group, x, ys, act=act)

    def nbytes(self, tags=None):
        return sum(c[4] for c in self.calls if tags is None or c[5] in tags)

    def ncalls(self, tags=None):
        return sum(1 for c in self.calls if tags is None or c[5] in tags)

    def free(self):
        for t in self.tensors:
            t.free()


def gen_weight(torch, gen, out, inn):
    return torch.randn((out, inn), generator=gen, device="cuda", dtype=torch.float32).mul_(0.02)


def build_cfg2(ctx, torch, M, layers, seed):
    import beglin_amd
    gen = torch.Generator(device="cuda").manual_seed(seed)
    wl = Workload(ctx, torch)
    xs = {k: torch.randn((M, k), generator=gen, device="cuda") for k in (1536, 8960)}
    for _ in range(layers):
        for tag, shapes in qwen_layer_shapes():
            group = []
            nb = 0
            for out, inn in shapes:
                w = gen_weight(torch, gen, out, inn)
                group.append(ctx.quantize(beglin_amd.K_Q4G256SF, w))
                del w
                nb += alg_bytes(3, out, inn, 4, M) - 4 * M * inn - 4 * M * out     # weight bytes
            H = shapes[0][1]
            if tag == "mlp":          # x and y, and h written once and read once (g and u stay on chip)
                nb += 4 * M * H + 8 * M * shapes[0][0] + 4 * M * H
            else:
                nb += 4 * M * H + sum(4 * M * out for out, _ in shapes)
            wl.add(group, xs[H], beglin_amd.ACT_W4A8, nb, tag)
    return wl


def llama8b_layer_shapes():
    return [("qkv", [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096)]), ("o", [("o", 4096, 4096)]),
            ("gate_up", [("gate", 14336, 4096), ("up", 14336, 4096)]), ("down", [("down", 4096, 14336)])]


def cfg5_kinds(layers, seed):
    """Per-tensor (kind, bits): attention int8, MLP Q4G32H, a seeded 20% of all tensors qNg64 n=5."""
    import numpy as np
    rng = np.random.default_rng(seed + 5)
    out = []
    for _ in range(layers):
        lay = {}
        for _, shapes in llama8b_layer_shapes():
            for name, _, _ in shapes:
                base = (2, 8) if name in ("q", "k", "v", "o") else (5, 4)
                lay[name] = (4, 5) if rng.random() < 0.2 else base
        out.append(lay)
    return out


def build_cfg5(ctx, torch, M, layers, seed):
    """Fused groups only where the tensors share a kind (the engine's fused blobs are one kind)."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    wl = Workload(ctx, torch)
    xs = {k: torch.randn((M, k), generator=gen, device="cuda") for k in (4096, 14336)}
    kinds = cfg5_kinds(layers, seed)
    for li in range(layers):
        for tag, shapes in llama8b_layer_shapes():
            groups = {}
            for name, out, inn in shapes:
                groups.setdefault(kinds[li][name], []).append((name, out, inn))
            for (kind, bits), members in groups.items():
                group, nb = [], 0
                for name, out, inn in members:
                    w = gen_weight(torch, gen, out, inn)
                    group.append(ctx.quantize(kind, w, bits=bits))
                    del w
                    nb += alg_bytes(kind, out, inn, bits, M) - 4 * M * inn
                nb += 4 * M * members[0][2]
                wl.add(group, xs[members[0][2]], 0, nb, tag)
    wl.kinds = kinds
    return wl


def build_rotated(ctx, torch, kind, bits, out, inn, M, seed, act):
    """Enough distinct copies of one tensor that the rotation exceeds 2x the MALL."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    per = alg_bytes(kind, out, inn, bits, M)
    copies = max(4, int(2 * MALL_BYTES / per) + 1)
    wl = Workload(ctx, torch)
    x = torch.randn((M, inn), generator=gen, device="cuda")
    for _ in range(copies):
        w = gen_weight(torch, gen, out, inn)
        wl.add([ctx.quantize(kind, w, bits=bits, qng64_encoder=(bits != 4))], x, act, per, "gemv")
        del w
    return wl


# DeepSeek-V2-Lite routed MoE layer
DSV2 = dict(E=64, H=2048, I=1408, K=6, Ish=2 * 1408)
CFG4_FORMATS = [(5, 0), (2, 0)] + [(4, n) for n in range(7, 16)]


def wbytes(kind, out, inn, bits):
    return alg_bytes(kind, out, inn, bits, 0)


def shared_on_matrix_cores(kind, bits, T):
    """Whether bgl_moe_layer_dev runs the shared experts as a dense block on the matrix cores (the
    library's rule, bgl_moe.hip `shm`: >= BGL_MFMA_MIN_M = 16 tokens, BGL_NO_MFMA unset, and a kind
    bgl_mfma_ok accepts: Q4G64, Q4G32H, Q8G64, or qNg64 with 2 <= n <= MF_MAXN = 10)."""
    import beglin_amd
    if T < 16 or os.environ.get("BGL_NO_MFMA", "0") not in ("", "0"):
        return False
    return kind in (beglin_amd.K_Q4G64, beglin_amd.K_Q4G32H, beglin_amd.K_Q8G64) or (kind == beglin_amd.K_QNG64 and 2 <= bits <= 10)


class MoeWorkload:
    """`layers` routed MoE layers, each run whole on the device (bgl_moe_layer_dev: router, sort,
    gate/up/SwiGLU, down, combine, shared experts); layer = (stacks, shared, idx, w, out, bytes
    touched, experts touched, router weights)."""

    def __init__(self, ctx, torch, T, layers, seed):
        import beglin_amd
        self.ctx, self.torch, self.T = ctx, torch, T
        E, H, I, K, Ish = (DSV2[k] for k in ("E", "H", "I", "K", "Ish"))
        gen = torch.Generator(device="cuda").manual_seed(seed)
        rng = __import__("numpy").random.default_rng(seed)
        self.x = torch.randn((T, H), generator=gen, device="cuda")
        self.layers = []
        self.formats = []
        self.probe_sets = []          # per layer: the single tensors each gather launch streams
        self.shm = []                 # per layer: the shared experts run on the matrix cores (not in the gathers)
        for _ in range(layers):
            fm = [CFG4_FORMATS[i] for i in rng.integers(0, len(CFG4_FORMATS), E)]
            shf = CFG4_FORMATS[int(rng.integers(0, len(CFG4_FORMATS)))]
            stacks, handles = [], []
            for (o, i) in ((I, H), (I, H), (H, I)):
                ts = []
                for (k, b) in fm:
                    w = gen_weight(torch, gen, o, i)
                    ts.append(ctx.quantize(k, w, bits=b))
                    del w
                handles.append([t.h.value for t in ts])        # the stack owns them; kept for the read probe
                stacks.append(ctx.experts_from_tensors(ts))
            sh = []
            for (o, i) in ((Ish, H), (Ish, H), (H, Ish)):
                w = gen_weight(torch, gen, o, i)
                sh.append(ctx.quantize(shf[0], w, bits=shf[1]))
                del w
            # router [E][H] fp32 with N(0, 1/H) entries: N(0, 1) logits for N(0, 1) tokens
            rw = torch.randn((E, H), generator=gen, device="cuda") * (1.0 / H ** 0.5)
            idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
            w = torch.empty((T, K), device="cuda")
            ctx.moe_route(rw, self.x, K, idx, w)             # once here, to count the experts the step reads
            touched = sorted(set(idx.cpu().flatten().tolist()))
            nb = sum(2 * wbytes(fm[e][0], I, H, fm[e][1]) + wbytes(fm[e][0], H, I, fm[e][1]) for e in touched)
            nb += 2 * wbytes(shf[0], Ish, H, shf[1]) + wbytes(shf[0], H, Ish, shf[1])
            nb += 4 * E * H                                          # router weights
            nb += 2 * 4 * T * H                                      # x in, out
            out = torch.empty((T, H), device="cuda")
            self.layers.append((stacks, tuple(sh), idx, w, out, nb, len(touched), rw))
            self.formats.append((fm, shf))
            # the gather launches' tensors: routed gate+up (+ the shared gate+up, in the same launch
            # below 16 tokens or where the shared experts stay in the gathers), routed down, shared down
            view = lambda hs: [beglin_amd.Tensor(hs[e]) for e in touched]
            shm = shared_on_matrix_cores(shf[0], shf[1], T)
            self.shm.append(shm)
            gu = view(handles[0]) + view(handles[1])
            sets = [gu, view(handles[2]), [sh[0], sh[1]], [sh[2]]] if shm else [gu + [sh[0], sh[1]], view(handles[2]), [sh[2]]]
            self.probe_sets.append(sets)

    def run(self, tags=None):
        K = DSV2["K"]
        for stacks, sh, idx, w, out, _, _, rw in self.layers:
            self.ctx.moe_layer(rw, stacks[0], stacks[1], stacks[2], sh, self.x, K, out)

    def read_probe(self):
        """A plain read of exactly the weight bytes each gather launch streams, launch by launch
        (bgl_read_probe_dev takes up to 64 tensors, so a launch of more becomes several)."""
        for sets in self.probe_sets:
            for ts in sets:
                for i in range(0, len(ts), 64):
                    self.ctx.read_probe(ts[i:i + 64])

    def nbytes(self, tags=None):
        return sum(l[5] for l in self.layers)

    def ncalls(self, tags=None):
        return len(self.layers)

    def free(self):
        for stacks, sh, *_ in self.layers:
            for t in list(stacks) + list(sh):
                t.free()


EAGER = False        # --eager: launch the step's kernels directly (counter-collection runs)


def time_graph(torch, stream, fn, steps, warmup):
    with torch.cuda.stream(stream):
        fn()                                   # eager once: reserves every scratch buffer
    torch.cuda.synchronize()
    if EAGER:
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            e0.record(stream)
            for _ in range(steps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
        return e0.elapsed_time(e1) / steps, wall, None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / steps, wall, g


def plain_read(ctx, torch, stream, wl, steps):
    """The same step with every call replaced by a plain streaming read of exactly its tensors'
    device bytes (bgl_read_probe_dev, 1024 workgroups x 256 threads, 16-byte loads), graph-timed
    the same way: the memory system's floor for this sequence of launches."""
    def reads():
        for group, *_ in wl.calls:
            ctx.read_probe(group)
    ms, _, _ = time_graph(torch, stream, reads, steps, 3)
    return ms


# The kernel sources behind each workload's dominant kernel (its file and the headers it includes).
KERNEL_SOURCES = {
    "cfg2": ("bgl_mlp_q.hip", "bgl_gemv.hip", "bgl_gemv_q.h", "bgl_gemv_impl.h", "bgl_device.h", "bgl_kernels.h"),
    "cfg1": ("bgl_gemv_x.hip", "bgl_gemv_x.h", "bgl_prep.hip", "bgl_device.h", "bgl_kernels.h"),
    "cfg3": ("bgl_gemv_x.hip", "bgl_gemv_x.h", "bgl_prep.hip", "bgl_device.h", "bgl_kernels.h"),
    "cfg4": ("bgl_moe_x.hip", "bgl_moe_x.h", "bgl_moe.hip", "bgl_gemv_x.h", "bgl_prep.hip", "bgl_mfma.hip", "bgl_mlp.hip",
             "bgl_device.h", "bgl_kernels.h"),
    "cfg5": ("bgl_mfma.hip", "bgl_device.h", "bgl_kernels.h"),
}


def kernel_sources_sha16(workload="cfg2"):
    """Hash of a workload's kernel sources: a committed counter reading is used only while it matches."""
    import hashlib
    h = hashlib.sha256()
    for f in KERNEL_SOURCES[workload]:
        with open(os.path.join(ROOT, "beglin_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def traffic_key(args):
    """The profiles/traffic.json entry measured on exactly this bench configuration."""
    base = {"cfg3": f"cfg3_{args.shape}_n{args.bits}"}.get(args.workload, args.workload)
    return f"{base}_M{args.M}_L{args.layers}" if args.workload in ("cfg2", "cfg4", "cfg5") else f"{base}_M{args.M}"


def attach_traffic(roof, args, alg_per_launch):
    """HBM traffic per launch of the dominant kernel from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes over this same configuration, scaled by a known-size copy -- used only while
    the kernel sources it was measured on are the current ones."""
    try:
        tr = json.load(open(os.path.join(ROOT, "profiles", "traffic.json")))[traffic_key(args)]
    except (OSError, KeyError, ValueError):
        roof["traffic_note"] = f"no committed counter reading for {traffic_key(args)}"
        return
    if tr.get("kernel_sources_sha16") != kernel_sources_sha16(args.workload):
        roof["traffic_note"] = "profiles/traffic.json was measured on other kernel sources: not used"
        return
    roof["traffic"] = tr["traffic_bytes_per_launch"]
    roof["traffic_over_algorithmic"] = round(tr["traffic_bytes_per_launch"] / alg_per_launch, 3)
    roof["traffic_source"] = tr["summary"]


def time_prep(ctx, torch, stream, wl, steps, tags):
    """Graph-timed activation-prep kernels alone (one per call of the given call types: the ones
    whose path launches a prep kernel)."""
    def prep_only():
        for group, x, ys, act, _, tag in wl.calls:
            if tag in tags:
                ctx.prep_only(x, act, group[0])
    ms, _, _ = time_graph(torch, stream, prep_only, steps, 2)
    return ms


def moe_roofline(ctx, torch, stream, wl, reps):
    """The gather kernel's own time: eager steps with an event pair around every launch (bgl_prof_*),
    summed per phase on the context's stream; achieved = step bytes / gather-GEMV time."""
    ctx.prof_enable(True)
    ctx.prof_read()
    with torch.cuda.stream(stream):
        for _ in range(reps):
            wl.run()
    ctx.sync()
    ph = ctx.prof_read()
    ctx.prof_enable(False)
    g_ms, g_n = ph["gemv"][0] / reps, ph["gemv"][1] // reps
    p_ms, p_n = ph["prep"][0] / reps, ph["prep"][1] // reps
    o_ms, o_n = ph["other"][0] / reps, ph["other"][1] // reps
    achieved = wl.nbytes() / (g_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "k_moe_x / k_moe_x2 gathers (bgl_moe_x.h); from 16 tokens the shared experts' k_gemm_mfma (bgl_mfma.hip)",
            "launches_per_step": g_n, "kernel_us_per_launch": round(g_ms * 1e3 / max(g_n, 1), 3),
            "bytes_per_launch": round(wl.nbytes() / max(g_n, 1)),
            "prep_us_per_step": round(p_ms * 1e3, 2), "prep_launches": p_n,
            "route_bucket_combine_us_per_step": round(o_ms * 1e3, 2), "route_bucket_combine_launches": o_n,
            "timing": f"eager, event pair per launch, {reps} steps"}


MFMA_F16_PEAK_TFLOPS = 2500.0


def mfma_roofline(ctx, torch, stream, wl, M, reps):
    """k_gemm_mfma's own time: eager steps with an event pair per launch (phase 1 = the GEMM
    kernel, which also converts the activations; 2 = K-split reduce); achieved = step bytes / GEMM
    time.
    Matrix-core rate: the kernel issues 2 (hi, lo) x ceil(M/16)*16 x N_tiles*64 x K x 2 flops per
    call; useful flops are 2*M*N*K."""
    ctx.prof_enable(True)
    ctx.prof_read()
    with torch.cuda.stream(stream):
        for _ in range(reps):
            wl.run()
    ctx.sync()
    ph = ctx.prof_read()
    ctx.prof_enable(False)
    g_ms, g_n = ph["gemv"][0] / reps, ph["gemv"][1] // reps
    o_ms = ph["other"][0] / reps
    achieved = wl.nbytes() / (g_ms * 1e-3) / 1e9
    useful, issued = 0.0, 0.0
    mp = (M + 15) // 16 * 16
    for group, x, ys, act, nb, tag in wl.calls:
        for t in group:
            inf = t.info()
            useful += 2.0 * M * inf["out"] * inf["inn"]
            issued += 2.0 * 2 * mp * ((inf["out"] + 63) // 64 * 64) * inf["inn"]
    tflops = issued / (g_ms * 1e-3) / 1e12
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_gemm_mfma (bgl_mfma.hip)",
            "launches_per_step": g_n, "kernel_us_per_launch": round(g_ms * 1e3 / max(g_n, 1), 3),
            "bytes_per_launch": round(wl.nbytes() / max(g_n, 1)),
            "mfma": {"issued_tflops": round(tflops, 1), "useful_tflops": round(useful / (g_ms * 1e-3) / 1e12, 1),
                     "peak_fp16_tflops": MFMA_F16_PEAK_TFLOPS, "util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)},
            "reduce_us_per_step": round(o_ms * 1e3, 2),
            "timing": f"eager, event pair per launch, {reps} steps"}


# ------------------------------------------------------------------------------------- CPU baseline
def cpu_baseline_cfg5(M, budget_s, seed):
    """The reference's fp32-activation GEMV restated (or_pool_gemv_f32 per column, q4pool row-block
    split) on one layer of the same shapes and precision map; timed columns scaled to M."""
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle
    orc = Oracle()
    rng = np.random.default_rng(seed)
    T = host_threads()
    pool = orc.lib.or_pool_create(T, 14336)
    kinds = cfg5_kinds(1, seed)[0]
    mats, nb = [], 0
    for _, shapes in llama8b_layer_shapes():
        for name, out, inn in shapes:
            kind, bits = kinds[name]
            w = (rng.standard_normal((out, inn), dtype=np.float32) * np.float32(0.02))
            if kind == 2:
                pk, sc = orc.quantize_q8g64(w)
            elif kind == 5:
                pk, sc = orc.quantize_q4g32h(w)
            else:
                pk, sc = orc.quantize_qng64(w, bits)
            mats.append((kind, bits, pk, sc, out, inn, np.zeros(out, np.float32)))
            nb += alg_bytes(kind, out, inn, bits, M)
    xs = {k: rng.standard_normal((M, k), dtype=np.float32) for k in (4096, 14336)}
    P = lambda a: C.c_void_p(a.ctypes.data)
    t0 = time.perf_counter()
    cols = 0
    while True:
        for kind, bits, pk, sc, out, inn, y in mats:
            xr = np.ascontiguousarray(xs[inn][cols % M])
            orc.lib.or_pool_gemv_f32(pool, kind, bits, P(pk), P(sc), P(xr), None, P(y), out, inn)
        cols += 1
        if time.perf_counter() - t0 >= budget_s or cols >= M:
            break
    el = time.perf_counter() - t0
    dt = el / cols * M                                    # one layer at M columns
    orc.lib.or_pool_destroy(pool)
    return {"value": round(nb / dt / 1e9, 3), "unit": "GB/s", "cores": T, "host_nproc": host_nproc(), "kind": "port",
            "us_per_layer": round(dt * 1e6, 1),
            "sample": f"one Llama-3.1-8B layer (7 tensors, same precision map), {cols} of {M} columns timed "
                      f"({el:.1f} s) and scaled to {M}, per column through the row-block pool, {T} threads"}


def cpu_baseline_cfg4(wl, budget_s, seed):
    """moe_ffn_batched's portable C restatement (router scores, routing and the bucketed FFN with
    every expert matvec's rows split over the row-block pool, moe_matvec_af_mt) on layer 0's router
    and formats, for min(T, 8) tokens; only the experts those tokens touch are quantized (the others
    are never read)."""
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle, expert_array
    orc = Oracle()
    rng = np.random.default_rng(seed + 1)
    E, H, I, K, Ish = (DSV2[k] for k in ("E", "H", "I", "K", "Ish"))
    fm, shf = wl.formats[0]
    rw = wl.layers[0][7].cpu().numpy()
    T = min(wl.T, 8)
    NT = host_threads()
    pool = orc.lib.or_pool_create(NT, 1)
    x = rng.standard_normal((T, H), dtype=np.float32)
    idx, w = orc.route(orc.router_logits(rw, x), K)
    touched = sorted(set(idx.flatten().tolist()))

    def q(k, b, o, i):
        m = (rng.standard_normal((o, i), dtype=np.float32) * np.float32(0.02))
        if k == 5:
            p, sc = orc.quantize_q4g32h(m)
        elif k == 2:
            p, sc = orc.quantize_q8g64(m)
        else:
            p, sc = orc.quantize_qng64(m, b)
        return (k, b if k == 4 else (8 if k == 2 else 4), p, sc)

    dummy = (5, 4, np.zeros((1, 1), np.uint8), np.zeros((1, 1), np.uint16))
    gate, up, down = [dummy] * E, [dummy] * E, [dummy] * E
    gate, up, down = list(gate), list(up), list(down)
    nb = 0
    for e in touched:
        k, b = fm[e]
        gate[e], up[e], down[e] = q(k, b, I, H), q(k, b, I, H), q(k, b, H, I)
        nb += 2 * wbytes(k, I, H, b) + wbytes(k, H, I, b)
    shared = (q(shf[0], shf[1], Ish, H), q(shf[0], shf[1], Ish, H), q(shf[0], shf[1], H, Ish))
    nb += 2 * wbytes(shf[0], Ish, H, shf[1]) + wbytes(shf[0], H, Ish, shf[1]) + 4 * E * H + 2 * 4 * T * H
    (ga, gk), (ua, uk), (da, dk), (sa, sk) = expert_array(gate), expert_array(up), expert_array(down), expert_array(list(shared))
    out = np.zeros((T, H), np.float32)
    P = lambda a: C.c_void_p(a.ctypes.data)
    t0 = time.perf_counter()
    reps = 0
    while True:
        idx, w = orc.route(orc.router_logits(rw, x), K)
        z = C.sizeof(sa[0])
        orc.lib.or_pool_moe_ffn_bucketed(C.c_void_p(pool), ga, ua, da, E, C.byref(sa, 0), C.byref(sa, z), C.byref(sa, 2 * z),
                                         H, I, Ish, T, K, P(x), P(idx), P(w), P(out))
        reps += 1
        if time.perf_counter() - t0 >= budget_s or reps >= 1000:
            break
    dt = (time.perf_counter() - t0) / reps
    orc.lib.or_pool_destroy(pool)
    return {"value": round(nb / dt / 1e9, 3), "unit": "GB/s", "cores": NT, "host_nproc": host_nproc(), "kind": "port",
            "us_per_layer": round(dt * 1e6, 1),
            "sample": f"layer 0, {T} token(s), router + {len(touched)} experts touched + shared ({nb / 1e6:.1f} MB), "
                      f"or_moe_router_logits + or_moe_route + or_pool_moe_ffn_bucketed (rows over {NT} threads), "
                      f"{reps} calls over {dt * reps:.1f} s"}


def cpu_baseline_cfg2(M, budget_s, layers=2, seed=7):
    """The reference's threaded CPU path (gemv_q4g256sf_sdot_mt, q4gemv_g256.h:339-364 semantics,
    q4pool row-block split) on `layers` layers of the same shapes."""
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle
    orc = Oracle()
    rng = np.random.default_rng(seed)
    T = host_threads()
    pool = orc.lib.or_pool_create(T, 8960)
    one, lb = [], 0
    for _, shapes in qwen_layer_shapes():
        for out, inn in shapes:
            w = (rng.standard_normal((out, inn), dtype=np.float32) * np.float32(0.02))
            pk, ws, sub = orc.quantize_g256sf(w)
            one.append((pk, ws, sub, out, inn))
            lb += alg_bytes(3, out, inn, 4, 1)
    # distinct copies of one quantized layer until the footprint passes ROTATE_BYTES, so every pass
    # streams its weights from memory rather than the host caches
    layers = max(layers, -(-ROTATE_BYTES // int(lb)))
    mats, nbytes = [], 0
    for _ in range(layers):
        for pk, ws, sub, out, inn in one:
            mats.append((pk.copy(), ws.copy(), sub.copy(), out, inn, np.zeros(out, np.float32)))
        nbytes += lb
    xs = {k: rng.standard_normal(k, dtype=np.float32) for k in (1536, 8960)}
    P = lambda a: C.c_void_p(a.ctypes.data)

    def one_pass():
        for pk, ws, sub, out, inn, y in mats:
            orc.lib.or_pool_gemv_g256sf_sdot(pool, P(pk), P(ws), P(sub), P(xs[inn]), None, P(y), out, inn)

    one_pass()
    t0 = time.perf_counter()
    reps = 0
    while True:
        one_pass()
        reps += 1
        if time.perf_counter() - t0 >= budget_s or reps >= 1000000:
            break
    dt = (time.perf_counter() - t0) / reps
    orc.lib.or_pool_destroy(pool)
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": T, "host_nproc": host_nproc(), "kind": "port",
            "us_per_layer": round(dt / layers * 1e6, 1),
            "sample": f"{layers} copies of one Qwen2.5-1.5B layer of q4g256sf (7 projections each, {nbytes / 1e6:.1f} MB "
                      f"rotated), M=1 W4A8, {reps} passes over {dt * reps:.1f} s, {T} threads (the box's 16-core share)"}


def cpu_baseline_rotated(kind, bits, out, inn, budget_s, seed=7):
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle
    orc = Oracle()
    rng = np.random.default_rng(seed)
    T = host_threads()
    pool = orc.lib.or_pool_create(T, inn)
    w = (rng.standard_normal((out, inn), dtype=np.float32) * np.float32(0.02))
    if kind == 5:
        pk, sc = orc.quantize_q4g32h(w)
    else:
        pk, sc = orc.quantize_qng64(w, bits)
    x = rng.standard_normal(inn, dtype=np.float32)
    y = np.zeros(out, np.float32)
    P = lambda a: C.c_void_p(a.ctypes.data)
    nb = alg_bytes(kind, out, inn, bits, 1)
    ncopy = max(1, -(-ROTATE_BYTES // int(nb)))               # distinct copies: >= ROTATE_BYTES in all
    copies = [(pk.copy(), sc.copy()) for _ in range(ncopy)]
    orc.lib.or_pool_gemv_f32(pool, kind, bits, P(pk), P(sc), P(x), None, P(y), out, inn)
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < budget_s and reps < 100000:
        cpk, csc = copies[reps % ncopy]
        orc.lib.or_pool_gemv_f32(pool, kind, bits, P(cpk), P(csc), P(x), None, P(y), out, inn)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    orc.lib.or_pool_destroy(pool)
    return {"value": round(nb / dt / 1e9, 3), "unit": "GB/s", "cores": T, "host_nproc": host_nproc(), "kind": "port",
            "us_per_call": round(dt * 1e6, 1),
            "sample": f"{ncopy} rotated copies of one {out}x{inn} tensor (kind {kind}, n={bits}; {ncopy * nb / 1e6:.0f} MB), "
                      f"{reps} calls over {dt * reps:.1f} s, {T} threads (the box's 16-core share)"}


def copy_calib(mib):
    import torch
    n = (mib << 20) // 4
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calib_bytes_read": n * 4, "copy_calib_bytes_written": n * 4, "launches": 5}), flush=True)


# ------------------------------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="cfg2", choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5"])
    ap.add_argument("--M", type=int, default=None,
                    help="activation rows (default 1; cfg2: 1, 4 or 8; cfg5: 32); cfg4: tokens T (1, 8, 64)")
    ap.add_argument("--layers", type=int, default=None, help="cfg2: 28 layers; cfg4: 8 MoE layers; cfg5: 4 layers")
    ap.add_argument("--bits", type=int, default=15, help="cfg3: qNg64 width n")
    ap.add_argument("--shape", default="gate", choices=["gate", "down"], help="cfg3: MLP gate (K=4096) or down (K=14336)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--eager", action="store_true", help="no HIP graph: launch every kernel directly (for "
                    "rocprofv3 --pmc passes); timings then include host launch gaps")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB 5 times (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes) and exit")
    ap.add_argument("--counter-steps", type=int, default=0, metavar="N",
                    help="only build the workload and launch exactly N eager steps, no timing (a rocprofv3 --pmc "
                         "pass over it then holds N steps' dispatches of the path's kernels and nothing else)")
    args = ap.parse_args()
    if args.copy_calib:
        copy_calib(args.copy_calib)
        return
    global EAGER
    EAGER = args.eager

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py: this build measures one GPU; --gpus {max(args.gpus, world)} is not supported "
              "(the path would shard by output rows with one all-gather of y -- not built).", file=sys.stderr)
        sys.exit(2)

    import torch

    import beglin_amd
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    stream = torch.cuda.Stream()
    ctx = beglin_amd.Context(0, stream=stream.cuda_stream)
    if args.layers is None:
        args.layers = {"cfg4": 8, "cfg5": 4}.get(args.workload, 28)
    if args.M is None:
        args.M = 32 if args.workload == "cfg5" else 1
    M = args.M
    if args.workload == "cfg5":
        with torch.cuda.stream(stream):
            wl = build_cfg5(ctx, torch, M, args.layers, args.seed)
        workload = (f"cfg5: Llama-3.1-8B projections x{args.layers} layers, M={M} fp32 rows, attention int8, "
                    f"MLP int4 g32, seeded 20% qNg64 n=5, matrix-core path")
        dtype = "fp16 (exact codes; activations hi+lo fp16)"
        nq = sum(1 for lay in wl.kinds for v in lay.values() if v == (4, 5))
        cfg = {"workload": workload, "M": M, "layers": args.layers, "calls_per_step": wl.ncalls(),
               "qng64_n5_tensors": nq, "tensors": 7 * args.layers, "bytes_per_step": int(wl.nbytes()), "seed": args.seed}
    elif args.workload == "cfg2":
        with torch.cuda.stream(stream):
            wl = build_cfg2(ctx, torch, M, args.layers, args.seed)
        torch.cuda.synchronize()
        workload = (f"cfg2: Qwen2.5-1.5B decode layer x{args.layers}, q4g256sf W4A8 GEMV, 7 projections as forward_token "
                    f"issues them (fused qkv, o, MLP block gate+up -> SwiGLU -> down), M={M}")
        dtype = DT_W4A8
        cfg = {"workload": workload, "layers": args.layers, "M": M, "format": "q4g256sf", "activations": "W4A8 (int8, group 256)",
               "calls_per_step": wl.ncalls(), "weight_bytes_per_step": int(wl.nbytes()), "seed": args.seed}
    elif args.workload == "cfg1":
        with torch.cuda.stream(stream):
            wl = build_rotated(ctx, torch, 5, 4, 8960, 1536, M, args.seed, beglin_amd.ACT_F32)
        workload = f"cfg1: int4 g32 fp16-scale GEMV K=1536 N=8960, fp32 activations, M={M}, {wl.ncalls()} rotated copies"
        dtype = DT_F32ACT
        cfg = {"workload": workload, "M": M, "format": "q4g32h", "copies": wl.ncalls(), "seed": args.seed}
    elif args.workload == "cfg4":
        with torch.cuda.stream(stream):
            wl = MoeWorkload(ctx, torch, M, args.layers, args.seed)
        touched = [l[6] for l in wl.layers]
        workload = (f"cfg4: DeepSeek-V2-Lite routed MoE layer x{args.layers} (router + top-6 + experts + shared on "
                    f"the device), E=64+2 shared, hidden 2048, inter 1408, T={M}, per-expert precision from the seed")
        dtype = DT_F32ACT
        cfg = {"workload": workload, "T": M, "layers": args.layers, "experts_touched_per_layer": touched,
               "formats": "q4g32h | q8g64 | qNg64 n=7..15 per expert (fp32 activations)", "seed": args.seed,
               "bytes_per_step": int(wl.nbytes())}
    else:
        out, inn = (14336, 4096) if args.shape == "gate" else (4096, 14336)
        with torch.cuda.stream(stream):
            wl = build_rotated(ctx, torch, 4, args.bits, out, inn, M, args.seed, beglin_amd.ACT_F32)
        workload = f"cfg3: qNg64 n={args.bits} GEMV {out}x{inn} (Llama-3.1-8B MLP {args.shape}), fp32 activations, M={M}, {wl.ncalls()} rotated copies"
        dtype = DT_F32ACT
        cfg = {"workload": workload, "M": M, "format": f"qNg64 n={args.bits}", "copies": wl.ncalls(), "seed": args.seed}
    torch.cuda.synchronize()

    if args.counter_steps:
        with torch.cuda.stream(stream):
            for _ in range(args.counter_steps):
                wl.run()
        torch.cuda.synchronize()
        print(json.dumps({"counter_steps": args.counter_steps, "config": cfg, "calls_per_step": wl.ncalls(),
                          "bytes_per_step": int(wl.nbytes())}), flush=True)
        return

    step_ms, wall, graph = time_graph(torch, stream, wl.run, args.steps, args.warmup)
    nbytes = wl.nbytes()
    value = nbytes / (step_ms * 1e-3) / 1e9

    # per-call latency of each call type (graph over all its instances)
    if args.workload == "cfg5":
        per_call = {"layer": {"us": round(step_ms * 1e3 / args.layers, 2), "GB/s": round(value, 1)}}
        roof = mfma_roofline(ctx, torch, stream, wl, M, max(3, args.steps // 10))
        attach_traffic(roof, args, roof["bytes_per_launch"])
        pr_ms = plain_read(ctx, torch, stream, wl, max(5, args.steps // 5))
        roof["plain_read"] = {"us_per_step": round(pr_ms * 1e3, 2), "GB/s": round(wl.nbytes() / (pr_ms * 1e-3) / 1e9, 1),
                              "step_over_plain": round(step_ms / pr_ms, 3),
                              "how": "bgl_read_probe_dev over each call's tensors, 1024 x 256 threads, graph-timed"}
        cpu = None if args.no_cpu else cpu_baseline_cfg5(M, args.cpu_seconds, args.seed)
        finish(args, wl, ctx, graph, value, step_ms, wall, dtype, cfg, per_call, roof, cpu)
        return
    if args.workload == "cfg4":
        per_call = {"moe_layer": {"us": round(step_ms * 1e3 / args.layers, 2), "GB/s": round(value, 1)}}
        roof = moe_roofline(ctx, torch, stream, wl, max(3, args.steps // 10))
        attach_traffic(roof, args, roof["bytes_per_launch"])
        pr_ms, _, _ = time_graph(torch, stream, wl.read_probe, max(5, args.steps // 5), 3)
        roof["plain_read"] = {"us_per_step": round(pr_ms * 1e3, 2), "GB/s": round(wl.nbytes() / (pr_ms * 1e-3) / 1e9, 1),
                              "step_over_plain": round(step_ms / pr_ms, 3),
                              "how": "bgl_read_probe_dev over the touched experts' and the shared experts' tensors of "
                                     "each gather launch (launches of up to 64 tensors), 1024 x 256 threads, graph-timed; "
                                     "router weights and activations not read",
                              "shared_on_matrix_cores_per_layer": [bool(v) for v in wl.shm]}
        cpu = None if args.no_cpu else cpu_baseline_cfg4(wl, args.cpu_seconds, args.seed)
        finish(args, wl, ctx, graph, value, step_ms, wall, dtype, cfg, per_call, roof, cpu)
        return

    per_call = {}
    tags = sorted({c[5] for c in wl.calls})
    for tag in tags:
        ms, _, _ = time_graph(torch, stream, lambda: wl.run([tag]), max(5, args.steps // 5), 3)
        n = wl.ncalls([tag])
        per_call[tag] = {"us": round(ms * 1e3 / n, 2), "GB/s": round(wl.nbytes([tag]) / (ms * 1e-3) / 1e9, 1)}

    # Launches per call type, and which call types launch an activation-prep kernel: one profiled
    # eager run of each.  (The fused W4A8 kernel and the one-column fp32 GEMV over a short K make
    # their operands themselves; several W4A8 columns over a long K and long fp32 K are quantized
    # up front.  The MLP block at one W4A8 column is one launch, otherwise three.)
    prep_tags, launches_of, kern_of = [], {}, {}
    for tag in tags:
        ctx.prof_enable(True)
        ctx.prof_read()
        with torch.cuda.stream(stream):
            wl.run([tag])
        ctx.sync()
        pr = ctx.prof_read()
        if pr["prep"][1] > 0:
            prep_tags.append(tag)
        launches_of[tag] = sum(v[1] for v in pr.values())
        kern_of[tag] = pr["gemv"][1] + pr["other"][1]          # the launches after any prep kernel
        ctx.prof_enable(False)
    launches = sum(launches_of.values())
    if args.workload == "cfg2" and launches_of.get("mlp") == wl.ncalls(["mlp"]):
        # The dominant kernel is the single-launch MLP block (22 of the layer's 25 MB): its average
        # launch duration is the graph of the step's MLP calls alone (HIP events on the context's
        # stream around the timed replays) over their count.
        n_m = wl.ncalls(["mlp"])
        b_m = wl.nbytes(["mlp"]) / n_m
        us_m = per_call["mlp"]["us"]
        achieved = b_m / (us_m * 1e-6) / 1e9
        others = {t: {"launches_per_step": launches_of[t], "us_per_launch": per_call[t]["us"]} for t in tags if t != "mlp"}
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "k_mlp_q<fmt,TRG,TRD> (bgl_mlp_q.hip): gate+up, SwiGLU and down of one MLP block in one launch",
                "launches_per_step": n_m, "kernel_us_per_launch": round(us_m, 3), "bytes_per_launch": round(b_m),
                "how": "graph of the step's MLP launches alone, HIP events on the context's stream",
                "step_launches": launches, "other_kernels": {"k_gemv_q<fmt,TR,QP,MB> (bgl_gemv.hip)": others}}
        dom_bytes = b_m
    else:
        # The dominant kernel is the GEMV; where it is the only kernel of the step (one-column
        # fp32 GEMV over a short K) its average launch duration is the graph-timed step over the
        # launches per step.  Call types whose path adds an activation-prep kernel have those timed
        # the same way from a graph of the prep alone, subtracted from the step.
        prep_ms = 0.0
        if prep_tags:
            prep_ms = time_prep(ctx, torch, stream, wl, max(5, args.steps // 5), set(prep_tags))
        k_ms = max(step_ms - prep_ms, 1e-6)
        klaunches = max(sum(kern_of.values()), 1)              # prep launches are timed apart
        achieved = nbytes / (k_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": ("k_gemv_q<fmt,TR,QP,MB> (bgl_gemv.hip) + k_swiglu (bgl_mlp.hip)" if args.workload == "cfg2" else
                           "k_gemv_x<fmt,n,TR,FUSE> (bgl_gemv_x.hip)" if M == 1 else "k_gemv<fmt,act,n,MB> (bgl_gemv.hip)"),
                "launches_per_step": klaunches, "kernel_us_per_launch": round(k_ms * 1e3 / klaunches, 3),
                "prep_launches_per_step": launches - klaunches,
                "prep_us_per_launch": round(prep_ms * 1e3 / max(launches - klaunches, 1), 3), "prep_call_types": prep_tags,
                "bytes_per_launch": round(nbytes / klaunches)}
        dom_bytes = nbytes / klaunches

    # the plain-read floor for the same bytes and launch count, measured in this run
    pr_ms = plain_read(ctx, torch, stream, wl, max(5, args.steps // 5))
    roof["plain_read"] = {"us_per_step": round(pr_ms * 1e3, 2), "us_per_launch": round(pr_ms * 1e3 / wl.ncalls(), 3),
                          "GB/s": round(nbytes / (pr_ms * 1e-3) / 1e9, 1), "step_over_plain": round(step_ms / pr_ms, 3),
                          "how": "bgl_read_probe_dev over each call's tensors (one launch per call), 1024 x 256 threads, "
                                 "graph-timed"}

    attach_traffic(roof, args, dom_bytes)

    cpu = None
    if not args.no_cpu:
        if args.workload == "cfg2":
            cpu = cpu_baseline_cfg2(M, args.cpu_seconds)
        elif args.workload == "cfg1":
            cpu = cpu_baseline_rotated(5, 4, 8960, 1536, args.cpu_seconds)
        else:
            out, inn = (14336, 4096) if args.shape == "gate" else (4096, 14336)
            cpu = cpu_baseline_rotated(4, args.bits, out, inn, args.cpu_seconds)

    finish(args, wl, ctx, graph, value, step_ms, wall, dtype, cfg, per_call, roof, cpu)


def finish(args, wl, ctx, graph, value, step_ms, wall, dtype, cfg, per_call, roof, cpu):
    line = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations)",
            "config": cfg, "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4), "us_per_call": per_call,
            "wall_s_timed": round(wall, 3), "roofline": roof, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    del graph
    wl.free()
    ctx.close()


if __name__ == "__main__":
    main()
