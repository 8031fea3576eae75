"""Builds beglin_amd/libbeglin_hip.so (the C-ABI of include/beglin_qgemv.h) for gfx950 with hipcc.

Run as `python -m beglin_amd.build` or through __graft_entry__.build().  Always compiles."""
import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libbeglin_hip.so")
# The MoE gather's kernel instances are one unit each (bgl_moe_x_i*.hip) so they compile in
# parallel; the longest units come first.
SOURCES = [f"bgl_moe_x_i{i}.hip" for i in range(10)] + [
    "bgl_gemv.hip", "bgl_moe.hip", "bgl_mfma.hip", "bgl_gemv_x.hip", "bgl_api.hip", "bgl_prep.hip", "bgl_moe_x.hip",
    "bgl_registry.hip", "bgl_loader.hip", "bgl_mlp.hip", "bgl_mlp_q.hip", "bgl_gemv_qm.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
    # every fp32 expression rounds as written: the packers and the W4A8 fold must reproduce the
    # reference bit for bit, and HIP would otherwise contract a*b+c into FMAs
    "-ffp-contract=off",
    # no packed-fp32 VALU ops anywhere (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc", "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def build(verbose=False, jobs=None):
    t0 = time.time()
    objs = []
    procs = []
    for s in SOURCES:
        src = os.path.join(CSRC, s)
        obj = os.path.join(CSRC, s.replace(".hip", ".o"))
        objs.append(obj)
        cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
        procs.append((s, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = False
    for s, p in procs:
        out, _ = p.communicate()
        out = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            failed = True
            sys.stderr.write(f"--- hipcc {s} failed ---\n{out}\n")
        elif verbose and out.strip():
            sys.stderr.write(out + "\n")
    if failed:
        raise RuntimeError("HIP build failed")
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
