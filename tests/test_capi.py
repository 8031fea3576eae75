"""CPU-side checks of the C-ABI library: it loads, exports every symbol include/beglin_qgemv.h
declares, and its signatures table covers the header (no compute calls: no GPU here)."""
import ctypes as C
import subprocess

import pytest

from beglin_amd import capi


def test_library_exports_every_header_symbol():
    lib = capi.load()
    missing = [s for s in capi.header_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_signature_table_matches_header():
    declared = set(capi.header_symbols())
    bound = {n for n, _, _ in capi.SIGNATURES}
    assert declared == bound, (declared ^ bound)


def test_exports_are_extern_c_and_gfx950():
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True).stdout
    names = {l.split()[-1] for l in out.splitlines() if " T " in l}
    for s in capi.header_symbols():
        assert s in names, f"{s} not exported with C linkage"
    # the device code object inside is for gfx950 only
    blob = open(capi.LIB_PATH, "rb").read()
    assert b"gfx950" in blob and b"gfx942" not in blob


def test_no_device_is_reported_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present: covered by the gpu tests")
    lib = capi.load()
    assert lib.bgl_available() == 0
    h = C.c_void_p()
    rc = lib.bgl_ctx_create(0, None, C.byref(h))
    assert rc != 0 and b"device" in lib.bgl_last_error()


def test_build_compiles_every_hip_source():
    """Every .hip file under beglin_amd/csrc is a unit of the library build (the MoE gather's kernel
    instances are one unit each: a unit left out would leave its launcher unresolved at load)."""
    import os
    from beglin_amd import build
    on_disk = {f for f in os.listdir(build.CSRC) if f.endswith(".hip")}
    assert on_disk == set(build.SOURCES), on_disk ^ set(build.SOURCES)
    assert len(build.SOURCES) == len(set(build.SOURCES))


def test_moe_kernel_instances_are_all_defined():
    """All ten MoE gather launch helpers the host side calls are defined in the library (each is
    explicitly instantiated in its own unit; a missing one would leave the load unresolved)."""
    out = subprocess.run(["nm", "-C", "--defined-only", capi.LIB_PATH], capture_output=True, text=True).stdout
    go = [l.split(" ", 2)[2] for l in out.splitlines()
          if (" T " in l or " W " in l) and ("moe_x_go<" in l or "moe_x2_go<" in l)]
    assert len(go) == 10 and len(set(go)) == 10, go
