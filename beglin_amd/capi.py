"""ctypes binding of include/beglin_qgemv.h (libbeglin_hip.so).

The library is the product; this module only declares its C signatures.  Importing it fails
loudly when the shared library is missing -- there is no CPU fallback anywhere in the package."""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# BGL_LIB names another build of the same C-ABI (A/B timing of two builds); default: the in-tree one
LIB_PATH = os.environ.get("BGL_LIB") or os.path.join(HERE, "libbeglin_hip.so")

# mirrors of the header's enums
K_Q4G64, K_Q8G64, K_Q4G256SF, K_QNG64, K_Q4G32H = 1, 2, 3, 4, 5
K_Q4G64A, K_F16, K_F32, K_MXFP4, K_Q4G256P = 6, 7, 8, 9, 10
ACT_F32, ACT_W4A8 = 0, 1

_P = C.c_void_p
_I = C.c_int
_L = C.c_long


class bgl_wt(C.Structure):
    _fields_ = [("kind", C.c_int), ("bits", C.c_int), ("out", C.c_int), ("in_", C.c_int),
                ("packed", C.c_void_p), ("scales", C.c_void_p), ("sub", C.c_void_p)]


# (name, restype, argtypes) for every entry point declared in include/beglin_qgemv.h
SIGNATURES = [
    ("bgl_available", _I, []),
    ("bgl_last_error", C.c_char_p, []),
    ("bgl_ctx_create", _I, [_I, _P, C.POINTER(_P)]),
    ("bgl_ctx_destroy", None, [_P]),
    ("bgl_synchronize", _I, [_P]),
    ("bgl_ctx_check", _I, [_P]),
    ("bgl_ctx_stream", _P, [_P]),
    ("bgl_prof_enable", _I, [_P, _I]),
    ("bgl_prof_read", _I, [_P, C.POINTER(C.c_double), C.POINTER(_I), _I]),
    ("bgl_bind", _I, [_P, C.POINTER(bgl_wt), C.POINTER(_P)]),
    ("bgl_quantize_dev", _I, [_P, _I, _I, _I, _P, _I, _I, C.POINTER(_P), _P, _P, _P]),
    ("bgl_tensor_free", None, [_P]),
    ("bgl_tensor_info", _I, [_P, C.POINTER(_I), C.POINTER(_I), C.POINTER(_I), C.POINTER(_I), C.POINTER(C.c_size_t)]),
    ("bgl_dequant_dev", _I, [_P, _P, _I, _I, _P]),
    ("bgl_matmul_dev", _I, [_P, _P, _I, _P, _P, _P, _I]),
    ("bgl_mlp_dev", _I, [_P, _P, _P, _P, _I, _P, _P, _I, _P]),
    ("bgl_matmul_group_dev", _I, [_P, _I, C.POINTER(_P), _I, _P, C.POINTER(_P), C.POINTER(_P), _I]),
    ("bgl_matmul_group_noalloc_dev", _I, [_P, _I, C.POINTER(_P), _I, _P, C.POINTER(_P), C.POINTER(_P), _I]),
    ("bgl_read_probe_dev", _I, [_P, _I, C.POINTER(_P), _I, _I]),
    ("bgl_prep_act_dev", _I, [_P, _I, _I, _P, _I, _I]),
    ("bgl_matmul_prepped_dev", _I, [_P, _P, _I, _P, _P, _I]),
    ("bgl_quant_act_i8_dev", _I, [_P, _P, _I, _I, _I, _P, _P]),
    ("bgl_gemv_q4g64_mt", _I, [_P, _P, _P, _P, _P, _P, _I, _I]),
    ("bgl_gemv_q4g64_mt_fused", _I, [_P, _P, _P, _P, _P, _P, _I, _I]),
    ("bgl_gemv_q4g64_sdot_mt", _I, [_P, _P, _P, _P, _P, _P, _I, _I]),
    ("bgl_gemm_qXg64_sdot_mt", _I, [_P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I]),
    ("bgl_gemm_q4g256sf_sdot_mt", _I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I]),
    ("bgl_gemv_q8g64_mt", _I, [_P, _P, _P, _P, _P, _P, _I, _I]),
    ("bgl_gemv_q8g64_sdot_mt", _I, [_P, _P, _P, _P, _P, _P, _I, _I]),
    ("bgl_gemm_qXg64_mt", _I, [_P, _I, _P, _P, _P, _P, _P, _I, _I, _I]),
    ("bgl_gemv_q4g256sf_sdot_mt", _I, [_P, _P, _P, _P, _P, _P, _P, _I, _I]),
    ("bgl_gemm_q4g256sf_mt", _I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I]),
    ("bgl_qng64_matvec_f32", _I, [_P, _P, _P, _I, _P, _P, _P, _I, _I]),
    ("bgl_qng64_matmul_f32", _I, [_P, _P, _P, _I, _P, _P, _P, _I, _I, _I]),
    ("bgl_gemv_q4g32h_mt", _I, [_P, _P, _P, _P, _P, _P, _I, _I]),
    ("bgl_forget", _I, [_P, _P]),
    ("bgl_bind_experts", _I, [_P, _I, C.POINTER(bgl_wt), C.POINTER(_P)]),
    ("bgl_experts_from_tensors", _I, [_P, _I, C.POINTER(_P), C.POINTER(_P)]),
    ("bgl_gather_matvec_dev", _I, [_P, _P, _P, _P, _I, _P]),
    ("bgl_moe_ffn_dev", _I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P]),
    ("bgl_moe_route_dev", _I, [_P, _P, _P, _I, _I, _P, _I, _I, _I, _P, _P]),
    ("bgl_moe_layer_dev", _I, [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P]),
    # name-keyed registry (mlx_moe.h boundary)
    ("bgl_gpu_available", _I, []),
    ("bgl_gpu_bind_router", _I, [C.c_char_p, _P, _P, _L, _L]),
    ("bgl_bind_qng64_mixed", _I, [_P, _P, _L, _P, _P, _P, _I, _I, C.POINTER(_P)]),
    ("bgl_int4_layout_check", _I, [C.c_char_p, C.c_char_p, C.POINTER(_I)]),
    ("bgl_af_layout_check", _I, [C.c_char_p, _L, C.POINTER(_I)]),
    ("bgl_gpu_load_layout_af", _I, [C.c_char_p, _P, _L]),
    ("bgl_model_load_int4", _I, [_P, C.c_char_p, C.c_char_p, C.POINTER(_P)]),
    ("bgl_model_count", _I, [_P]),
    ("bgl_model_find", _I, [_P, C.c_char_p, C.POINTER(_I), C.POINTER(_I), C.POINTER(_I), C.POINTER(_P), C.POINTER(_P)]),
    ("bgl_model_free", _I, [_P]),
    ("bgl_model_save_cache", _I, [_P, C.c_char_p, C.c_char_p, C.c_char_p]),
    ("bgl_model_cache_valid", _I, [C.c_char_p, C.c_char_p, C.c_char_p]),
    ("bgl_model_load_cache", _I, [_P, C.c_char_p, C.c_char_p, C.c_char_p, C.POINTER(_P)]),
    ("bgl_gpu_qng64_mixed_dense_probe", _I, [_P, _L, _P, _P, _P, _L, _L, _P, _I, _P]),
    ("bgl_gpu_bind_qng64_mixed_dense_probe", _I, [_P, _L, _P, _P, _P, C.c_char_p, _L, _L]),
    ("bgl_gpu_moe_layer", _I, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, _P, _I, _I,
                               _I, _P, _P, _P]),
    ("bgl_gpu_synchronize", _I, []),
    ("bgl_gpu_reset_runtime_epoch", _I, []),
    ("bgl_gpu_bind_af", _I, [_P, _L, C.c_char_p, _L, _L, _L, _L, _L, _L, _L, _I]),
    ("bgl_gpu_binding_kind", _I, [C.c_char_p, C.POINTER(_I)]),
    ("bgl_gpu_snapshot_binding", _I, [C.c_char_p, C.POINTER(C.c_uint64)]),
    ("bgl_gpu_restore_binding_snapshot", _I, [C.c_uint64]),
    ("bgl_gpu_drop_binding_snapshot", _I, [C.c_uint64]),
    ("bgl_gpu_binding_snapshot_count", _I, []),
    ("bgl_gpu_zerocopy_count", _I, [C.POINTER(_I), C.POINTER(_I), C.POINTER(C.c_size_t)]),
    ("bgl_gpu_dequant_probe", _I, [C.c_char_p, _L, _L, _L, _I, _P]),
    ("bgl_gpu_qng64_gather_probe", _I, [_P, _L, _L, _L, _L, _I, _P, _P, _I, _P, _P]),
    ("bgl_gpu_bind_qng64_dense_probe", _I, [_P, _P, C.c_char_p, _L, _L, _I]),
    ("bgl_gpu_matvec_probe", _I, [C.c_char_p, _L, _P, _P]),
    ("bgl_gpu_report_memory", None, [C.POINTER(C.c_size_t)] * 3),
    ("bgl_gpu_set_batch", _I, [_I]),
    ("bgl_gpu_set_sort_threshold", _I, [_I]),
    ("bgl_gpu_test_ffn_uniform", _I, [C.c_char_p] * 3),
    ("bgl_gpu_ffn_gather", _I, [C.c_char_p, _P, _I, _P, _P]),
    ("bgl_gpu_moe_ffn", _I, [C.c_char_p] * 6 + [_P, _I, _P, _P, _I, _P]),
    ("bgl_gpu_context", _P, []),
    ("bgl_gpu_lookup", _P, [C.c_char_p]),
]


def header_symbols():
    """Function names declared in include/beglin_qgemv.h (parsed from the header text)."""
    import re
    hdr = os.path.join(os.path.dirname(HERE), "include", "beglin_qgemv.h")
    txt = open(hdr).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(bgl_[A-Za-z0-9_]+)\s*\(", txt)))


def load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build() (python -m beglin_amd.build)")
    lib = C.CDLL(LIB_PATH)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib
