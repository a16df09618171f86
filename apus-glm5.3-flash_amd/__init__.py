"""apus-glm5.3-flash_amd — MI355X (gfx950) backend for the apus FP8-block MoE
hot path.

The product is the C-ABI library libapus_ghip.so (include/backend_hip.h,
include/apus_synth.h): C host layer + hand-written HIP kernels. This module
only loads it through ctypes and declares the signatures, for the tests and
bench.py. It computes nothing itself and has no CPU fallback: load() raises
when the library is missing.

Import by path (the directory name is not a Python identifier):
    spec = importlib.util.spec_from_file_location(
        "apus_ghip", "<repo>/apus-glm5.3-flash_amd/__init__.py")
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libapus_ghip.so")

c_size = ctypes.c_size_t
c_int = ctypes.c_int
c_u64 = ctypes.c_uint64
c_vp = ctypes.c_void_p
c_float = ctypes.c_float

# name -> (restype, argtypes); every symbol include/*.h declares.
SIGNATURES = {
    # mirror of c/backend_gmetal.h
    "apus_ghip_enable": (c_int, [ctypes.c_char_p, c_size]),
    "apus_ghip_disable": (None, []),
    "apus_ghip_is_enabled": (c_int, []),
    "apus_ghip_register_region": (c_int, [c_vp, c_size]),
    "apus_ghip_unregister_region": (None, [c_vp]),
    "apus_ghip_bytes_wrapped": (c_u64, []),
    "apus_ghip_bytes_pinned": (c_u64, []),
    "apus_ghip_dispatches": (c_u64, []),
    "apus_ghip_offload_bf16": (c_u64, []),
    "apus_ghip_offload_fp8blk": (c_u64, []),
    "apus_ghip_bytes_h2d": (c_u64, []),
    "apus_ghip_bytes_d2h": (c_u64, []),
    "apus_ghip_bf16_gemm": (c_int, [c_vp, c_vp, c_vp, c_size, c_size, c_size]),
    "apus_ghip_fp8blk_linear": (c_int, [c_vp, c_vp, c_vp, c_vp, c_size,
                                        c_size, c_size]),
    "apus_ghip_last_error": (ctypes.c_char_p, []),
    # extensions
    "apus_ghip_fp8blk_dequant": (c_int, [c_vp, c_vp, c_vp, c_size, c_size]),
    "apus_ghip_fp8blk_dequant_dev": (c_int, [c_vp, c_vp, c_vp, c_size, c_size,
                                             c_int, c_vp]),
    "apus_ghip_fp8blk_linear_dev": (c_int, [c_vp, c_vp, c_vp, c_vp, c_size,
                                            c_size, c_size, c_int, c_vp]),
    "apus_ghip_bf16_gemm_dev": (c_int, [c_vp, c_vp, c_vp, c_size, c_size,
                                        c_size, c_vp]),
    "apus_ghip_store_open": (c_int, [ctypes.POINTER(c_vp), c_int, c_size,
                                     c_size, c_float, ctypes.c_char_p, c_size]),
    "apus_ghip_store_close": (None, [c_vp]),
    "apus_ghip_store_slab_bytes": (c_size, [c_vp]),
    "apus_ghip_store_put": (c_int, [c_vp, c_int, c_vp, c_size]),
    "apus_ghip_store_synth": (c_int, [c_vp, c_u64, c_int, c_float, c_float]),
    "apus_ghip_store_slab_dev": (c_vp, [c_vp, c_int]),
    "apus_ghip_store_get": (c_int, [c_vp, c_int, c_vp, c_size]),
    "apus_ghip_store_put_shared": (c_int, [c_vp, c_vp, c_size]),
    "apus_ghip_store_load_container": (c_int, [c_vp, ctypes.c_char_p, c_int,
                                               ctypes.POINTER(c_int), ctypes.c_char_p,
                                               c_size]),
    "apus_ghip_container_slab": (c_int, [ctypes.c_char_p, c_int, c_int, c_size,
                                         ctypes.c_char_p, c_size,
                                         ctypes.POINTER(c_u64), ctypes.c_char_p,
                                         c_size]),
    "apus_ghip_store_expert_bf16": (c_int, [c_vp, c_int, c_vp]),
    "apus_ghip_moe_decode": (c_int, [c_vp, c_vp, c_vp, c_vp, c_int, c_vp]),
    "apus_ghip_moe_decode_dev": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int,
                                         c_vp, c_vp]),
    "apus_ghip_moe_router_dev": (c_int, [c_vp, c_vp, c_vp, c_vp, c_int, c_size, c_int,
                                         c_float, c_vp, c_vp, c_vp, c_vp]),
    "apus_ghip_moe_decode_router_dev": (c_int, [c_vp, c_vp, c_vp, c_vp, c_float, c_int,
                                                c_vp, c_vp, c_vp, c_vp]),
    "apus_ghip_moe_prefill_reserve": (c_int, [c_vp, c_size, c_int]),
    "apus_ghip_moe_prefill": (c_int, [c_vp, c_vp, c_size, c_vp, c_vp, c_int,
                                      c_vp]),
    "apus_ghip_moe_prefill_dev": (c_int, [c_vp, c_vp, c_size, c_vp, c_vp,
                                          c_int, c_vp, c_vp]),
    "apus_ghip_moe_prefill_dev_noalloc": (c_int, [c_vp, c_vp, c_size, c_vp, c_vp,
                                                  c_int, c_vp, c_vp]),
    "apus_ghip_store_status": (c_int, [c_vp, c_vp, c_int,
                                       ctypes.POINTER(ctypes.c_uint32)]),
    "apus_ghip_set_trace_events": (None, [ctypes.POINTER(c_vp), c_int]),
    "apus_ghip_stream_hold": (c_int, [c_vp, ctypes.c_uint32]),
    # include/apus_synth.h
    "apus_synth_mix64": (c_u64, [c_u64]),
    "apus_synth_key": (c_u64, [c_u64, c_u64]),
    "apus_synth_u64": (c_u64, [c_u64, c_u64]),
    "apus_synth_fp8_codes": (None, [c_vp, c_size, c_u64, c_u64, c_u64]),
    "apus_synth_scales": (None, [c_vp, c_size, c_u64, c_u64, c_float, c_float]),
    "apus_synth_normal_table": (None, [c_vp]),
    "apus_synth_normal_table_ptr": (c_vp, []),
    "apus_synth_bf16_normal": (None, [c_vp, c_size, c_u64, c_u64, c_u64]),
    "apus_synth_f32_normal": (None, [c_vp, c_size, c_u64, c_u64, c_u64]),
    "apus_synth_route": (c_int, [c_vp, c_vp, c_size, c_int, c_int,
                                 ctypes.c_double, c_u64]),
    "apus_synth_expert_stream": (c_u64, [c_int, c_int, c_int]),
    "apus_synth_fp8_codes_dev": (c_int, [c_vp, c_size, c_u64, c_u64, c_u64,
                                         c_vp]),
    "apus_synth_bf16_normal_dev": (c_int, [c_vp, c_size, c_u64, c_u64, c_u64,
                                           c_vp]),
}

_lib = None


def load():
    """Load libapus_ghip.so (built by build.py) and declare signatures.
    Raises RuntimeError when the library has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            "libapus_ghip.so not built (%s); run __graft_entry__.build()"
            % LIB_PATH)
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error():
    return (load().apus_ghip_last_error() or b"").decode(errors="replace")


def check(rc, what):
    """Raise with the backend's message when an entry point returned nonzero."""
    if rc != 0:
        raise RuntimeError("%s failed (rc=%d): %s" % (what, rc, last_error()))
