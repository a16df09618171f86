"""oracle/oracle.py — TEST INFRASTRUCTURE ONLY: ctypes bindings of the CPU
checker libraries built by oracle/Makefile.

  liboracle.so         the C restatement of the reference semantics
                       (apus_oracle.c; every function cites reference file:line)
  _ref/libapusref.so   the reference's own CPU kernels compiled from
                       /root/reference/c via ref_shim.c (optional: absent
                       when the reference tree was not available at build)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libapusref.so")

c_size = ctypes.c_size_t
c_int = ctypes.c_int
c_vp = ctypes.c_void_p
c_float = ctypes.c_float
c_u8 = ctypes.c_uint8
c_u16 = ctypes.c_uint16

class SlabLayout(ctypes.Structure):
    """ApoSlabLayout: byte offsets of the six slab members and the size."""
    _fields_ = [(n, c_size) for n in ("gw", "gs", "uw", "us", "dw", "ds",
                                      "bytes")]


_ORACLE_SIGS = {
    "apo_e4m3_f32": (c_float, [c_u8]),
    "apo_bf16_bits": (c_u16, [c_float]),
    "apo_bf16_round": (c_float, [c_float]),
    "apo_bf16_f32": (c_float, [c_u16]),
    "apo_nblocks": (c_size, [c_size]),
    "apo_fp8blk_dequant": (None, [c_vp, c_vp, c_vp, c_size, c_size]),
    "apo_fp8blk_dequant_mt": (None, [c_vp, c_vp, c_vp, c_size, c_size, c_int]),
    "apo_bf16_gemm": (None, [c_vp, c_vp, c_vp, c_size, c_size, c_size]),
    "apo_bf16_gemm_mt": (c_int, [c_vp, c_vp, c_vp, c_size, c_size, c_size,
                                 c_int]),
    "apo_fp8blk_linear": (c_int, [c_vp, c_vp, c_vp, c_vp, c_size, c_size,
                                  c_size, c_int]),
    "apo_bf16_gemm_absdot": (None, [c_vp, c_vp, c_vp, c_size, c_size, c_size]),
    "apo_sigmoid_np": (c_float, [c_float]),
    "apo_pw_sum": (c_float, [c_vp, c_size]),
    "apo_topk_stable": (None, [c_vp, c_int, c_int, c_vp]),
    "apo_swiglu_expert": (c_int, [c_vp, c_vp, c_vp, c_vp, c_size, c_size,
                                  c_float, c_vp, c_vp, c_vp, c_vp, c_int]),
    "apo_slab_layout": (SlabLayout, [c_size, c_size]),
    "apo_slab_dequant": (None, [c_vp, c_size, c_size, c_vp, c_int]),
    "apo_moe_forward": (c_int, [c_vp, c_int, c_size, c_size, c_float, c_vp,
                                c_size, c_vp, c_vp, c_int, c_vp, c_vp, c_int]),
    "apo_moe_forward_grouped": (c_int, [c_vp, c_int, c_vp, c_size, c_size, c_float, c_vp,
                                        c_size, c_vp, c_vp, c_int, c_vp, c_vp, c_int]),
    "apo_moe_chain64_grouped": (c_int, [c_vp, c_int, c_vp, c_size, c_size, c_float, c_vp,
                                        c_size, c_vp, c_vp, c_int, c_vp, c_vp, c_int]),
    "apo_moe_floor_grouped": (c_int, [c_vp, c_int, c_vp, c_size, c_size, c_float, c_vp,
                                      c_size, c_vp, c_vp, c_int, c_vp, c_vp, c_int]),
    "apo_moe_forward_shared": (c_int, [c_vp, c_int, c_vp, c_size, c_size, c_float, c_vp,
                                       c_size, c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_int]),
    "apo_route_softmax": (None, [c_vp, c_int, c_int, c_vp, c_vp]),
    "apo_gate_dot": (c_float, [c_vp, c_vp, c_size]),
    "apo_gmoe_router": (None, [c_vp, c_vp, c_int, c_size, c_int, c_float, c_vp,
                               c_vp, c_vp, c_vp]),
    "apo_gmoe_router_from_logits": (None, [c_vp, c_vp, c_int, c_int, c_float, c_vp,
                                           c_vp, c_vp]),
    "apo_default_threads": (c_int, []),
}

_REF_SIGS = {
    "ref_e4m3_f32": (c_float, [c_u8]),
    "ref_bf16_bits": (c_u16, [c_float]),
    "ref_bf16_round": (c_float, [c_float]),
    "ref_sigmoid": (c_float, [c_float]),
    "ref_pw_sum": (c_float, [c_vp, c_size]),
    "ref_topk_stable": (None, [c_vp, c_int, c_int, c_vp]),
    "ref_fp8blk_dequant_scalar": (None, [c_vp, c_vp, c_vp, c_size, c_size]),
    "ref_fp8blk_dequant_mt": (None, [c_vp, c_vp, c_vp, c_size, c_size]),
    "ref_bf16_gemm_scalar": (None, [c_vp, c_vp, c_vp, c_size, c_size, c_size]),
    "ref_bf16_gemm_mt": (c_int, [c_vp, c_vp, c_vp, c_size, c_size, c_size]),
    "ref_fp8blk_linear_mt": (c_int, [c_vp, c_vp, c_vp, c_vp, c_size, c_size,
                                     c_size]),
    "ref_gmoe_expert": (c_int, [c_vp, c_vp, c_vp, c_vp, c_size, c_size,
                                c_float, c_vp]),
    "ref_pool_threads": (c_int, []),
    "ref_gmoe_forward2": (None, [c_vp, c_int, c_size, c_size, c_vp, c_size, c_float, c_vp,
                                 c_vp, c_int, c_float, c_vp, c_size, c_vp, c_vp, c_vp]),
    "ref_gmoe_router": (None, [c_vp, c_vp, c_int, c_size, c_int, c_float, c_vp,
                               c_vp, c_vp, c_vp]),
}

_oracle = None
_ref = None


def _bind(path, sigs):
    lib = ctypes.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError("oracle/liboracle.so not built (make -C oracle)")
        _oracle = _bind(ORACLE_PATH, _ORACLE_SIGS)
    return _oracle


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own CPU kernels (raises when not built)."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError("oracle/_ref/libapusref.so not built")
        _ref = _bind(REF_PATH, _REF_SIGS)
    return _ref


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


# ---- numpy conveniences over the C functions ------------------------------

def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """RNE narrow (c/num.h:153-159), vectorized restatement for test inputs."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, u >> 16, r)
    return r.astype(np.uint16)


def nblocks(n):
    return (n + 127) // 128


def dequant(codes, scales, threads=1):
    codes = np.ascontiguousarray(codes, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    O, K = codes.shape
    out = np.empty((O, K), np.uint16)
    if threads == 1:
        lib().apo_fp8blk_dequant(ptr(codes), ptr(scales), ptr(out), O, K)
    else:
        lib().apo_fp8blk_dequant_mt(ptr(codes), ptr(scales), ptr(out), O, K,
                                    threads)
    return out


def gemm(w, x, threads=1):
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.uint16)
    O, K = w.shape
    M = x.shape[0]
    y = np.empty((M, O), np.uint16)
    if threads == 1:
        lib().apo_bf16_gemm(ptr(w), ptr(x), ptr(y), M, O, K)
    else:
        assert lib().apo_bf16_gemm_mt(ptr(w), ptr(x), ptr(y), M, O, K,
                                      threads) == 0
    return y


def fp8_linear(codes, scales, x, threads=1):
    codes = np.ascontiguousarray(codes, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    x = np.ascontiguousarray(x, np.uint16)
    O, K = codes.shape
    M = x.shape[0]
    y = np.empty((M, O), np.uint16)
    assert lib().apo_fp8blk_linear(ptr(codes), ptr(scales), ptr(x), ptr(y), M,
                                   O, K, threads) == 0
    return y


def absdot(w, x):
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.uint16)
    O, K = w.shape
    M = x.shape[0]
    a = np.empty((M, O), np.float64)
    lib().apo_bf16_gemm_absdot(ptr(w), ptr(x), ptr(a), M, O, K)
    return a


def swiglu_expert(wg, wu, wd, x, limit=10.0, threads=1):
    wg, wu, wd = (np.ascontiguousarray(a, np.uint16) for a in (wg, wu, wd))
    x = np.ascontiguousarray(x, np.uint16)
    inter, dim = wg.shape
    out = np.empty(dim, np.uint16)
    g = np.empty(inter, np.uint16)
    u = np.empty(inter, np.uint16)
    h = np.empty(inter, np.uint16)
    assert lib().apo_swiglu_expert(ptr(wg), ptr(wu), ptr(wd), ptr(x), dim,
                                   inter, limit, ptr(out), ptr(g), ptr(u),
                                   ptr(h), threads) == 0
    return out, g, u, h


def gmoe_router(gate_w, gate_bias, x, topk, route_scale=2.5):
    """c/gmoe.h:191-208 -> (scores [E], idx [topk], w [topk])."""
    gate_w = np.ascontiguousarray(gate_w, np.uint16)
    E, dim = gate_w.shape
    bias = np.ascontiguousarray(gate_bias, np.float32)
    x = np.ascontiguousarray(x, np.uint16)
    sc = np.empty(E, np.float32)
    idx = np.empty(topk, np.int32)
    w = np.empty(topk, np.float32)
    lib().apo_gmoe_router(ptr(gate_w), ptr(bias), E, dim, topk, route_scale, ptr(x),
                          ptr(sc), ptr(idx), ptr(w))
    return sc, idx, w


def gmoe_router_from_logits(logits, gate_bias, topk, route_scale=2.5):
    logits = np.ascontiguousarray(logits, np.float32)
    bias = np.ascontiguousarray(gate_bias, np.float32)
    E = logits.size
    sc = np.empty(E, np.float32)
    idx = np.empty(topk, np.int32)
    w = np.empty(topk, np.float32)
    lib().apo_gmoe_router_from_logits(ptr(logits), ptr(bias), E, topk, route_scale,
                                      ptr(sc), ptr(idx), ptr(w))
    return sc, idx, w


def route_softmax(logits, k):
    logits = np.ascontiguousarray(logits, np.float32)
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().apo_route_softmax(ptr(logits), logits.size, k, ptr(idx), ptr(w))
    return idx, w


def moe_forward(slabs, dim, inter, x, idx, w, limit=10.0, threads=1,
                want_expert_out=False, grouped=False, chain64=False, shared=None):
    """slabs: list of uint8 arrays (one slab per expert id; None allowed for
    experts no token routes to). grouped: compute expert by expert
    (apo_moe_forward_grouped, the same bits, far faster at many tokens).
    chain64: the f64-sum yardstick (apo_moe_chain64_grouped) instead.
    shared: the shared expert's slab (uint8), added last (c/gmoe.h:325-336)."""
    E = len(slabs)
    arr = (c_vp * E)()
    for e, s in enumerate(slabs):
        arr[e] = s.ctypes.data if s is not None else None
    x = np.ascontiguousarray(x, np.uint16).reshape(-1, dim)
    T = x.shape[0]
    idx = np.ascontiguousarray(idx, np.int32).reshape(T, -1)
    w = np.ascontiguousarray(w, np.float32).reshape(T, -1)
    k = idx.shape[1]
    out = np.empty((T, dim), np.uint16)
    eo = np.empty((T, k, dim), np.uint16) if want_expert_out else None
    sp = ptr(shared) if shared is not None else None
    eop = ptr(eo) if eo is not None else None
    if chain64 or grouped:
        fn = lib().apo_moe_chain64_grouped if chain64 else lib().apo_moe_forward_grouped
        rc = fn(arr, E, sp, dim, inter, limit, ptr(x), T, ptr(idx), ptr(w), k, ptr(out),
                eop, threads)
    elif shared is not None:
        rc = lib().apo_moe_forward_shared(arr, E, sp, dim, inter, limit, ptr(x), T,
                                          ptr(idx), ptr(w), k, ptr(out), eop, None, threads)
    else:
        rc = lib().apo_moe_forward(arr, E, dim, inter, limit, ptr(x), T, ptr(idx), ptr(w),
                                   k, ptr(out), eop, threads)
    assert rc == 0
    return (out, eo) if want_expert_out else out


def moe_expert_floor(slabs, dim, inter, x, idx, w, limit=10.0, threads=1, shared=None):
    """Per output element, sum over the token's kept pairs of |w_e| *
    sum_i |h_i * wd_e[j, i]| (f64, [T, dim]): the combine's tolerance floor
    that carries each expert output's own floor (apo_moe_floor_grouped)."""
    E = len(slabs)
    arr = (c_vp * E)()
    for e, s in enumerate(slabs):
        arr[e] = s.ctypes.data if s is not None else None
    x = np.ascontiguousarray(x, np.uint16).reshape(-1, dim)
    T = x.shape[0]
    idx = np.ascontiguousarray(idx, np.int32).reshape(T, -1)
    w = np.ascontiguousarray(w, np.float32).reshape(T, -1)
    out = np.empty((T, dim), np.uint16)
    fl = np.empty((T, dim), np.float64)
    sp = ptr(shared) if shared is not None else None
    assert lib().apo_moe_floor_grouped(arr, E, sp, dim, inter, limit, ptr(x), T, ptr(idx),
                                       ptr(w), idx.shape[1], ptr(out), ptr(fl), threads) == 0
    return fl
