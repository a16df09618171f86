"""K2 and the hook boundary on the GPU: FP8-block linear (dequant fused in
the GEMV/GEMM) and the BF16 GEMM against the oracle / reference-written
golden outputs, to the contract tolerance (tests/tolerance.py). Covers the
BASELINE configs 0 and 1, the DSA shapes of tests/m7b/test_gkernels.c:
157-211, ceil shapes, NaN codes, the floors/fail-soft contract
(tests/m7b/test_gkernels.c:283-324) and registered regions."""
import ctypes
import json
import os

import numpy as np
import pytest

import oracle as O
import gpu_util as G
from tolerance import assert_close

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def fx():
    return np.load(os.path.join(GOLD, "fixtures.npz"))


@pytest.fixture(scope="module")
def man():
    return json.load(open(os.path.join(GOLD, "manifest.json")))


def gpu_linear(ghip, codes, scales, x):
    Oo, K = codes.shape
    M = x.shape[0]
    y = np.empty((M, Oo), np.uint16)
    rc = ghip.apus_ghip_fp8blk_linear(O.ptr(codes), O.ptr(scales), O.ptr(x),
                                      O.ptr(y), M, Oo, K)
    assert rc == 0, ghip.apus_ghip_last_error()
    return y


def floor_linear(codes, scales, x):
    return 2.0 ** -8 * O.absdot(O.dequant(codes, scales, threads=8), x)


def synth_linear(lib, seed, M, N, K):
    codes = np.empty((N, K), np.uint8)
    lib.apus_synth_fp8_codes(O.ptr(codes), codes.size, seed, 10, 0)
    scales = np.empty((O.nblocks(N), O.nblocks(K)), np.float32)
    lib.apus_synth_scales(O.ptr(scales), scales.size, seed, 11, 1e-4, 1e-2)
    x = np.empty((M, K), np.uint16)
    lib.apus_synth_bf16_normal(O.ptr(x), x.size, seed, 12, 0)
    return codes, scales, x


def test_golden_linear(ghip, fx, man):
    for i, sh in enumerate(man["linear"]):
        c, s, x = fx[f"lin{i}_codes"], fx[f"lin{i}_scales"], fx[f"lin{i}_x"]
        assert_close(gpu_linear(ghip, c, s, x), fx[f"lin{i}_y"],
                     floor_linear(c, s, x), "lin%d %s" % (i, sh))


def test_config0(ghip, pkg, fx, man):
    c, s, x = synth_linear(pkg.load(), 0xC0, 1, 2048, 4096)
    st = assert_close(gpu_linear(ghip, c, s, x), fx["cfg0_y"],
                      floor_linear(c, s, x), "config0")
    print("config0", st)


def test_config1_m124(ghip, pkg, fx, man):
    c, s, x = synth_linear(pkg.load(), 0xC1, 4, 16384, 4096)
    fl = floor_linear(c, s, x)
    for M in (1, 2, 4):
        st = assert_close(gpu_linear(ghip, c, s, x[:M]), fx["cfg1_y"][:M],
                          fl[:M], "config1 M=%d" % M)
        print("config1 M=%d" % M, st)


DSA = [(1, 1536, 4096), (5, 1536, 4096), (1, 16384, 1536), (3, 16384, 1536),
       (1, 512, 4096), (1, 4096, 16384), (2, 4096, 16384), (1, 200, 300),
       (2, 200, 300), (5, 129, 127), (1, 128, 128), (3, 127, 129),
       (1, 2048, 4096), (9, 64, 256)]


@pytest.mark.parametrize("M,N,K", DSA)
def test_fp8_battery(ghip, M, N, K):
    rng = np.random.default_rng(M * 100003 + N * 7 + K)
    codes = rng.integers(0, 254, (N, K), dtype=np.uint8)
    codes[codes >= 0x7F] += 1
    m = 0.25 + 3.75 * rng.random((O.nblocks(N), O.nblocks(K)))
    e = rng.integers(-24, 17, m.shape)
    scales = (np.ldexp(m, e) * rng.choice([-1, 1], m.shape)).astype(np.float32)
    x = O.f32_to_bf16(rng.uniform(-4, 4, (M, K)).astype(np.float32))
    want = O.fp8_linear(codes, scales, x, threads=8)
    assert_close(gpu_linear(ghip, codes, scales, x), want,
                 floor_linear(codes, scales, x), "M%d N%d K%d" % (M, N, K))


# prefill-sized M: the MFMA GEMM path (M >= 16, N % 256 == 0, K % 128 == 0),
# incl. ragged row tiles, K = 128 and K = 16384 (o_proj), the DSA shapes of
# c/gdsa.h:599-611,660-661 at M = s; M = 15 stays on the GEMV passes. Most
# small-M shapes run split-K (fp32 partials summed in a fixed order):
# (16, 256, 16384) with 64 splits of 2 k blocks, (64, 4096, 16384) with 12,
# (2048, 512, 4096) with 6 on 128-row tiles; (513, 256, 128) cannot split
GEMM = [(16, 512, 4096), (100, 1536, 4096), (300, 2048, 1536), (40, 16384, 1536),
        (256, 4096, 16384), (513, 256, 128), (15, 512, 1024), (17, 300, 512),
        (16, 256, 16384), (64, 4096, 16384), (2048, 512, 4096)]


@pytest.mark.parametrize("M,N,K", GEMM)
def test_fp8_gemm_prefill_shapes(ghip, M, N, K):
    rng = np.random.default_rng(M * 7919 + N * 13 + K)
    codes = rng.integers(0, 254, (N, K), dtype=np.uint8)
    codes[codes >= 0x7F] += 1
    m = 0.25 + 3.75 * rng.random((O.nblocks(N), O.nblocks(K)))
    e = rng.integers(-24, 17, m.shape)
    scales = (np.ldexp(m, e) * rng.choice([-1, 1], m.shape)).astype(np.float32)
    x = O.f32_to_bf16(rng.uniform(-4, 4, (M, K)).astype(np.float32))
    want = O.fp8_linear(codes, scales, x, threads=16)
    got = gpu_linear(ghip, codes, scales, x)
    st = assert_close(got, want, floor_linear(codes, scales, x), "M%d N%d K%d" % (M, N, K))
    print("gemm M%d N%d K%d" % (M, N, K), st)
    assert np.array_equal(got, gpu_linear(ghip, codes, scales, x))   # deterministic


def test_fp8_gemm_nan_codes_exact_decode(ghip):
    """Every code incl. 0x7F/0xFF through the GEMM path (the NaN scan
    selects the exact integer decode)."""
    M, N, K = 48, 512, 1024
    codes = (np.arange(N * K) & 0xFF).astype(np.uint8).reshape(N, K)
    rng = np.random.default_rng(5)
    scales = np.exp2(rng.uniform(-10, -4, (O.nblocks(N), O.nblocks(K)))).astype(np.float32)
    x = O.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    want = O.fp8_linear(codes, scales, x, threads=8)
    assert_close(gpu_linear(ghip, codes, scales, x), want,
                 floor_linear(codes, scales, x), "gemm all codes")


@pytest.mark.parametrize("M,N,K", [(1, 512, 512), (2, 300, 768), (1, 256, 1024)])
def test_all_256_codes_incl_nan_codes(ghip, M, N, K):
    """Every code incl. 0x7F/0xFF (decoded as +-480 by the reference): the
    scan routes such weights to the exact decode."""
    codes = (np.arange(N * K) & 0xFF).astype(np.uint8).reshape(N, K)
    rng = np.random.default_rng(N)
    scales = np.exp2(rng.uniform(-10, -4, (O.nblocks(N), O.nblocks(K)))).astype(np.float32)
    x = O.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    want = O.fp8_linear(codes, scales, x, threads=8)
    assert_close(gpu_linear(ghip, codes, scales, x), want,
                 floor_linear(codes, scales, x), "all codes N%d K%d" % (N, K))


def test_linear_dev_entry(ghip, pkg):
    c, s, x = synth_linear(pkg.load(), 0x51, 4, 4096, 2048)
    want = O.fp8_linear(c, s, x, threads=8)
    dc, ds, dx = G.dev(c), G.dev(s), G.dev(x)
    for exact in (0, 1, -1):
        dy = G.empty(4 * 4096 * 2)
        assert ghip.apus_ghip_fp8blk_linear_dev(G.vp(dc), G.vp(ds), G.vp(dx), G.vp(dy),
                                                4, 4096, 2048, exact, G.stream()) == 0
        assert_close(G.host(dy, np.uint16, (4, 4096)), want, floor_linear(c, s, x),
                     "dev exact=%d" % exact)


def test_linear_dev_unaligned_y(ghip, pkg):
    """The GEMM path (M >= 16) stores 16-byte vectors, so it needs a 16-byte
    aligned y; a y two bytes off goes to the streaming GEMV (4 rows per
    launch, 2-byte stores) instead. Checked at M = 32 against the oracle,
    with the elements either side of y left untouched."""
    M, N, K = 32, 1024, 2048
    c, s, x = synth_linear(pkg.load(), 0x53, M, N, K)
    want = O.fp8_linear(c, s, x, threads=8)
    guard = np.full(M * N + 16, 0x7E57, np.uint16)
    dc, ds, dx, dy = G.dev(c), G.dev(s), G.dev(x), G.dev(guard)
    yp = ctypes.c_void_p(G.vp(dy).value + 2)
    assert ghip.apus_ghip_fp8blk_linear_dev(G.vp(dc), G.vp(ds), G.vp(dx), yp, M, N, K, -1,
                                            G.stream()) == 0, ghip.apus_ghip_last_error()
    got = G.host(dy, np.uint16, guard.shape)
    assert got[0] == 0x7E57 and np.all(got[1 + M * N:] == 0x7E57), "wrote outside y"
    assert_close(got[1:1 + M * N].reshape(M, N), want, floor_linear(c, s, x),
                 "unaligned y, M=32")


def test_deterministic(ghip, pkg):
    c, s, x = synth_linear(pkg.load(), 0x52, 2, 4096, 4096)
    y1 = gpu_linear(ghip, c, s, x)
    y2 = gpu_linear(ghip, c, s, x)
    assert np.array_equal(y1, y2)


def test_bf16_gemm_golden(ghip, fx, man):
    for i, sh in enumerate(man["gemm"]):
        w, x = fx[f"gem{i}_w"], fx[f"gem{i}_x"]
        y = np.empty((sh["M"], sh["O"]), np.uint16)
        assert ghip.apus_ghip_bf16_gemm(O.ptr(w), O.ptr(x), O.ptr(y), sh["M"],
                                        sh["O"], sh["K"]) == 0
        assert_close(y, fx[f"gem{i}_y"], 2.0 ** -8 * O.absdot(w, x), "gem%d" % i)


def test_bf16_gemm_real_shapes(ghip):
    """Real shapes (streaming MFMA GEMV, M in groups of <= 4) and ragged
    ones: O % 16 != 0, K = 64, K % 64 != 0 (the generic kernel)."""
    rng = np.random.default_rng(3)
    for (Oo, K) in [(2048, 4096), (4096, 2048), (288, 4096), (300, 64), (129, 200)]:
        for M in (1, 3, 5):
            w = O.f32_to_bf16(rng.uniform(-4, 4, (Oo, K)).astype(np.float32))
            x = O.f32_to_bf16(rng.uniform(-4, 4, (M, K)).astype(np.float32))
            y = np.empty((M, Oo), np.uint16)
            assert ghip.apus_ghip_bf16_gemm(O.ptr(w), O.ptr(x), O.ptr(y), M, Oo, K) == 0
            assert_close(y, O.gemm(w, x, threads=8), 2.0 ** -8 * O.absdot(w, x),
                         "bf16 %dx%d M%d" % (Oo, K, M))


def test_hooks_floor_failsoft_and_regions(ghip):
    """Hooks are filled by enable; an oversized floor makes the hook decline
    (the engine then runs its CPU kernel) while the direct entry still runs;
    disable clears the hooks; registered weights are not re-uploaded."""
    hooks = (ctypes.c_void_p * 2).in_dll(ghip, "apus_ghip_hooks")
    assert hooks[0] and hooks[1]
    HookBf16 = ctypes.CFUNCTYPE(ctypes.c_int, *([ctypes.c_void_p] * 3 + [ctypes.c_size_t] * 3))
    rng = np.random.default_rng(8)
    w = O.f32_to_bf16(rng.uniform(-2, 2, (512, 4096)).astype(np.float32))
    x = O.f32_to_bf16(rng.uniform(-2, 2, (1, 4096)).astype(np.float32))
    y = np.empty((1, 512), np.uint16)
    os.environ["APUS_GHIP_MIN_KB"] = "100000000"
    try:
        ghip.apus_ghip_disable()
        assert hooks[0] is None and hooks[1] is None
        buf = ctypes.create_string_buffer(256)
        assert ghip.apus_ghip_enable(buf, 256) == 0
        hook = HookBf16(hooks[0])
        assert hook(O.ptr(w), O.ptr(x), O.ptr(y), 1, 512, 4096) != 0
        assert ghip.apus_ghip_bf16_gemm(O.ptr(w), O.ptr(x), O.ptr(y), 1, 512, 4096) == 0
    finally:
        del os.environ["APUS_GHIP_MIN_KB"]
        ghip.apus_ghip_disable()
        assert ghip.apus_ghip_enable(ctypes.create_string_buffer(256), 256) == 0
    hook = HookBf16(hooks[0])
    before = ghip.apus_ghip_offload_bf16()
    assert hook(O.ptr(w), O.ptr(x), O.ptr(y), 1, 512, 4096) == 0
    assert ghip.apus_ghip_offload_bf16() == before + 1
    assert_close(y, O.gemm(w, x), 2.0 ** -8 * O.absdot(w, x), "hooked bf16")
    # registered region: the FP8 weights are uploaded once
    codes = rng.integers(0, 254, (1024, 2048), dtype=np.uint8)
    scales = np.exp2(rng.uniform(-9, -5, (8, 16))).astype(np.float32)
    xx = O.f32_to_bf16(rng.standard_normal((1, 2048)).astype(np.float32))
    assert ghip.apus_ghip_register_region(O.ptr(codes), codes.nbytes) == 0
    assert ghip.apus_ghip_register_region(O.ptr(scales), scales.nbytes) == 0
    wrapped = ghip.apus_ghip_bytes_wrapped()
    y1 = gpu_linear(ghip, codes, scales, xx)
    y2 = gpu_linear(ghip, codes, scales, xx)
    assert ghip.apus_ghip_bytes_wrapped() == wrapped
    assert np.array_equal(y1, y2)
    assert_close(y1, O.fp8_linear(codes, scales, xx), floor_linear(codes, scales, xx),
                 "registered")
    ghip.apus_ghip_unregister_region(O.ptr(codes))
    ghip.apus_ghip_unregister_region(O.ptr(scales))


def test_fp8_hook_through_table_floors(ghip):
    """The fp8blk_linear hook called through the table, the analog of
    tests/m7b/test_gkernels.c:283-324 for the FP8 site (c/gdsa.h:529-531):
    with APUS_GHIP_FP8_MIN_KB above the weight size, or APUS_GHIP_MAX_M below
    M, the hook declines (nonzero: the engine runs its CPU kernel) and the
    offload counter does not move; the direct entry ignores the floors;
    without floors the hook runs, moves offload_fp8blk by one, and meets
    the tolerance. Both the GEMV (M = 1) and GEMM (M = 32) paths."""
    hooks = (ctypes.c_void_p * 2).in_dll(ghip, "apus_ghip_hooks")
    HookFp8 = ctypes.CFUNCTYPE(ctypes.c_int, *([ctypes.c_void_p] * 4 + [ctypes.c_size_t] * 3))
    rng = np.random.default_rng(0xF8)
    N, K = 512, 2048
    codes = rng.integers(0, 254, (N, K), dtype=np.uint8)
    codes[codes >= 0x7F] += 1
    scales = np.exp2(rng.uniform(-10, -6, (N // 128, K // 128))).astype(np.float32)
    env = {"APUS_GHIP_FP8_MIN_KB": str(N * K // 1024 + 1), "APUS_GHIP_MAX_M": "8"}
    try:
        for name, val in env.items():
            os.environ[name] = val
            ghip.apus_ghip_disable()
            assert hooks[1] is None
            assert ghip.apus_ghip_enable(ctypes.create_string_buffer(256), 256) == 0
            hook = HookFp8(hooks[1])
            M = 1 if name == "APUS_GHIP_FP8_MIN_KB" else 32
            x = O.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
            y = np.full((M, N), 0xABCD, np.uint16)
            before = ghip.apus_ghip_offload_fp8blk()
            assert hook(O.ptr(codes), O.ptr(scales), O.ptr(x), O.ptr(y), M, N, K) != 0, name
            assert ghip.apus_ghip_offload_fp8blk() == before, name
            assert np.all(y == 0xABCD), "a declining hook must not write y (%s)" % name
            y2 = gpu_linear(ghip, codes, scales, x)         # direct: no floors
            assert_close(y2, O.fp8_linear(codes, scales, x, threads=8),
                         floor_linear(codes, scales, x), "direct under " + name)
            del os.environ[name]
    finally:
        for name in env:
            os.environ.pop(name, None)
        ghip.apus_ghip_disable()
        assert ghip.apus_ghip_enable(ctypes.create_string_buffer(256), 256) == 0
    hook = HookFp8(hooks[1])
    for M in (1, 32):
        x = O.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
        y = np.empty((M, N), np.uint16)
        before = ghip.apus_ghip_offload_fp8blk()
        assert hook(O.ptr(codes), O.ptr(scales), O.ptr(x), O.ptr(y), M, N, K) == 0
        assert ghip.apus_ghip_offload_fp8blk() == before + 1
        assert_close(y, O.fp8_linear(codes, scales, x, threads=8),
                     floor_linear(codes, scales, x), "hooked fp8 M=%d" % M)
