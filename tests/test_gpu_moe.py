"""K3 + the HBM expert store on the GPU: dequant-on-fill is bitwise
(c/gcache.h:413-426); the one-launch MoE decode matches the oracle's
SwiGLU experts + ascending-expert bf16 combine (c/gmoe.h:210-227, 307-320)
to the contract tolerance, including the BASELINE config-2 case written by
the reference kernels (tests/golden)."""
import ctypes
import json
import os

import numpy as np
import pytest

import oracle as O
import gpu_util as G
from tolerance import assert_close, assert_close_combined, record

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def open_store(ghip, E, dim, inter, limit=10.0):
    s = ctypes.c_void_p()
    err = ctypes.create_string_buffer(256)
    assert ghip.apus_ghip_store_open(ctypes.byref(s), E, dim, inter, limit, err,
                                     256) == 0, err.value
    return s


def random_slabs(E, dim, inter, rng, nan_codes_in=()):
    slabs = []
    for e in range(E):
        parts = []
        for (o, k) in [(inter, dim), (inter, dim), (dim, inter)]:
            c = rng.integers(0, 254, (o, k), dtype=np.uint8)
            c[c >= 0x7F] += 1
            if e in nan_codes_in:
                c.reshape(-1)[::97] = 0x7F
                c.reshape(-1)[5::101] = 0xFF
            s = np.exp2(rng.uniform(-9, -5, (O.nblocks(o), O.nblocks(k)))).astype(np.float32)
            parts += [c.ravel(), s.view(np.uint8).ravel()]
        slabs.append(np.concatenate(parts))
    return slabs


def moe_floor(eo, w, idx):
    """sum_e |contrib_e| per output element (tests/tolerance.py)."""
    c = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(eo) * w[:, :, None]))
    return np.abs(c.astype(np.float64)).sum(1)


@pytest.fixture(scope="module")
def small(ghip):
    E, dim, inter = 16, 256, 128
    rng = np.random.default_rng(2024)
    slabs = random_slabs(E, dim, inter, rng, nan_codes_in=(3,))
    s = open_store(ghip, E, dim, inter)
    for e, sl in enumerate(slabs):
        assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
    assert ghip.apus_ghip_store_slab_bytes(s) == slabs[0].nbytes
    yield ghip, s, slabs, (E, dim, inter)
    ghip.apus_ghip_store_close(s)


def test_store_roundtrip(small):
    """get returns the put slab bitwise; the device slab holds the members
    in the reference order at 256-byte aligned offsets."""
    ghip, s, slabs, (E, dim, inter) = small
    sb = slabs[0].nbytes
    nbg = O.nblocks(inter) * O.nblocks(dim) * 4
    up = lambda v: (v + 255) // 256 * 256  # noqa: E731
    h_off, d_off, parts = 0, 0, []
    for n in (inter * dim, nbg, inter * dim, nbg, dim * inter, nbg):
        parts.append((h_off, d_off, n))
        h_off += n
        d_off += up(n)
    for e in (0, 3, 15):
        got = np.empty(sb, np.uint8)
        assert ghip.apus_ghip_store_get(s, e, O.ptr(got), sb) == 0
        assert np.array_equal(got, slabs[e]), e
        dev = G.download_ptr(ghip.apus_ghip_store_slab_dev(s, e), np.uint8, (d_off,))
        for h, d, n in parts:
            assert np.array_equal(dev[d:d + n], slabs[e][h:h + n]), (e, h)


def test_store_load_container(ghip, tmp_path):
    """A converted v2 container (two layers in two shards): the layer's
    listed experts load bitwise (one pread per slab), unlisted ones keep
    their bytes, another layer loads its own slabs, and the decode over the
    loaded bank matches the oracle on the same slabs."""
    from container_util import write_container
    E, dim, inter = 16, 256, 128
    rng = np.random.default_rng(77)
    l3 = random_slabs(E, dim, inter, rng)
    l4 = random_slabs(E, dim, inter, rng)
    listed = [e for e in range(E) if e != 6]
    write_container(str(tmp_path), {3: {e: l3[e] for e in listed},
                                    4: {e: l4[e] for e in range(E)}}, l3[0].nbytes)
    s = open_store(ghip, E, dim, inter)
    try:
        sb = ghip.apus_ghip_store_slab_bytes(s)
        assert ghip.apus_ghip_store_put(s, 6, O.ptr(l4[6]), sb) == 0
        n = ctypes.c_int()
        err = ctypes.create_string_buffer(512)
        assert ghip.apus_ghip_store_load_container(s, str(tmp_path).encode(), 3,
                                                   ctypes.byref(n), err, 512) == 0, err.value
        assert n.value == E - 1
        got = np.empty(sb, np.uint8)
        for e in range(E):
            assert ghip.apus_ghip_store_get(s, e, O.ptr(got), sb) == 0
            assert np.array_equal(got, l4[6] if e == 6 else l3[e]), e
        bank = [l4[6] if e == 6 else l3[e] for e in range(E)]
        x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
        idx = np.array([6, 2, 11], np.int32)
        w = np.array([0.5, 0.3, 0.2], np.float32)
        out = np.empty(dim, np.uint16)
        assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), 3, O.ptr(out)) == 0
        want, eo = O.moe_forward(bank, dim, inter, x, idx[None], w[None], want_expert_out=True)
        assert_close_combined(out, want[0], moe_floor(eo, w[None], idx[None])[0],
                              "decode over a container-loaded bank")
        assert ghip.apus_ghip_store_load_container(s, str(tmp_path).encode(), 4,
                                                   ctypes.byref(n), err, 512) == 0
        assert n.value == E
        assert ghip.apus_ghip_store_get(s, 0, O.ptr(got), sb) == 0
        assert np.array_equal(got, l4[0])
        # a container for another slab size is refused, nothing loaded
        s2 = open_store(ghip, E, dim, 2 * inter)
        try:
            assert ghip.apus_ghip_store_load_container(s2, str(tmp_path).encode(), 3,
                                                       ctypes.byref(n), err, 512) == 1
            assert b"holds" in err.value and n.value == 0
        finally:
            ghip.apus_ghip_store_close(s2)
    finally:
        ghip.apus_ghip_store_close(s)


def test_store_synth_matches_host_generator(ghip, pkg):
    """The device synthetic fill writes the host generator's slab
    (include/apus_synth.h streams), read back through store_get."""
    lib = pkg.load()
    E, dim, inter, seed, bank = 3, 256, 128, 0x5EED, 2
    s = open_store(ghip, E, dim, inter)
    try:
        assert ghip.apus_ghip_store_synth(s, seed, bank, 1e-4, 1e-2) == 0
        sb = ghip.apus_ghip_store_slab_bytes(s)
        for e in range(E):
            parts = []
            for j, (o, k) in enumerate([(inter, dim), (inter, dim), (dim, inter)]):
                c = np.empty(o * k, np.uint8)
                lib.apus_synth_fp8_codes(O.ptr(c), c.size, seed,
                                         lib.apus_synth_expert_stream(bank, e, 2 * j), 0)
                sc = np.empty(O.nblocks(o) * O.nblocks(k), np.float32)
                lib.apus_synth_scales(O.ptr(sc), sc.size, seed,
                                      lib.apus_synth_expert_stream(bank, e, 2 * j + 1),
                                      ctypes.c_float(1e-4), ctypes.c_float(1e-2))
                parts += [c, sc.view(np.uint8)]
            want = np.concatenate(parts)
            got = np.empty(sb, np.uint8)
            assert ghip.apus_ghip_store_get(s, e, O.ptr(got), sb) == 0
            assert np.array_equal(got, want), e
    finally:
        ghip.apus_ghip_store_close(s)


def test_store_dequant_on_fill_bitwise(small):
    ghip, s, slabs, (E, dim, inter) = small
    for e in (0, 3, 15):
        pl = np.empty(3 * inter * dim, np.uint16)
        assert ghip.apus_ghip_store_expert_bf16(s, e, O.ptr(pl)) == 0
        want = np.empty_like(pl)
        O.lib().apo_slab_dequant(O.ptr(slabs[e]), dim, inter, O.ptr(want), 1)
        assert np.array_equal(pl, want), e


@pytest.mark.parametrize("k", [1, 3, 8])
def test_moe_decode_vs_oracle(small, k):
    ghip, s, slabs, (E, dim, inter) = small
    rng = np.random.default_rng(k)
    for trial in range(4):
        x = O.f32_to_bf16((rng.standard_normal(dim) * (1 + 3 * trial)).astype(np.float32))
        idx = rng.permutation(E)[:k].astype(np.int32)
        if trial == 1:
            idx[0] = 3                       # the expert holding NaN codes
            idx = np.unique(np.concatenate([[3], idx]))[:k].astype(np.int32)
            idx = rng.permutation(idx).astype(np.int32)
        w = rng.uniform(0.01, 1.0, idx.size).astype(np.float32)
        out = np.empty(dim, np.uint16)
        rc = ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), idx.size,
                                       O.ptr(out))
        assert rc == 0, ghip.apus_ghip_last_error()
        want, eo = O.moe_forward(slabs, dim, inter, x, idx[None], w[None],
                                 want_expert_out=True)
        assert_close_combined(out, want[0], moe_floor(eo, w[None], idx[None])[0],
                     "k=%d trial %d" % (k, trial))
        out2 = np.empty(dim, np.uint16)
        assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), idx.size,
                                         O.ptr(out2)) == 0
        assert np.array_equal(out, out2), "run-to-run determinism"


@pytest.mark.parametrize("dim,inter,k", [(256, 128, 12), (4352, 128, 4), (4352, 256, 11),
                                         (256, 384, 8), (512, 640, 5)])
def test_moe_decode_multipass(ghip, dim, inter, k):
    """The decode's second passes: more than 8 slots (the down phase takes
    the slots 8 at a time per workgroup) and more 16-row output groups than
    workgroups (a workgroup takes a second row group, reusing its staged
    h), and intermediate sizes of an odd count of 128-blocks (the h
    hand-off words hold row pairs), against the oracle and run to run."""
    E = 16
    rng = np.random.default_rng(dim + k)
    slabs = random_slabs(E, dim, inter, rng, nan_codes_in=(5,))
    s = open_store(ghip, E, dim, inter)
    try:
        for e, sl in enumerate(slabs):
            assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
        for trial in range(2):
            x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
            idx = rng.permutation(E)[:k].astype(np.int32)
            w = rng.uniform(0.01, 1.0, k).astype(np.float32)
            out = np.empty(dim, np.uint16)
            assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), k,
                                             O.ptr(out)) == 0, ghip.apus_ghip_last_error()
            want, eo = O.moe_forward(slabs, dim, inter, x, idx[None], w[None],
                                     want_expert_out=True)
            assert_close_combined(out, want[0], moe_floor(eo, w[None], idx[None])[0],
                                  "dim=%d k=%d trial %d" % (dim, k, trial))
            out2 = np.empty(dim, np.uint16)
            assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), k,
                                             O.ptr(out2)) == 0
            assert np.array_equal(out, out2), "run-to-run determinism"
    finally:
        ghip.apus_ghip_store_close(s)


def test_moe_decode_duplicate_ids_first_slot(small):
    ghip, s, slabs, (E, dim, inter) = small
    rng = np.random.default_rng(99)
    x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
    idx = np.array([5, 2, 5, 9], np.int32)
    w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    out = np.empty(dim, np.uint16)
    assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), 4, O.ptr(out)) == 0
    want, eo = O.moe_forward(slabs, dim, inter, x, idx[None], w[None],
                             want_expert_out=True)
    fl = moe_floor(eo[:, [0, 1, 3]], w[None, [0, 1, 3]], None)[0]
    assert_close_combined(out, want[0], fl, "duplicate ids")


def test_moe_decode_dev_logits(small):
    """Routing on the device: stable top-k of f32 logits + softmax."""
    ghip, s, slabs, (E, dim, inter) = small
    rng = np.random.default_rng(5)
    logits = rng.standard_normal(E).astype(np.float32)
    logits[7] = logits[11] = np.float32(3.5)          # a tie -> lower id first
    x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
    idx, w = O.route_softmax(logits, 8)
    want, eo = O.moe_forward(slabs, dim, inter, x, idx[None], w[None],
                             want_expert_out=True)
    dx, dl, dout = G.dev(x), G.dev(logits), G.empty(dim * 2)
    assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), G.vp(dl), None, None, 8,
                                         G.vp(dout), G.stream()) == 0
    assert_close_combined(G.host(dout, np.uint16, (dim,)), want[0],
                 moe_floor(eo, w[None], idx[None])[0], "device routing")


@pytest.mark.parametrize("topk", [3, 12, 16])
def test_moe_decode_dev_logits_topk(small, topk):
    """Device routing at other top-k: fewer slots than waves, and more (a
    second down pass per workgroup; the combine over 16 positions, its
    weights placed by the softmax step), with a tie inside the selection."""
    ghip, s, slabs, (E, dim, inter) = small
    rng = np.random.default_rng(50 + topk)
    for trial in range(2):
        logits = rng.standard_normal(E).astype(np.float32)
        logits[2] = logits[9] = np.float32(2.75)      # a tie -> lower id first
        x = O.f32_to_bf16((rng.standard_normal(dim) * (1 + 2 * trial)).astype(np.float32))
        idx, w = O.route_softmax(logits, topk)
        want, eo = O.moe_forward(slabs, dim, inter, x, idx[None], w[None],
                                 want_expert_out=True)
        dx, dl, dout = G.dev(x), G.dev(logits), G.empty(dim * 2)
        assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), G.vp(dl), None, None, topk,
                                             G.vp(dout), G.stream()) == 0
        assert_close_combined(G.host(dout, np.uint16, (dim,)), want[0],
                              moe_floor(eo, w[None], idx[None])[0],
                              "device routing topk=%d trial %d" % (topk, trial))
        assert status(ghip, s, stream=G.stream()) == 0


def test_config2_golden(ghip, pkg):
    """288-expert synthetic bank (~7.2 GB in HBM), one
    token, device top-8 + softmax; expected output written by the reference
    kernels (tests/golden/gen_golden.py)."""
    man = json.load(open(os.path.join(GOLD, "manifest.json")))["config2"]
    fx = np.load(os.path.join(GOLD, "fixtures.npz"))
    lib = pkg.load()
    E, k, dim, inter, seed = man["E"], man["topk"], man["dim"], man["inter"], man["seed"]
    s = open_store(ghip, E, dim, inter)
    try:
        assert ghip.apus_ghip_store_synth(s, seed, 0, 1e-4, 1e-2) == 0
        logits = np.empty(E, np.float32)
        lib.apus_synth_f32_normal(O.ptr(logits), E, seed, 20, 0)
        x = np.empty(dim, np.uint16)
        lib.apus_synth_bf16_normal(O.ptr(x), dim, seed, 21, 0)
        idx, w = O.route_softmax(logits, k)
        assert list(idx) == man["idx"]
        fl = moe_floor(fx["cfg2_expert_out"][None], w[None], idx[None])[0]
        dx, dl, dout = G.dev(x), G.dev(logits), G.empty(dim * 2)
        assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), G.vp(dl), None, None, k,
                                             G.vp(dout), G.stream()) == 0
        st = assert_close_combined(G.host(dout, np.uint16, (dim,)), fx["cfg2_out"], fl,
                          "config2 device routing")
        print("config2", st)
        record("config2_golden_device_routing", st)
        out = np.empty(dim, np.uint16)
        assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), k,
                                         O.ptr(out)) == 0
        st = assert_close_combined(out, fx["cfg2_out"], fl, "config2 host routing")
        record("config2_golden_host_routing", st)
    finally:
        ghip.apus_ghip_store_close(s)


def test_moe_decode_tag_wrap(ghip):
    """The launch tag is 16 bits: launch 65536 on a workspace clears the
    router's logit words (a fill kernel ordered on the stream) and restarts
    at tag 1, while the h buffers keep alternating. Calls on both sides of
    the wrap, enqueued back to back after 65,527 others, give the outputs
    the same inputs gave on the fresh workspace, bitwise."""
    E, dim, inter = 16, 256, 128
    rng = np.random.default_rng(65536)
    slabs = random_slabs(E, dim, inter, rng)
    s = open_store(ghip, E, dim, inter)
    try:
        for e, sl in enumerate(slabs):
            assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
        calls = []
        for k in (8, 3, 8, 5, 8, 1):
            x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
            idx = rng.choice(E, k, replace=False).astype(np.int32)
            w = rng.uniform(0.05, 0.5, k).astype(np.float32)
            calls.append((x, idx, w))
        fresh = []
        for x, idx, w in calls:                   # launches 1..6 (tags 1..6)
            out = np.empty(dim, np.uint16)
            assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), len(idx),
                                             O.ptr(out)) == 0, ghip.apus_ghip_last_error()
            fresh.append(out)
        x0, i0, w0 = calls[0]
        dx, di, dw, do = G.dev(x0), G.dev(i0), G.dev(w0), G.empty(dim * 2)
        st = G.stream()
        for _ in range(65533 - 6):                # launches 7..65533
            assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw),
                                                 len(i0), G.vp(do), st) == 0
        bufs = [(G.dev(x), G.dev(idx), G.dev(w), G.empty(dim * 2), len(idx))
                for x, idx, w in calls]
        for bx, bi, bw, bo, k in bufs:            # launches 65534..65539 (wrap at 65536)
            assert ghip.apus_ghip_moe_decode_dev(s, G.vp(bx), None, G.vp(bi), G.vp(bw), k,
                                                 G.vp(bo), st) == 0
        for n, ((bx, bi, bw, bo, k), want) in enumerate(zip(bufs, fresh)):
            assert np.array_equal(G.host(bo, np.uint16, (dim,)), want), \
                "launch %d (k=%d) across the tag wrap" % (65534 + n, k)
        assert np.array_equal(G.host(do, np.uint16, (dim,)), fresh[0])
        assert status(ghip, s) == 0, "no device failure across 65,539 launches"
    finally:
        ghip.apus_ghip_store_close(s)


def test_moe_decode_refuses_graph_capture(small):
    """Which h buffer a decode call writes is host state flipped per call
    (with the launch tag), so a launch recorded into a HIP graph would
    replay into a stale buffer: the device entry refuses a capturing stream
    (returns 1, launches nothing), the capture ends cleanly, and calls
    afterwards are unaffected."""
    ghip, s, slabs, (E, dim, inter) = small
    rt = G.rt()
    rng = np.random.default_rng(404)
    x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
    idx = rng.choice(E, 4, replace=False).astype(np.int32)
    w = rng.uniform(0.05, 0.5, 4).astype(np.float32)
    want = np.empty(dim, np.uint16)
    assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), 4, O.ptr(want)) == 0
    dx, di, dw, do = G.dev(x), G.dev(idx), G.dev(w), G.empty(dim * 2)
    st = rt.Stream()
    g = rt.Graph(st)
    g.begin()
    try:
        rc = ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), 4,
                                           G.vp(do), st.vp)
    finally:
        g.end()
        g.close()
    assert rc == 1
    assert b"captur" in ghip.apus_ghip_last_error().lower()
    assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), 4,
                                         G.vp(do), st.vp) == 0
    st.synchronize()
    assert np.array_equal(G.host(do, np.uint16, (dim,)), want)


def test_moe_decode_back_to_back_calls(small):
    """Decode calls enqueued back to back on one stream, no host sync in
    between: a launch writes h into the buffer the launch before it refilled
    with the sentinel (the two buffers alternate), so a launch never takes
    an earlier launch's h for its own, and every output equals the same
    call run alone, bitwise."""
    ghip, s, slabs, (E, dim, inter) = small
    rng = np.random.default_rng(21)
    calls = []
    for k in (4, 1, 8, 3, 8):
        x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
        idx = rng.choice(E, k, replace=False).astype(np.int32)
        w = rng.uniform(0.05, 0.5, k).astype(np.float32)
        calls.append((x, idx, w))
    alone = []
    for x, idx, w in calls:
        out = np.empty(dim, np.uint16)
        assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), len(idx),
                                         O.ptr(out)) == 0
        alone.append(out)
    bufs = [(G.dev(x), G.dev(idx), G.dev(w), G.empty(dim * 2), len(idx)) for x, idx, w in calls]
    for dx, di, dw, do, k in bufs:
        assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), k,
                                             G.vp(do), G.stream()) == 0
    for (dx, di, dw, do, k), want in zip(bufs, alone):
        assert np.array_equal(G.host(do, np.uint16, (dim,)), want), "k=%d back to back" % k
    assert status(ghip, s) == 0


def test_moe_decode_refused_calls_between_launches(small):
    """Calls the entry refuses (topk 0 or past 16) launch nothing and leave
    the workspace's h-buffer parity where it was: valid calls enqueued back
    to back with refused ones between them give the outputs they give run
    alone, bitwise, and no device failure is recorded."""
    ghip, s, slabs, (E, dim, inter) = small
    rng = np.random.default_rng(33)
    calls = []
    for k in (8, 5, 8, 2):
        x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
        idx = rng.choice(E, k, replace=False).astype(np.int32)
        w = rng.uniform(0.05, 0.5, k).astype(np.float32)
        calls.append((x, idx, w))
    alone = []
    for x, idx, w in calls:
        out = np.empty(dim, np.uint16)
        assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), len(idx),
                                         O.ptr(out)) == 0
        alone.append(out)
    bufs = [(G.dev(x), G.dev(idx), G.dev(w), G.empty(dim * 2), len(idx)) for x, idx, w in calls]
    for dx, di, dw, do, k in bufs:
        assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), k,
                                             G.vp(do), G.stream()) == 0
        for bad in (0, 17):
            assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), bad,
                                                 G.vp(do), G.stream()) != 0
    for (dx, di, dw, do, k), want in zip(bufs, alone):
        assert np.array_equal(G.host(do, np.uint16, (dim,)), want), "k=%d" % k
    assert status(ghip, s) == 0


def test_moe_decode_all_ones_nan_activations(small):
    """An h pair of two all-ones NaNs (0xffff, 0xffff) would read as the
    hand-off's "not written yet" sentinel; the decode stores such a pair
    with the even row's NaN payload one lower. A token whose activations
    are all that NaN (whether its h pairs collide depends on the NaN
    payload the device arithmetic carries) must still end promptly: no
    hand-off error, every output NaN like the oracle's, and the next call
    on the same store within the tolerance of the oracle."""
    ghip, s, slabs, (E, dim, inter) = small
    x = np.full(dim, 0xFFFF, np.uint16)
    idx = np.array([0, 5, 9, 12], np.int32)
    w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    out = np.empty(dim, np.uint16)
    assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), len(idx),
                                     O.ptr(out)) == 0, ghip.apus_ghip_last_error()
    assert status(ghip, s) == 0
    want = O.moe_forward(slabs, dim, inter, x, idx[None], w[None])[0]
    nan = lambda b: ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    assert nan(want).all()
    assert nan(out).all()
    rng = np.random.default_rng(77)
    x2 = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
    after = np.empty(dim, np.uint16)
    assert ghip.apus_ghip_moe_decode(s, O.ptr(x2), O.ptr(idx), O.ptr(w), len(idx),
                                     O.ptr(after)) == 0, ghip.apus_ghip_last_error()
    want2, eo = O.moe_forward(slabs, dim, inter, x2, idx[None], w[None], want_expert_out=True)
    assert_close_combined(after, want2[0], moe_floor(eo, w[None], idx[None])[0],
                          "the call after the NaN token")


def status(ghip, s, clear=1, stream=None):
    code = ctypes.c_uint32(0xFFFFFFFF)
    assert ghip.apus_ghip_store_status(s, stream, clear, ctypes.byref(code)) == 0, \
        ghip.apus_ghip_last_error()
    return code.value


def test_store_status_reports_dev_failures(small):
    """The asynchronous entries return 0 once queued; an id outside the bank
    is dropped on the device and ORed into the store's sticky error word
    (bit 2), which apus_ghip_store_status reads after the stream and clears
    on request. A valid call leaves the word at 0, and the host-pointer
    decode reports only its own launch (it resets the word first)."""
    ghip, s, slabs, (E, dim, inter) = small
    assert status(ghip, s) == 0
    rng = np.random.default_rng(808)
    x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
    good = np.array([1, 4, 9], np.int32)
    bad = np.array([1, E, 9], np.int32)                 # id E is outside the bank
    w = np.array([0.5, 0.3, 0.2], np.float32)
    dx, dw, do = G.dev(x), G.dev(w), G.empty(dim * 2)
    dg, db = G.dev(good), G.dev(bad)
    assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(dg), G.vp(dw), 3,
                                         G.vp(do), G.stream()) == 0
    assert status(ghip, s) == 0
    assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(db), G.vp(dw), 3,
                                         G.vp(do), G.stream()) == 0
    assert status(ghip, s, clear=0) == 2                # read, kept
    assert status(ghip, s) == 2                         # read, cleared
    assert status(ghip, s) == 0
    # the decode without the dropped id: same output as the valid pair alone
    want = np.empty(dim, np.uint16)
    two, w2 = np.array([1, 9], np.int32), np.array([0.5, 0.2], np.float32)
    assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(two), O.ptr(w2), 2,
                                     O.ptr(want)) == 0
    assert np.array_equal(G.host(do, np.uint16, (dim,)), want)
    # prefill: the same word, bit 2
    T = 3
    xs = O.f32_to_bf16(rng.standard_normal((T, dim)).astype(np.float32))
    pidx = np.array([[0, 1], [2, E + 5], [3, 4]], np.int32)
    pw = np.ones((T, 2), np.float32)
    px, pi, pwd, po = G.dev(xs), G.dev(pidx), G.dev(pw), G.empty(T * dim * 2)
    assert ghip.apus_ghip_moe_prefill_dev(s, G.vp(px), T, G.vp(pi), G.vp(pwd), 2,
                                          G.vp(po), G.stream()) == 0
    assert status(ghip, s) == 2
    # a pending device failure is not reported by a later host-pointer call
    assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(db), G.vp(dw), 3,
                                         G.vp(do), G.stream()) == 0
    out = np.empty(dim, np.uint16)
    assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(good), O.ptr(w), 3,
                                     O.ptr(out)) == 0, ghip.apus_ghip_last_error()
    assert status(ghip, s) == 0
