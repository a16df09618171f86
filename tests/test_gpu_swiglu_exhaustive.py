"""The SwiGLU epilogue over its whole input domain, bitwise against the
oracle (c/gmoe.h:217-225 with the numpy-stable sigmoid of c/gmhc.h:157-160
on the host's libm expf, the reference's own).

The gate value g is a bf16 (the gate GEMV's rounded output), so the map
g -> bf16(min(g, limit) * sigmoid(min(g, limit))) has 65,536 inputs. An
expert with one-hot FP8 weights (code 0x38 = 1.0, scale 1.0) passes them
straight through the kernels: gate row i reads x[i] (g_i = x[i] exactly),
every up row reads x[2048] = 1.0 (u = 1), down row j reads h_j (out_j =
h_j), top-1 with weight 1.0 (the combine adds it to +0: out = h, a -0 h
reading +0 in both the GPU and the oracle). Gate row 2047 weighs its
column by 2.0, so x[2047] = +-max bf16 gives g = +-inf (an f32 overflow)
without a non-finite x, which would turn every row's 0 * x into NaN.

  finite g (65,280 codes)  32 tokens of 2,047 codes each, out[0..2046]
  g = +inf                 the last sweep token's row 2047
  g = -inf                 h = -inf * 0 = NaN: its own token, all NaN
  g = NaN (254 codes)      x[0] = NaN: its own token, all outputs NaN

Paths: the decode (one launch per token) and both prefill kernels (all
tokens in one call; one expert of a 3-expert bank takes the one-wave-per-
SIMD bodies, of a 1-expert bank the two-waves-per-SIMD bodies: 256-row
and 31-row tiles). Every finite output is compared bitwise and the
mismatches are recorded per path."""
import numpy as np
import pytest

import oracle as O
from tolerance import record
from test_gpu_moe import open_store
from test_gpu_prefill import prefill

pytestmark = pytest.mark.gpu

DIM, INTER, LIMIT = 4096, 2048, 10.0
ONE, TWO = 0x38, 0x40                       # E4M3 codes of 1.0 and 2.0
BF_MAX, BF_ONE = 0x7F7F, 0x3F80


def onehot_slab():
    gw = np.zeros((INTER, DIM), np.uint8)
    gw[np.arange(INTER), np.arange(INTER)] = ONE
    gw[INTER - 1, INTER - 1] = TWO
    uw = np.zeros((INTER, DIM), np.uint8)
    uw[:, INTER] = ONE
    dw = np.zeros((DIM, INTER), np.uint8)
    dw[np.arange(INTER), np.arange(INTER)] = ONE
    sg = np.ones((O.nblocks(INTER), O.nblocks(DIM)), np.float32)
    sd = np.ones((O.nblocks(DIM), O.nblocks(INTER)), np.float32)
    return np.concatenate([gw.ravel(), sg.view(np.uint8).ravel(), uw.ravel(),
                           sg.view(np.uint8).ravel(), dw.ravel(), sd.view(np.uint8).ravel()])


def tokens():
    """x rows and what each covers: ("sweep", codes at rows 0..n-1, g of
    row 2047) or ("nan", g code)."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    fin = codes[(codes & 0x7F80) != 0x7F80]
    assert fin.size == 65280
    xs, what = [], []
    per = INTER - 1
    for t0 in range(0, fin.size, per):
        x = np.zeros(DIM, np.uint16)
        part = fin[t0:t0 + per]
        x[:part.size] = part
        last = t0 + per >= fin.size
        x[INTER - 1] = BF_MAX if last else 0          # g_2047 = +inf or 0
        x[INTER] = BF_ONE
        xs.append(x)
        what.append(("sweep", part))
    x = np.zeros(DIM, np.uint16)
    x[INTER - 1] = 0x8000 | BF_MAX                    # g_2047 = -inf
    x[INTER] = BF_ONE
    xs.append(x)
    what.append(("nan", 0xFF80))
    for c in codes[((codes & 0x7F80) == 0x7F80) & ((codes & 0x7F) != 0)]:
        x = np.zeros(DIM, np.uint16)
        x[0] = c
        x[INTER] = BF_ONE
        xs.append(x)
        what.append(("nan", int(c)))
    return np.stack(xs), what


@pytest.fixture(scope="module")
def case():
    slab = onehot_slab()
    x, what = tokens()
    T = x.shape[0]
    idx = np.zeros((T, 1), np.int32)
    w = np.ones((T, 1), np.float32)
    want = O.moe_forward([slab], DIM, INTER, x, idx, w, limit=LIMIT, threads=16)
    # the oracle's own reading of the one-hot expert: out_j = h(g_j) for the
    # sweep rows, h(+inf) = h(limit) on row 2047 of the last sweep token
    sig = O.lib().apo_sigmoid_np
    for t, (kind, part) in enumerate(what):
        if kind != "sweep":
            assert np.all(np.isnan(O.bf16_to_f32(want[t]))), t
            continue
        g = np.minimum(O.bf16_to_f32(part), np.float32(LIMIT))
        h = O.f32_to_bf16(np.array([np.float32(v) * np.float32(sig(float(v))) for v in g],
                                   np.float32))
        h = np.where(h == 0x8000, 0, h)               # -0 reads +0 after the sums
        assert np.array_equal(want[t, :part.size], h), t
    return slab, x, what, want


def compare(got, want, what, path):
    mism, nan_bad, rows = [], 0, 0
    for t, (kind, part) in enumerate(what):
        if kind == "nan":
            nan_bad += int(not np.all(np.isnan(O.bf16_to_f32(got[t]))))
            continue
        n = part.size
        rows += n
        bad = np.nonzero(got[t, :n] != want[t, :n])[0]
        mism += [(int(part[i]), int(got[t, i]), int(want[t, i])) for i in bad]
        # row 2047: g = +inf on the last sweep token, 0 on the others; rows
        # past the sweep and the unused output rows
        assert np.array_equal(got[t, n:], want[t, n:]), (path, t)
    record("swiglu_exhaustive_" + path, {"n_gate_codes": rows + 1 + 1 + 254,
                                         "finite_mismatches": len(mism),
                                         "nonfinite_not_nan": nan_bad},
           mismatches=[["0x%04x" % g, "0x%04x" % a, "0x%04x" % b] for g, a, b in mism[:64]])
    print(path, "finite mismatches", len(mism), mism[:16], "non-finite not NaN", nan_bad)
    assert not mism and nan_bad == 0, (path, len(mism), mism[:16], nan_bad)


def test_swiglu_exhaustive_decode(ghip, case):
    slab, x, what, want = case
    s = open_store(ghip, 1, DIM, INTER, LIMIT)
    try:
        assert ghip.apus_ghip_store_put(s, 0, O.ptr(slab), slab.nbytes) == 0
        got = np.empty_like(want)
        idx = np.zeros(1, np.int32)
        w = np.ones(1, np.float32)
        for t in range(x.shape[0]):
            assert ghip.apus_ghip_moe_decode(s, O.ptr(x[t]), O.ptr(idx), O.ptr(w), 1,
                                             O.ptr(got[t])) == 0, ghip.apus_ghip_last_error()
        compare(got, want, what, "decode")
    finally:
        ghip.apus_ghip_store_close(s)


@pytest.mark.parametrize("E,body", [(3, "4wave"), (1, "8wave")])
def test_swiglu_exhaustive_prefill(ghip, case, E, body):
    slab, x, what, want = case
    T = x.shape[0]
    assert (T >= E * 128) == (body == "8wave")      # the launcher's body choice
    s = open_store(ghip, E, DIM, INTER, LIMIT)
    try:
        for e in range(E):
            assert ghip.apus_ghip_store_put(s, e, O.ptr(slab), slab.nbytes) == 0
        idx = np.zeros((T, 1), np.int32)
        w = np.ones((T, 1), np.float32)
        compare(prefill(ghip, s, x, idx, w), want, what, "prefill_" + body)
    finally:
        ghip.apus_ghip_store_close(s)
