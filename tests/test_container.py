"""The converted-container index reader (CPU only): apus.index.json of a v2
glm5_next container, slab records per layer (c/gcache.h:832-930), the
record checks the reference makes (format/model type, one slab per
record), against containers written by tests/container_util.py."""
import ctypes
import json
import os

import numpy as np
import pytest

from container_util import write_container


def lookup(lib, d, layer, e, slab_bytes):
    shard = ctypes.create_string_buffer(256)
    off = ctypes.c_uint64()
    err = ctypes.create_string_buffer(512)
    rc = lib.apus_ghip_container_slab(d.encode(), layer, e, slab_bytes, shard, 256,
                                      ctypes.byref(off), err, 512)
    return rc, shard.value.decode(), off.value, err.value.decode()


@pytest.fixture()
def lib(pkg):
    return pkg.load()


def test_records_found_per_layer(lib, tmp_path):
    rng = np.random.default_rng(1)
    sb = 1000
    layers = {3: {e: rng.integers(0, 256, sb, dtype=np.uint8) for e in (0, 5, 7)},
              4: {e: rng.integers(0, 256, sb, dtype=np.uint8) for e in (5,)}}
    recs = write_container(str(tmp_path), layers, sb)
    for r in recs:
        layer = int(r["block"].split(".")[1])
        rc, shard, off, err = lookup(lib, str(tmp_path), layer, r["expert"], sb)
        assert rc == 0, err
        assert shard == r["shard"] and off == r["offset"]
        with open(os.path.join(tmp_path, shard), "rb") as f:
            f.seek(off)
            assert f.read(sb) == layers[layer][r["expert"]].tobytes()
    rc, _, _, err = lookup(lib, str(tmp_path), 3, 1, sb)          # no record
    assert rc == 1 and "no slab record" in err
    rc, _, _, err = lookup(lib, str(tmp_path), 4, 5, sb + 1)      # slab size
    assert rc == 1 and "holds 1000 bytes" in err


@pytest.mark.parametrize("fmt,mt", [(1, "glm5_next"), (2, "glm5")])
def test_rejects_other_containers(lib, tmp_path, fmt, mt):
    write_container(str(tmp_path), {3: {0: np.zeros(64, np.uint8)}}, 64, fmt=fmt,
                    model_type=mt)
    rc, _, _, err = lookup(lib, str(tmp_path), 3, 0, 64)
    assert rc == 1 and "not a glm5_next v2 container" in err


def test_rejects_bad_record_and_bad_json(lib, tmp_path):
    write_container(str(tmp_path), {3: {0: np.zeros(64, np.uint8), 1: np.zeros(64, np.uint8)}},
                    64, bad_nbytes=(3, 1))
    rc, _, _, err = lookup(lib, str(tmp_path), 3, 0, 64)
    assert rc == 1 and "(layers.3, 1) holds 68 bytes" in err
    p = os.path.join(tmp_path, "apus.index.json")
    idx = json.load(open(p))
    idx["expert_slabs"][0]["block"] = "blocks.3"
    json.dump(idx, open(p, "w"))
    rc, _, _, err = lookup(lib, str(tmp_path), 3, 0, 64)
    assert rc == 1 and "bad slab record" in err
    open(p, "w").write('{"format_version": 2, "model_type": "glm5_next", "expert_slabs": [')
    rc, _, _, err = lookup(lib, str(tmp_path), 3, 0, 64)
    assert rc == 1 and "index json" in err
    rc, _, _, err = lookup(lib, str(tmp_path / "absent"), 3, 0, 64)
    assert rc == 1 and "cannot open" in err


def test_string_escapes_and_unicode(lib, tmp_path):
    """Shard names go through the JSON string decoder (escapes, \\u)."""
    d = str(tmp_path)
    write_container(d, {3: {2: np.arange(64, dtype=np.uint8)}}, 64,
                    shard_of=lambda layer: "apus-A.safetensors")
    p = os.path.join(d, "apus.index.json")
    txt = open(p).read().replace('"shard": "apus-A.safetensors"',
                                 '"shard": "apus-\\u0041.safe\\u0074ensors"')
    open(p, "w").write(txt)
    rc, shard, off, err = lookup(lib, d, 3, 2, 64)
    assert rc == 0, err
    assert shard == "apus-A.safetensors"


@pytest.mark.parametrize("bad", [4294967296, 2147483648, -1, 1.5, 1e300])
def test_rejects_expert_id_out_of_int_range(lib, tmp_path, bad):
    """An expert id that does not fit an int (or is not an integer) is a bad
    record: cast to int it would wrap negative and index far outside the
    store (the reference bounds the parsed long, c/gcache.h:911-913)."""
    d = str(tmp_path)
    write_container(d, {3: {0: np.zeros(64, np.uint8), 1: np.zeros(64, np.uint8)}}, 64)
    p = os.path.join(d, "apus.index.json")
    idx = json.load(open(p))
    idx["expert_slabs"][1]["expert"] = bad
    json.dump(idx, open(p, "w"))
    rc, _, _, err = lookup(lib, d, 3, 0, 64)
    assert rc == 1 and "bad slab record 1" in err
