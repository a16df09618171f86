"""Writes small converted-v2 containers (tests/m1/README.md:21-55 schema:
apus.index.json with expert_slabs records {block, expert, shard, offset,
nbytes}, safetensors shards whose data region holds the six members of each
expert slab contiguously) for the container-loader tests."""
import json
import os
import struct


def write_container(root, layers, slab_bytes, fmt=2, model_type="glm5_next",
                    bad_nbytes=None, shard_of=lambda layer: "apus-%05d.safetensors" % (layer % 2 + 1)):
    """layers: {layer: {expert: slab bytes (np.uint8)}}. Each shard starts
    with a safetensors header (u64 length + JSON), then the slabs back to
    back; records carry file-absolute offsets."""
    os.makedirs(root, exist_ok=True)
    shards = {}
    for layer, experts in layers.items():
        for e, slab in experts.items():
            shards.setdefault(shard_of(layer), []).append((layer, e, slab))
    records, tmap = [], {}
    for name, items in shards.items():
        hdr = json.dumps({"__metadata__": {"format": "pt"}}).encode()
        hdr += b" " * ((8 - len(hdr) % 8) % 8)
        data_off = 8 + len(hdr)
        with open(os.path.join(root, name), "wb") as f:
            f.write(struct.pack("<Q", len(hdr)))
            f.write(hdr)
            off = data_off
            for layer, e, slab in items:
                f.write(slab.tobytes())
                nb = slab.nbytes
                if bad_nbytes is not None and (layer, e) == bad_nbytes:
                    nb += 4
                records.append({"block": "layers.%d" % layer, "expert": int(e),
                                "shard": name, "offset": off, "nbytes": nb})
                tmap["layers.%d.mlp.experts.%d.gate_proj.weight" % (layer, e)] = {
                    "shard": name, "offset": off}
                off += slab.nbytes
    index = {"format_version": fmt, "model_type": model_type, "config_hash": "0" * 16,
             "header_reserve": 16 << 20, "n_main_layers": 45,
             "expert_slab_members": ["gate_proj.weight", "gate_proj.weight_scale_inv",
                                     "up_proj.weight", "up_proj.weight_scale_inv",
                                     "down_proj.weight", "down_proj.weight_scale_inv"],
             "tensor_map": tmap, "expert_slabs": records,
             "stripped": {"tensors": 347, "note": "vision \\u0041 stripped"}}
    with open(os.path.join(root, "apus.index.json"), "w") as f:
        json.dump(index, f, indent=1)
    return records
