"""Checkpoint reading without a GPU: the safetensors container and the weight
index (src/format/safetensor.rs, src/model/weights.rs) and the checkpoint
validation of the runner's load (src/model/runner.rs:337-417, 2443-2457,
3769-3946), through the product's C ABI (lisa_weight_index_*)."""
import json
import struct

import numpy as np
import pytest

from _lisa import load_pkg
from _safetensors import layout, mtp_spec, target_spec, write_safetensors, write_snapshot

LAYERS, VOCAB = 4, 4096


def index(paths):
    return load_pkg().WeightIndex(paths=[str(p) for p in paths])


def test_reference_synthetic_shard(tmp_path):
    """safetensor.rs:104-133: two tensors tile a 40-byte data region; offsets
    are relative to the end of the header."""
    header = b'{"a":{"dtype":"F32","shape":[2,3],"data_offsets":[0,24]},' \
             b'"b":{"dtype":"BF16","shape":[8],"data_offsets":[24,40]}}'
    path = tmp_path / "engine_export.safetensors"
    path.write_bytes(struct.pack("<Q", len(header)) + header + bytes(40))
    idx = index([path])
    base = 8 + len(header)
    assert len(idx) == 2 and idx.shard_count == 1
    a, b = idx.slot("a"), idx.slot("b")
    assert a["data_start"] + a["offset"] == base and a["len"] == 24
    assert a["dtype"] == "F32" and a["shape"] == [2, 3]
    assert b["data_start"] + b["offset"] == base + 24 and b["len"] == 16
    assert b["dtype"] == "BF16" and b["shape"] == [8]


def test_metadata_escapes_and_values(tmp_path):
    path = tmp_path / "m.safetensors"
    arr = np.arange(6, dtype=np.uint32).reshape(2, 3)
    write_safetensors(path, {"wéight/\"q\"": arr, "z": ("BF16", (0,))},
                      metadata={"format": "mlx", "nested": "x"})
    idx = index([path])
    assert len(idx) == 2  # __metadata__ is not a tensor
    s = idx.slot("wéight/\"q\"")
    assert s["dtype"] == "U32" and s["shape"] == [2, 3] and s["len"] == 24
    raw = path.read_bytes()
    got = np.frombuffer(raw[s["data_start"] + s["offset"]:][:24], np.uint32)
    assert np.array_equal(got, arr.ravel())
    assert idx.slot("z")["len"] == 0


def test_index_over_shards_and_duplicates(tmp_path):
    p1, p2 = tmp_path / "a.safetensors", tmp_path / "b.safetensors"
    write_safetensors(p1, {"x": np.zeros(4, np.uint16), "y": np.ones(2, np.float32)})
    write_safetensors(p2, {"z": np.zeros(8, np.uint32)})
    idx = index([p1, p2])
    assert len(idx) == 3 and idx.shard_count == 2
    assert idx.slot("z")["shard"] == 1 and idx.slot("y")["shard"] == 0
    write_safetensors(p2, {"x": np.zeros(4, np.uint16)})
    with pytest.raises(load_pkg().LisaError, match="duplicate tensor x"):
        index([p1, p2])


@pytest.mark.parametrize("entry,message", [
    ({"dtype": "Q8", "shape": [4], "data_offsets": [0, 4]}, "unknown dtype Q8"),
    ({"dtype": "U32", "shape": [2], "data_offsets": [0, 16]}, "outside the"),
    ({"dtype": "U32", "shape": [3], "data_offsets": [0, 8]}, "need 12"),
    ({"dtype": "U32", "shape": [2], "data_offsets": [8, 0]}, "outside the"),
    ({"dtype": "U32", "shape": [-2], "data_offsets": [0, 8]}, "shape"),
    ({"dtype": "U32", "shape": [2]}, "required"),
])
def test_malformed_shards_are_rejected(tmp_path, entry, message):
    header = json.dumps({"t": entry}).encode()
    path = tmp_path / "bad.safetensors"
    path.write_bytes(struct.pack("<Q", len(header)) + header + bytes(8))
    with pytest.raises(load_pkg().LisaError, match=message):
        index([path])


def test_truncated_header_is_rejected(tmp_path):
    path = tmp_path / "t.safetensors"
    path.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(load_pkg().LisaError, match="header length"):
        index([path])
    path.write_bytes(struct.pack("<Q", 5) + b'{"a":')
    with pytest.raises(load_pkg().LisaError, match="parse safetensors header"):
        index([path])


def test_snapshot_listing(tmp_path):
    pkg = load_pkg()
    with pytest.raises(pkg.LisaError, match="no safetensors shards in"):
        pkg.WeightIndex(snapshot=tmp_path)
    with pytest.raises(pkg.LisaError, match="read snapshot"):
        pkg.WeightIndex(snapshot=tmp_path / "absent")
    (tmp_path / "notes.txt").write_text("not a shard")
    write_safetensors(tmp_path / "b.safetensors", {"y": np.zeros(2, np.uint16)})
    write_safetensors(tmp_path / "a.safetensors", {"x": np.zeros(2, np.uint16)})
    idx = pkg.WeightIndex(snapshot=tmp_path)
    assert len(idx) == 2 and idx.slot("x")["shard"] == 0 and idx.slot("y")["shard"] == 1  # sorted paths


@pytest.fixture(scope="module")
def target_layout():
    return layout(target_spec(LAYERS, VOCAB))


def snapshot(tmp_path, tensors, shards=3, extra=None):
    return load_pkg().WeightIndex(snapshot=write_snapshot(tmp_path, tensors, shards, extra))


def test_target_checkpoint_validates(tmp_path, target_layout):
    extra = {"vision_tower.patch_embed.weight": ("BF16", (16, 16))}  # tensors the runner does not read
    idx = snapshot(tmp_path, target_layout, extra=extra)
    assert len(idx) == len(target_layout) + 1 and idx.shard_count == 3
    idx.validate(LAYERS, VOCAB)
    # a model of the other geometry is not this checkpoint
    with pytest.raises(load_pkg().LisaError, match="missing tensor language_model.model.layers.4.input_layernorm"):
        idx.validate(8, VOCAB)
    with pytest.raises(load_pkg().LisaError, match="invalid tensor language_model.model.embed_tokens.weight"):
        idx.validate(LAYERS, 2 * VOCAB)


@pytest.mark.parametrize("name,change,message", [
    ("language_model.model.layers.3.self_attn.k_norm.weight", None,
     "missing tensor language_model.model.layers.3.self_attn.k_norm.weight"),
    ("language_model.model.layers.0.linear_attn.in_proj_b.scales", None,
     "missing tensor language_model.model.layers.0.linear_attn.in_proj_b.scales"),
    ("language_model.lm_head.biases", None, "missing tensor language_model.lm_head.biases"),
    ("language_model.model.layers.1.input_layernorm.weight", ("F32", (5120,)),
     r"invalid tensor language_model.model.layers.1.input_layernorm.weight: F32 \[5120\], expected BF16 \[5120\]"),
    ("language_model.model.layers.2.linear_attn.conv1d.weight", ("BF16", (10240, 4)),
     r"invalid tensor language_model.model.layers.2.linear_attn.conv1d.weight: BF16 \[10240, 4\], "
     r"expected BF16 \[10240, 4, 1\]"),
    ("language_model.model.layers.0.mlp.down_proj.weight", ("U32", (5120, 17408 // 8 + 1)),
     r"invalid tensor language_model.model.layers.0.mlp.down_proj.weight: U32 \[5120, 2177\]"),
    ("language_model.model.layers.3.mlp.gate_proj.scales", ("F16", (17408, 80)),
     "invalid tensor language_model.model.layers.3.mlp.gate_proj.scales: F16"),
])
def test_target_checkpoint_errors(tmp_path, target_layout, name, change, message):
    t = dict(target_layout)
    if change is None:
        del t[name]
    else:
        t[name] = change
    idx = snapshot(tmp_path, t)
    with pytest.raises(load_pkg().LisaError, match=message):
        idx.validate(LAYERS, VOCAB)


def test_mtp_checkpoint_validation(tmp_path):
    spec = layout(mtp_spec())
    assert len(spec) == 31
    idx = snapshot(tmp_path / "ok", spec, shards=1)
    idx.validate(LAYERS, VOCAB, mtp=True)
    more = dict(spec)
    more["layers.0.extra.weight"] = ("BF16", (4,))
    with pytest.raises(load_pkg().LisaError, match="invalid MTP checkpoint: found 32 tensors, expected 31"):
        snapshot(tmp_path / "more", more, shards=1).validate(mtp=True)
    swapped = dict(spec)
    del swapped["fc.biases"]
    swapped["fc.bias"] = ("BF16", (5120, 160))
    with pytest.raises(load_pkg().LisaError, match="missing tensor fc.biases"):
        snapshot(tmp_path / "swap", swapped, shards=1).validate(mtp=True)
    wrong = dict(spec)
    wrong["fc.weight"] = ("U32", (10240, 5120 // 8))  # fc is (out 5120, in 10240)
    with pytest.raises(load_pkg().LisaError, match=r"invalid tensor fc.weight: U32 \[10240, 640\], expected U32 \[5120, 1280\]"):
        snapshot(tmp_path / "wrong", wrong, shards=1).validate(mtp=True)
