"""On-disk expert pack metadata (root/layer_NN.json) through the C ABI's
pbmoe_pack_inspect: host code only, no GPU.  Cases follow the reference's
own tests of ExpertLayerPackMetadata (tests/experts.rs:1336-1391: accepted
fixed-Q4 metadata, duplicate expert, pack longer than its slot, the
layer_NN path scheme, a PBQ4 V2 file read back) and the checks of
ExpertLayerPackMetadata::validate (experts/mod.rs:372-429)."""
from __future__ import annotations

import json
import os

import pytest

from pb_amd import abi, packs


def tiny_pack(layer, expert, packed_bytes):
    # tiny_pack_metadata (tests/experts.rs:1286-1293): no records
    return {"layer": layer, "expert": expert, "packed_bytes": packed_bytes, "records": []}


def meta(fmt, layer, expert_size, experts, pack_list):
    return {"format": fmt, "layer": layer, "expert_size": expert_size, "experts": experts, "packs": pack_list}


def write_json(root, layer, obj_or_text):
    path = os.path.join(root, f"layer_{layer:02d}.json")
    with open(path, "w") as f:
        f.write(obj_or_text if isinstance(obj_or_text, str) else json.dumps(obj_or_text))
    return path


def inspect_rc(root, layer):
    info = abi.PackInfo()
    rc = abi.lib().pbmoe_pack_inspect(str(root).encode(), layer, info)
    return rc, info, abi.lib().pbmoe_last_error().decode()


def test_fixed_q4_metadata_with_partial_packs_is_accepted(tmp_path):
    # expert_layer_metadata_validates_supported_formats_and_slots, first case
    write_json(tmp_path, 3, meta("FIXED_Q4_EXPERT_LAYER_V1", 3, 128, 2, [tiny_pack(3, 0, 128), tiny_pack(3, 1, 64)]))
    info = abi.pack_inspect(tmp_path, 3)
    assert info.format == b"FIXED_Q4_EXPERT_LAYER_V1"
    assert (info.layer, info.experts, info.expert_size, info.packs, info.records) == (3, 2, 128, 2, 0)
    assert info.file_bytes == 0  # no layer_03.bin


def test_duplicate_expert_is_rejected(tmp_path):
    write_json(tmp_path, 3, meta("FIXED_Q4_EXPERT_LAYER_V1", 3, 128, 2, [tiny_pack(3, 0, 128), tiny_pack(3, 0, 64)]))
    rc, _, msg = inspect_rc(tmp_path, 3)
    assert rc == abi.ERR_FORMAT and "duplicate expert 0" in msg


def test_pack_longer_than_its_slot_is_rejected(tmp_path):
    write_json(tmp_path, 3, meta("FIXED_Q4_EXPERT_LAYER_V1", 3, 128, 2, [tiny_pack(3, 1, 129)]))
    rc, _, msg = inspect_rc(tmp_path, 3)
    assert rc == abi.ERR_FORMAT and "length 129 exceeds slot size 128" in msg


def test_pbq4_v2_metadata_reads_back_with_layer_paths(tmp_path):
    # expert_metadata_reader_uses_expert_owned_paths_and_validation
    write_json(tmp_path, 5, meta("PBQ4EXPERT_LAYER_V2", 5, 256, 4, [tiny_pack(5, 2, 200)]))
    open(os.path.join(tmp_path, "layer_05.bin"), "wb").write(b"\0" * 1024)
    info = abi.pack_inspect(tmp_path, 5)
    assert info.format == b"PBQ4EXPERT_LAYER_V2"
    assert (info.experts, info.expert_size, info.packs, info.file_bytes) == (4, 256, 1, 1024)


@pytest.mark.parametrize("mutate,fragment", [
    (lambda m: m.update(format="PBQ9"), "unsupported format PBQ9"),
    (lambda m: m.update(layer=4), "describes layer 4, expected layer 3"),
    (lambda m: m.update(expert_size=0), "zero expert_size"),
    (lambda m: m.update(experts=0), "zero experts"),
    (lambda m: m["packs"].append(tiny_pack(3, 2, 16)), "describes expert 2 outside 0..2"),
    (lambda m: m["packs"][0].update(layer=9), "describes layer 9 expert 0, expected layer 3 expert 0"),
])
def test_validate_rejections(tmp_path, mutate, fragment):
    m = meta("FIXED_Q4_EXPERT_LAYER_V1", 3, 128, 2, [tiny_pack(3, 0, 128), tiny_pack(3, 1, 128)])
    mutate(m)
    write_json(tmp_path, 3, m)
    rc, _, msg = inspect_rc(tmp_path, 3)
    assert rc == abi.ERR_FORMAT, msg
    assert fragment in msg, msg


def test_missing_metadata_is_an_io_error(tmp_path):
    rc, _, msg = inspect_rc(tmp_path, 7)
    assert rc == abi.ERR_IO and "layer_07.json" in msg


@pytest.mark.parametrize("text,fragment", [
    ("", "unexpected end of input"),
    ("{", "expected string"),
    ('{"format": "FIXED_Q4_EXPERT_LAYER_V1", "layer": 3,}', "expected string"),
    ('{"format": "FIXED_Q4_EXPERT_LAYER_V1"} trailing', "trailing characters"),
    ('{"format": 7, "layer": 3, "expert_size": 1, "experts": 1, "packs": []}', "`format` is not a string"),
    ('{"format": "FIXED_Q4_EXPERT_LAYER_V1", "layer": -3, "expert_size": 1, "experts": 1, "packs": []}',
     "`layer` is not a non-negative integer"),
    ('{"format": "FIXED_Q4_EXPERT_LAYER_V1", "layer": 3.5, "expert_size": 1, "experts": 1, "packs": []}',
     "`layer` is not a non-negative integer"),
    ('{"format": "FIXED_Q4_EXPERT_LAYER_V1", "layer": 3, "experts": 1, "packs": []}', "missing field `expert_size`"),
    ('{"format": "FIXED_Q4_EXPERT_LAYER_V1", "layer": 3, "expert_size": 1, "experts": 1, "packs": [{"layer": 3}]}',
     "missing field `expert`"),
    ('{"format": "FIXED_Q4_EXPERT_LAYER_V1", "layer": 3, "expert_size": 1, "experts": 1, '
     '"packs": [{"layer": 3, "expert": 0}]}', "missing field `records`"),
    ('{"format": "FIX\\q", "layer": 3, "expert_size": 1, "experts": 1, "packs": []}', "invalid escape"),
    ('{"format": "FIXED_Q4_EXPERT_LAYER_V1", "layer": 03, "expert_size": 1, "experts": 1, "packs": []}',
     "leading zero"),
])
def test_malformed_json_is_rejected(tmp_path, text, fragment):
    write_json(tmp_path, 3, text)
    rc, _, msg = inspect_rc(tmp_path, 3)
    assert rc == abi.ERR_FORMAT, msg
    assert fragment in msg, msg


def test_serde_defaults_and_unknown_fields(tmp_path):
    """packed_bytes defaults to 0 and scale_bias_dtype to F32 (serde
    defaults, experts/mod.rs:435-436, 452-453); unknown fields, escapes,
    null source_hash and floats elsewhere are accepted."""
    rec = {"tensor": "model.layers.3.mlp.experts.0.gate_proj.weighté\\u0041", "dtype": "BF16",
           "shape": [4, 8], "source_offsets": [0, 16], "source_hash": None, "record_offset": 0,
           "packed_bytes": 16, "groups": 1, "group_size": 32, "future_field": [1.5e3, True, None, {"x": []}]}
    m = meta("FIXED_Q4_EXPERT_LAYER_V1", 3, 128, 2, [{"layer": 3, "expert": 1, "records": [rec]}])
    m["converter"] = {"version": "1.2", "ratio": 0.25}
    write_json(tmp_path, 3, json.dumps(m, ensure_ascii=True))
    info = abi.pack_inspect(tmp_path, 3)
    assert (info.packs, info.records) == (1, 1)


def test_written_pack_round_trips(tmp_path):
    """pb_amd.packs writes what pbmoe_pack_inspect reads: a fixed-Q4 layer
    with three records per expert, whole-slot entries, the .bin sized
    experts x slot bytes."""
    import numpy as np
    lay = abi.q4_layout_fixed(256, 256, 64, abi.DTYPE_F16)
    E = 3
    slots = np.arange(E * lay.expert_bytes, dtype=np.uint64).astype(np.uint8)
    packs.write_pack(str(tmp_path), 12, slots, packs.layer_metadata(12, E, lay, 256, 256))
    info = abi.pack_inspect(tmp_path, 12)
    assert info.format == b"FIXED_Q4_EXPERT_LAYER_V1"
    assert (info.layer, info.experts, info.expert_size) == (12, E, lay.expert_bytes)
    assert (info.packs, info.records, info.file_bytes) == (E, 3 * E, E * lay.expert_bytes)
