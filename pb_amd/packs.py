"""Writer of on-disk expert packs in the reference's fixed-Q4 format:
root/layer_NN.bin (the experts' fixed slots back to back) and
root/layer_NN.json (ExpertLayerPackMetadata as serde_json writes it, field
order of the structs in experts/mod.rs:283-290, 431-454; one record per
projection as copy_pbq4_record_to_fixed_q4_component writes them,
experts/slots.rs:1100-1111).  Used to produce packs for pbmoe_bind_layer_file
from seeded or converted slots."""
from __future__ import annotations

import json
import os

import numpy as np

from . import abi

FORMAT_FIXED_Q4 = "FIXED_Q4_EXPERT_LAYER_V1"


def projection_records(layer: int, expert: int, layout, hidden: int, intermediate: int,
                       source_dtype: str = "BF16") -> list[dict]:
    """The three per-tensor records of one fixed-Q4 slot."""
    sb = "BF16" if layout.scale_bias_dtype == abi.DTYPE_BF16 else "F16"
    out = []
    for p, (name, rows, cols) in enumerate((("gate_proj.weight", intermediate, hidden),
                                            ("up_proj.weight", intermediate, hidden),
                                            ("down_proj.weight", hidden, intermediate))):
        w, s = layout.components[3 * p], layout.components[3 * p + 1]
        out.append({
            "tensor": f"model.layers.{layer}.mlp.experts.{expert}.{name}",
            "dtype": source_dtype,
            "shape": [rows, cols],
            "source_offsets": [0, int(w.bytes)],
            "record_offset": int(w.offset),
            "packed_bytes": int(w.bytes),
            "groups": int(s.bytes) // 2,
            "group_size": int(layout.group_size),
            "scale_bias_dtype": sb,
        })
    return out


def layer_metadata(layer: int, experts: int, layout, hidden: int, intermediate: int,
                   records: bool = True) -> dict:
    size = int(layout.expert_bytes)
    return {
        "format": FORMAT_FIXED_Q4,
        "layer": layer,
        "expert_size": size,
        "experts": experts,
        "packs": [{"layer": layer, "expert": e, "packed_bytes": size,
                   "records": projection_records(layer, e, layout, hidden, intermediate) if records else []}
                  for e in range(experts)],
    }


def write_pack(root: str, layer: int, slots: np.ndarray, metadata: dict) -> tuple[str, str]:
    """Write layer_NN.bin (slots as given) and layer_NN.json; returns the paths."""
    os.makedirs(root, exist_ok=True)
    bin_path = os.path.join(root, f"layer_{layer:02d}.bin")
    json_path = os.path.join(root, f"layer_{layer:02d}.json")
    np.ascontiguousarray(slots, dtype=np.uint8).tofile(bin_path)
    with open(json_path, "w") as f:
        json.dump(metadata, f, indent=2)
    return bin_path, json_path
