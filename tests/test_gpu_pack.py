"""GPU: layers bound from on-disk expert packs (pbmoe_bind_layer_file).

A pack written in the reference's fixed-Q4 format (layer_NN.bin +
layer_NN.json, experts/mod.rs:283-454, 2478-2484) is streamed into HBM
byte for byte, and a layer bound from it routes and combines exactly like
the same slots bound from memory.  The store-level checks of
ExpertSlotStore::resolve_execution_descriptor_from (experts/store.rs:
481-565) reject mismatched packs before anything is allocated."""
from __future__ import annotations

import ctypes as C
import json
import os
import sys
import time

import numpy as np
import pytest

from pb_amd import abi, packs, synth
from pb_amd.configs import C2
from pb_amd.flashmoe import MoeLayer
from pb_amd.synth import MoeConfig
from tests.gpu_common import SEED, DeviceLayer

pytestmark = pytest.mark.gpu

T_SHARED = MoeConfig("t_pack_shared_bf16", hidden=512, intermediate=256, experts=16, k=4,
                     shared_intermediate=256, shared_gated=True, sb_dtype=abi.DTYPE_BF16)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = abi.Context(0)
    yield c
    c.close()


def _host_slots(cfg, layer, layout):
    return synth.q4_experts(SEED, synth.T_EXPERT, layer, 0, cfg.experts, cfg.hidden, cfg.intermediate, cfg.group,
                            cfg.sb_dtype, layout.offsets, int(layout.expert_bytes))


@pytest.mark.parametrize("cfg", [T_SHARED, C2], ids=["t_shared_bf16", "c2"])
def test_file_bound_layer_matches_memory_bound(ctx, cfg, tmp_path):
    _say(f"[test] pack bind {cfg.name}")
    layer = 7
    dl = DeviceLayer(ctx, cfg, layer, index=200)
    host = _host_slots(cfg, layer, dl.layout)
    packs.write_pack(str(tmp_path), layer, host,
                     packs.layer_metadata(layer, cfg.experts, dl.layout, cfg.hidden, cfg.intermediate))
    t0 = time.perf_counter()
    fl = MoeLayer(ctx, 201, cfg, dl.layout).bind_file(str(tmp_path), layer, dl.router, dl.bias, dl.host.shared_layout,
                                                      dl.shared, dl.gate)
    dt = time.perf_counter() - t0
    _say(f"[result] {cfg.name}: {host.nbytes / 1e6:.0f} MB bound from file in {dt * 1e3:.1f} ms "
         f"({host.nbytes / dt / 1e9:.2f} GB/s, page cache -> HBM)")
    ptr, nbytes = fl.slots()
    assert nbytes == host.nbytes
    got = np.empty(nbytes, np.uint8)
    abi.check(abi.lib().pbmoe_download(ctx.handle, got.ctypes.data, C.c_void_p(ptr), nbytes))
    assert np.array_equal(got, host)  # byte-exact residency
    T = 4
    xh, rh = synth.activations(SEED, 300, T, cfg.hidden)
    x, r = ctx.to_device(xh), ctx.to_device(rh)
    outs = []
    for m in (dl.moe, fl):
        ids = ctx.array((T, cfg.k), np.uint32)
        w = ctx.array((T, cfg.k), np.float32)
        out = ctx.array((T, cfg.hidden), np.float32)
        m.forward(x, r, out, ids, w)
        ctx.sync()
        outs.append((ids.download(), w.download(), out.download()))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))
    np.testing.assert_array_equal(outs[0][2].view(np.uint32), outs[1][2].view(np.uint32))
    fl.unbind()
    dl.moe.unbind()


def _bind_rc(ctx, cfg, layout, root, file_layer, index=210):
    m = MoeLayer(ctx, index, cfg, layout)
    rc = abi.lib().pbmoe_bind_layer_file(ctx.handle, index, C.byref(m.desc), C.byref(layout), str(root).encode(),
                                        file_layer)
    return rc, abi.lib().pbmoe_last_error().decode()


def _small_pack(root, cfg, layout, layer=3, **meta_overrides):
    host = np.random.default_rng(1).integers(0, 256, cfg.experts * int(layout.expert_bytes), dtype=np.uint8)
    meta = packs.layer_metadata(layer, cfg.experts, layout, cfg.hidden, cfg.intermediate)
    meta.update(meta_overrides)
    packs.write_pack(str(root), layer, host, meta)
    return meta


def _rewrite_json(root, layer, meta):
    with open(os.path.join(root, f"layer_{layer:02d}.json"), "w") as f:
        json.dump(meta, f)


def test_file_bind_rejections(ctx, tmp_path):
    cfg = T_SHARED
    lay = abi.q4_layout_fixed(cfg.hidden, cfg.intermediate, cfg.group, cfg.sb_dtype)
    meta = _small_pack(tmp_path, cfg, lay)
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == 0, msg
    abi.check(abi.lib().pbmoe_unbind_layer(ctx.handle, 210))

    # PBQ4 formats are import compatibility only (experts/store.rs:509-515)
    _rewrite_json(tmp_path, 3, dict(meta, format="PBQ4EXPERT_LAYER_V2"))
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == abi.ERR_UNSUPPORTED and "import compatibility only" in msg
    # slot size (experts/store.rs:529-535)
    other = abi.q4_layout_fixed(cfg.hidden, cfg.intermediate, 32, cfg.sb_dtype)
    _rewrite_json(tmp_path, 3, meta)
    rc, msg = _bind_rc(ctx, cfg, other, tmp_path, 3)
    assert rc == abi.ERR_SHAPE and "has slot size" in msg
    # expert count and entries (experts/store.rs:536-542)
    _rewrite_json(tmp_path, 3, dict(meta, packs=meta["packs"][:-1]))
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == abi.ERR_SHAPE and "records, expected" in msg
    # whole-slot entries (experts/store.rs:543-556)
    short = json.loads(json.dumps(meta))
    short["packs"][2]["packed_bytes"] = int(lay.expert_bytes) - 16
    _rewrite_json(tmp_path, 3, short)
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == abi.ERR_FORMAT and "expected whole-slot payload" in msg
    # records that do not describe the layout
    bad = json.loads(json.dumps(meta))
    bad["packs"][1]["records"][2]["record_offset"] += 16
    _rewrite_json(tmp_path, 3, bad)
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == abi.ERR_FORMAT and "down_proj.weight at offset" in msg
    bad = json.loads(json.dumps(meta))
    bad["packs"][0]["records"][0]["scale_bias_dtype"] = "F16"  # the layout is BF16
    _rewrite_json(tmp_path, 3, bad)
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == abi.ERR_DTYPE
    bad = json.loads(json.dumps(meta))
    bad["packs"][0]["records"][1]["shape"] = [cfg.hidden, cfg.intermediate]
    _rewrite_json(tmp_path, 3, bad)
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == abi.ERR_FORMAT and "shape does not match" in msg
    # file size (experts/store.rs:557-565)
    _rewrite_json(tmp_path, 3, meta)
    with open(os.path.join(tmp_path, "layer_03.bin"), "ab") as f:
        f.write(b"\0" * 16)
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == abi.ERR_SHAPE and "has file size" in msg
    os.remove(os.path.join(tmp_path, "layer_03.bin"))
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 3)
    assert rc == abi.ERR_IO
    # metadata of another layer than the file name says
    _small_pack(tmp_path, cfg, lay, layer=4)
    meta4 = packs.layer_metadata(5, cfg.experts, lay, cfg.hidden, cfg.intermediate)
    _rewrite_json(tmp_path, 4, meta4)
    rc, msg = _bind_rc(ctx, cfg, lay, tmp_path, 4)
    assert rc == abi.ERR_FORMAT and "describes layer 5, expected layer 4" in msg
    # nothing stayed bound by the failures
    assert abi.lib().pbmoe_unbind_layer(ctx.handle, 210) == abi.ERR_NOT_BOUND
