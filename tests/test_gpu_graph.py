"""GPU: the decode paths replayed from hipGraphs, as the benchmark times
them.  Each graph is replayed several times with the program's own eager
work and synchronisations in between, the output buffers poisoned before
every replay, and every replay is compared bit for bit with the eager
result (no memset nodes, no captured allocation, no state that a replay
would leave behind)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from pb_amd import abi, synth
from pb_amd.configs import C1, C2, C4_ATTN
from pb_amd.flashmoe import AttentionLayer
from tests.gpu_common import SEED, DeviceLayer, HipGraph

pytestmark = pytest.mark.gpu

NAN = np.float32(np.nan)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = abi.Context(0)
    yield c
    c.close()


def test_decode_layer_graph_replays_match_eager(ctx):
    _say("[test] graph replay: C2 decode layer")
    cfg = C2
    dl = DeviceLayer(ctx, cfg, 3, index=300)
    other = DeviceLayer(ctx, cfg, 4, index=301)
    xh, rh = synth.activations(SEED, 500, 1, cfg.hidden)
    x, r = ctx.to_device(xh), ctx.to_device(rh)
    ids = ctx.array((1, cfg.k), np.uint32)
    w = ctx.array((1, cfg.k), np.float32)
    out = ctx.array((1, cfg.hidden), np.float32)
    dl.moe.forward(x, r, out, ids, w)  # eager; sizes the scratch before capture
    ctx.sync()
    ref = (ids.download(), w.download(), out.download())
    graph = HipGraph(ctx.stream(), lambda: dl.moe.forward(x, r, out, ids, w))
    junk = ctx.array((1, cfg.hidden), np.float32)
    for rep in range(5):
        out.upload(np.full((1, cfg.hidden), NAN, np.float32))
        ids.upload(np.full((1, cfg.k), 0xFFFFFFFF, np.uint32))
        other.moe.forward(r, x, junk)  # eager work on the same scratch between replays
        ctx.sync()
        graph.launch()
        ctx.sync()
        np.testing.assert_array_equal(ids.download(), ref[0], err_msg=f"replay {rep}")
        np.testing.assert_array_equal(w.download().view(np.uint32), ref[1].view(np.uint32))
        np.testing.assert_array_equal(out.download().view(np.uint32), ref[2].view(np.uint32))
    graph.close()
    dl.moe.unbind()
    other.moe.unbind()


def test_fused_stack_graph_replays_match_eager(ctx):
    """Two C4 decoder layers with both RMSNorms fused (the stack benchmark's
    token): attention at position 130 (three chunks; the replay rewrites
    the same cache row with the same values) and the C1 MoE layer."""
    _say("[test] graph replay: fused C4 decoder layers")
    acfg, mcfg, pos = C4_ATTN, C1, 130
    H = acfg.hidden
    layers = []
    for l in range(2):
        att = AttentionLayer(ctx, 310 + l, acfg).bind_synth(SEED, 70 + l)
        moe = DeviceLayer(ctx, mcfg, 70 + l, abi.ORDER_REFERENCE_SLOT, index=310 + l, centred=True)
        layers.append((att, moe))
    rng = np.random.default_rng(9)
    for att, _ in layers:
        kp, vp = att.kv_cache()
        keys = rng.standard_normal((pos, acfg.kv_width)).astype(np.float16)
        vals = rng.standard_normal((pos, acfg.kv_width)).astype(np.float16)
        abi.check(abi.lib().pbmoe_upload(ctx.handle, kp, keys.ctypes.data, keys.nbytes))
        abi.check(abi.lib().pbmoe_upload(ctx.handle, vp, vals.ctypes.data, vals.nbytes))
    h0 = synth.activations(SEED, 501, 1, H)[1]
    h_a, h_b, mid = ctx.to_device(h0), ctx.array((1, H), np.float32), ctx.array((1, H), np.float32)
    ids = ctx.array((1, mcfg.k), np.uint32)
    w = ctx.array((1, mcfg.k), np.float32)

    def token():
        bufs = (h_a, h_b)
        for l, (att, moe) in enumerate(layers):
            h, hn = bufs[l % 2], bufs[(l + 1) % 2]
            att.decode(h, h, pos, mid, input_norm=att.input_norm)
            moe.moe.forward_norm(mid, att.post_norm, hn, ids, w)

    token()
    ctx.sync()
    ref = h_a.download()  # two layers: the result is back in h_a
    mid_ref = mid.download()
    graph = HipGraph(ctx.stream(), token)
    for rep in range(4):
        h_a.upload(h0)
        h_b.upload(np.full((1, H), NAN, np.float32))
        mid.upload(np.full((1, H), NAN, np.float32))
        layers[1][1].moe.forward(h_a, h_a, h_b)  # unrelated eager MoE call between replays
        h_b.upload(np.full((1, H), NAN, np.float32))
        ctx.sync()
        graph.launch()
        ctx.sync()
        np.testing.assert_array_equal(mid.download().view(np.uint32), mid_ref.view(np.uint32),
                                      err_msg=f"replay {rep}")
        np.testing.assert_array_equal(h_a.download().view(np.uint32), ref.view(np.uint32),
                                      err_msg=f"replay {rep}")
    graph.close()
    for att, moe in layers:
        abi.check(abi.lib().pbmoe_unbind_attention(ctx.handle, att.index))
        moe.moe.unbind()
