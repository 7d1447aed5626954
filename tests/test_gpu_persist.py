"""GPU: the one-launch batch-1 decode (persist_decode_kernel, selected for a
context created with PBMOE_DECODE_KERNELS=1) against the oracle and against
the default three-kernel decode, through the C ABI on the same seeded
layers."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

from oracle import oracle as orc
from pb_amd import abi, synth
from pb_amd.configs import C1, C2
from tests.gpu_common import SEED, DeviceLayer, HipGraph, assert_layer_tolerance

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _context(kernels: str | None):
    old = os.environ.get("PBMOE_DECODE_KERNELS")
    if kernels is None:
        os.environ.pop("PBMOE_DECODE_KERNELS", None)
    else:
        os.environ["PBMOE_DECODE_KERNELS"] = kernels
    try:
        return abi.Context(0)
    finally:
        if old is None:
            os.environ.pop("PBMOE_DECODE_KERNELS", None)
        else:
            os.environ["PBMOE_DECODE_KERNELS"] = old


@pytest.fixture(scope="module")
def ctx():
    c = _context("1")  # the one-launch path
    yield c
    c.close()


@pytest.fixture(scope="module")
def ctx3():
    c = _context(None)  # the default three-kernel path
    yield c
    c.close()


def _layer_call(ctx, dl, xh, rh, norm=None, next_norm=None):
    cfg = dl.cfg
    x, r = ctx.to_device(xh), ctx.to_device(rh)
    out = ctx.array((1, cfg.hidden), np.float32)
    ids = ctx.array((1, cfg.k), np.uint32)
    w = ctx.array((1, cfg.k), np.float32)
    nn = ctx.array((1, cfg.hidden), np.float32) if next_norm is not None else None
    if norm is not None:
        dl.moe.forward_norm(x, ctx.to_device(norm), out, ids, w)
    else:
        dl.moe.forward(x, r, out, ids, w, ctx.to_device(next_norm) if next_norm is not None else None, nn)
    ctx.sync()
    return ids.download().astype(np.int32), w.download(), out.download(), nn.download() if nn else None


@pytest.mark.parametrize("cfg,order,seed", [(C2, abi.ORDER_CANONICAL, 0), (C2, abi.ORDER_REFERENCE_SLOT, 1),
                                            (C1, abi.ORDER_CANONICAL, 2), (C1, abi.ORDER_REFERENCE_SLOT, 3)])
def test_one_launch_layer_matches_oracle_and_three_kernels(ctx, ctx3, cfg, order, seed):
    """Routes on the device's own logits bit-exact against the oracle's
    routing, the hidden state and the next-layer norm within the bar, and
    the same routes and outputs within the bar from the three-kernel path."""
    _say(f"[test] one-launch {cfg.name} order={order}")
    d1 = DeviceLayer(ctx, cfg, 5 + seed, order, index=500)
    d3 = DeviceLayer(ctx3, cfg, 5 + seed, order, index=500)
    xh, rh = synth.activations(SEED, 700 + seed, 1, cfg.hidden)
    nw = synth.uniform_f32(SEED, 98, 0, 0, 0, cfg.hidden, 0.5, 1.0)
    ids1, w1, h1, n1 = _layer_call(ctx, d1, xh, rh, next_norm=nw)
    ids3, w3, h3, n3 = _layer_call(ctx3, d3, xh, rh, next_norm=nw)
    # routing of the one-launch path on its own logits (the logits are the
    # oracle's within the summation bound; see test_router_logits_within_summation_bound)
    ref_l = d1.oracle_logits(xh)
    ref_ids, ref_w = orc.route_rows(ref_l, cfg.k, orc.ROUTING_SOFTMAX, order)
    wr = synth.f16_to_f32(d1.host.router_f16)
    bound = 2 * (cfg.hidden + 64) * 2.0**-24 * (np.abs(xh) @ np.abs(wr).T).max()
    srt = np.sort(ref_l[0])[::-1]
    if srt[cfg.k - 1] - srt[cfg.k] > bound:
        np.testing.assert_array_equal(ids1, ref_ids)
        np.testing.assert_array_equal(ids3, ref_ids)
        np.testing.assert_allclose(w1, ref_w, rtol=1e-4)
    ref_h, ref_n = d1.oracle_block(xh, rh, ids1, w1, next_norm=nw)
    mx, rel = assert_layer_tolerance(h1, ref_h)
    assert_layer_tolerance(n1, ref_n, "next_normed")
    _say(f"[result] one-launch {cfg.name}: max_abs={mx:.3e} rel_l2={rel:.3e}")
    if np.array_equal(ids1, ids3):
        assert_layer_tolerance(h1, h3, "one-launch vs three-kernel")
        assert_layer_tolerance(n1, n3, "one-launch vs three-kernel next_normed")
    d1.moe.unbind()
    d3.moe.unbind()


@pytest.mark.parametrize("cfg", [C1, C2])
def test_one_launch_fused_input_norm(ctx, cfg):
    """pbmoe_moe_layer_norm at one token (the stack's MoE call): the input
    RMSNorm folded into the router and gate/up rows of the one launch."""
    _say(f"[test] one-launch fused norm {cfg.name}")
    dl = DeviceLayer(ctx, cfg, 9, index=501)
    hh, _ = synth.activations(SEED, 710, 1, cfg.hidden)
    nw = synth.uniform_f32(SEED, 97, 0, 0, 0, cfg.hidden, 0.5, 1.5)
    ids, w, h, _ = _layer_call(ctx, dl, hh, hh, norm=nw)
    xn = (hh.astype(np.float64) / np.sqrt(np.mean(hh.astype(np.float64) ** 2) + 1e-6) * nw).astype(np.float32)
    ref_h, _ = dl.oracle_block(xn, hh, ids, w)
    assert_layer_tolerance(h, ref_h)
    dl.moe.unbind()


def test_one_launch_expert_mode_is_bitwise_full_mode(ctx):
    """Routes given (pbmoe_moe_decode) with the routes the full layer chose:
    the same kernel arithmetic, so the hidden state is bitwise equal."""
    _say("[test] one-launch expert mode")
    cfg = C2
    dl = DeviceLayer(ctx, cfg, 11, index=502)
    xh, rh = synth.activations(SEED, 720, 1, cfg.hidden)
    x, r = ctx.to_device(xh), ctx.to_device(rh)
    ids = ctx.array((1, cfg.k), np.uint32)
    w = ctx.array((1, cfg.k), np.float32)
    a = ctx.array((1, cfg.hidden), np.float32)
    b = ctx.array((1, cfg.hidden), np.float32)
    dl.moe.forward(x, r, a, ids, w)
    dl.moe.submit_scheduled_expert_command(x, r, ids, w, b)
    ctx.sync()
    np.testing.assert_array_equal(a.download().view(np.uint32), b.download().view(np.uint32))
    dl.moe.unbind()


def test_one_launch_repeated_calls_across_layers_are_deterministic(ctx):
    """Many calls in a row over three layers (the call tag advances every
    call): every repetition of a layer returns the same bits."""
    _say("[test] one-launch repeated calls")
    cfg = C2
    dls = [DeviceLayer(ctx, cfg, 20 + i, index=510 + i) for i in range(3)]
    xh, rh = synth.activations(SEED, 730, 1, cfg.hidden)
    first = [_layer_call(ctx, d, xh, rh)[2] for d in dls]
    assert not np.array_equal(first[0], first[1])
    for rep in range(20):
        for i, d in enumerate(dls):
            got = _layer_call(ctx, d, xh, rh)[2]
            np.testing.assert_array_equal(got.view(np.uint32), first[i].view(np.uint32), err_msg=f"rep {rep}")
    for d in dls:
        d.moe.unbind()


def test_one_launch_graph_replays_match_eager(ctx):
    """The one-launch layer captured in a hipGraph and replayed with other
    eager calls in between: the call tag lives in device memory and advances
    on every replay, so each replay equals the eager result bit for bit."""
    _say("[test] one-launch graph replay")
    cfg = C2
    dl = DeviceLayer(ctx, cfg, 30, index=520)
    other = DeviceLayer(ctx, cfg, 31, index=521)
    xh, rh = synth.activations(SEED, 740, 1, cfg.hidden)
    x, r = ctx.to_device(xh), ctx.to_device(rh)
    ids = ctx.array((1, cfg.k), np.uint32)
    w = ctx.array((1, cfg.k), np.float32)
    out = ctx.array((1, cfg.hidden), np.float32)
    dl.moe.forward(x, r, out, ids, w)
    ctx.sync()
    ref = (ids.download(), w.download(), out.download())
    graph = HipGraph(ctx.stream(), lambda: dl.moe.forward(x, r, out, ids, w))
    junk = ctx.array((1, cfg.hidden), np.float32)
    for rep in range(5):
        out.upload(np.full((1, cfg.hidden), np.nan, np.float32))
        for _ in range(rep):  # a varying number of eager calls between replays
            other.moe.forward(r, x, junk)
        ctx.sync()
        graph.launch()
        ctx.sync()
        np.testing.assert_array_equal(ids.download(), ref[0], err_msg=f"replay {rep}")
        np.testing.assert_array_equal(w.download().view(np.uint32), ref[1].view(np.uint32))
        np.testing.assert_array_equal(out.download().view(np.uint32), ref[2].view(np.uint32))
    graph.close()
    dl.moe.unbind()
    other.moe.unbind()
