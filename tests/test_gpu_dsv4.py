"""GPU parity of the DeepSeek-V4 router (PBMOE_ROUTING_SQRT_SOFTPLUS):
deepseek_v4_router_probabilities + deepseek_v4_select_routes
(deepseek.rs:1300-1394) with batch_route_rows' floor renormalisation x 1.5
(metal/deepseek_execution.rs:3547-3583), against the oracle on the same
device logits: bit-exact ids, weights within 4 ulp; then whole decode
layers routed this way against the fp32 oracle."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

from oracle import oracle as orc
from pb_amd import abi, synth
from pb_amd.flashmoe import MoeLayer
from pb_amd.synth import MoeConfig
from tests.gpu_common import SEED, DeviceLayer, assert_layer_tolerance

pytestmark = pytest.mark.gpu

DSV4 = MoeConfig("t_dsv4_router", hidden=1024, intermediate=512, experts=256, k=6,
                 routing=abi.ROUTING_SQRT_SOFTPLUS, normalization=abi.NORM_DEEPSEEK_FLOOR, routed_scale=1.5,
                 shared_intermediate=512, shared_gated=False)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = abi.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def dl(ctx):
    return DeviceLayer(ctx, DSV4, 5, index=400)


def _oracle_routes(l, bias):
    return orc.route_rows(l, DSV4.k, orc.ROUTING_SQRT_SOFTPLUS, orc.ORDER_CANONICAL, bias=bias,
                          policy=orc.NORM_DEEPSEEK_FLOOR, routed_scale=DSV4.routed_scale)


def _route_logits(ctx, moe, l):
    T = l.shape[0]
    ids = ctx.array((T, DSV4.k), np.uint32)
    w = ctx.array((T, DSV4.k), np.float32)
    moe.route_logits(ctx.to_device(l), ids, w)
    ctx.sync()
    return ids.download().astype(np.int32), w.download()


@pytest.mark.parametrize("T", [1, 3, 8, 40])
def test_routes_bit_exact_on_device_logits(ctx, dl, T):
    """T = 1, 3: one token per workgroup; 8: one per wave; 40: the
    many-token routing kernel."""
    _say(f"[test] dsv4 routes T={T}")
    rng = np.random.default_rng(T)
    l = (rng.standard_normal((T, DSV4.experts)) * 3).astype(np.float32)
    l[0, :8] = [25.0, -25.0, 20.0, -20.0, 19.5, 21.0, -30.0, 0.0]  # every softplus branch
    ids, w = _route_logits(ctx, dl.moe, l)
    ref_ids, ref_w = _oracle_routes(l, dl.host.selection_bias)
    np.testing.assert_array_equal(ids, ref_ids)
    np.testing.assert_allclose(w, ref_w, rtol=4.8e-7 * 4, atol=0)


def test_routes_without_bias_and_ties(ctx, dl):
    _say("[test] dsv4 no bias, ties")
    m = MoeLayer(ctx, 401, DSV4, dl.layout).bind_device(dl.slots, dl.router, None, dl.host.shared_layout,
                                                        dl.shared, dl.gate)
    T, E = 4, DSV4.experts
    l = np.zeros((T, E), np.float32)
    l[1, [200, 7, 100]] = 1.0
    l[2] = (np.random.default_rng(2).standard_normal(E) * 2).astype(np.float32)
    l[3, :] = -60.0  # every probability ~1e-13: the floor decides
    ids, w = _route_logits(ctx, m, l)
    ref_ids, ref_w = _oracle_routes(l, None)
    np.testing.assert_array_equal(ids, ref_ids)
    assert list(ids[0]) == [0, 1, 2, 3, 4, 5] and list(ids[1][:4]) == [7, 100, 200, 0]
    np.testing.assert_allclose(w, ref_w, rtol=2e-6, atol=0)
    m.unbind()


def test_slot_order_is_rejected(ctx, dl):
    m = MoeLayer(ctx, 402, DSV4, dl.layout, abi.ORDER_REFERENCE_SLOT)
    rc = abi.lib().pbmoe_bind_layer(ctx.handle, 402, C.byref(m.desc), C.byref(dl.layout), dl.slots.ptr,
                                    dl.slots.nbytes, abi.MEM_DEVICE)
    assert rc == abi.ERR_UNSUPPORTED


@pytest.mark.parametrize("T", [1, 4])
def test_decode_layer_matches_oracle(ctx, dl, T):
    """pbmoe_moe_layer: router projection, V4 routing, experts, shared
    expert (ungated: sigma(80) = 1) and combine in one call."""
    _say(f"[test] dsv4 decode layer T={T}")
    xh, rh = synth.activations(SEED, 600 + T, T, DSV4.hidden)
    x, res = ctx.to_device(xh), ctx.to_device(rh)
    ids = ctx.array((T, DSV4.k), np.uint32)
    w = ctx.array((T, DSV4.k), np.float32)
    out = ctx.array((T, DSV4.hidden), np.float32)
    logits = ctx.array((T, DSV4.experts), np.float32)
    dl.moe.route(x, ids, w, logits)
    ctx.sync()
    ref_ids, ref_w = _oracle_routes(logits.download(), dl.host.selection_bias)
    np.testing.assert_array_equal(ids.download().astype(np.int32), ref_ids)
    np.testing.assert_allclose(w.download(), ref_w, rtol=2e-6, atol=0)
    ids2 = ctx.array((T, DSV4.k), np.uint32)
    w2 = ctx.array((T, DSV4.k), np.float32)
    dl.moe.forward(x, res, out, ids2, w2)
    ctx.sync()
    np.testing.assert_array_equal(ids2.download(), ids.download())
    ref_h, _ = dl.oracle_block(xh, rh, ids2.download().astype(np.int32), w2.download())
    mx, rel = assert_layer_tolerance(out.download(), ref_h)
    _say(f"[result] dsv4 T={T}: max_abs={mx:.3e} rel_l2={rel:.3e}")
