"""GPU: a resident Q4 router projection and a Q4 shared-expert gate row (the
Q4 arm of encode_resident_projection_rows, metal/projection.rs:232-259,
kernel q4_mmap_fma_matvec[_bf16_scale_bias], shaders.metal:488-660), bound
through pbmoe_bind_router_q4 / pbmoe_bind_shared_gate_q4 and checked
against the oracle (router_logits_q4 and moe_block with a Q4 gate, both over
q4_fma_matvec, math.rs:861-911).

Logits: within the summation bound of the device's factored form
s*sum(q x) + b*sum(x) against the oracle's fma form.  Routes: ids bit-exact
against the oracle's routing of the device's own logits.  Layer: the parity
bar against the oracle block on the device's routes."""
from __future__ import annotations

import ctypes as C
import sys
from dataclasses import replace

import numpy as np
import pytest

from oracle import oracle as orc
from pb_amd import abi, synth
from pb_amd.configs import C1, C2
from pb_amd.synth import MoeConfig
from tests.gpu_common import SEED, DeviceLayer, assert_layer_tolerance, max_abs_rel_l2

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
C1_BF = replace(C1, name="c1_bf16_scale_bias", sb_dtype=abi.DTYPE_BF16)
C2_SIG = replace(C2, name="c2_sigmoid_noaux", routing=abi.ROUTING_SIGMOID_NOAUX)
# the C5 row width (7168 columns: the router stage stages x in LDS, times
# the norm weight when the norm is fused, with each token's sum of squares
# reduced across the workgroup) with a small expert intermediate to keep the
# resident slots small
C5W = MoeConfig("c5_width_q4_router", hidden=7168, intermediate=256, experts=256, k=8,
                routing=abi.ROUTING_SOFTMAX_TOPK, normalization=abi.NORM_RENORMALIZE_SELECTED,
                sb_dtype=abi.DTYPE_F16)
C5W_BF = replace(C5W, name="c5_width_q4_router_bf16", sb_dtype=abi.DTYPE_BF16)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = abi.Context(0)
    yield c
    c.close()


def _kind(cfg):
    return orc.ROUTING_SIGMOID_NOAUX if cfg.routing == abi.ROUTING_SIGMOID_NOAUX else orc.ROUTING_SOFTMAX


def _bound(dl, xh):
    """2 (H + 64) u sum_c |w_ec| |x_tc| with |w| <= 15|s| + |b| per group."""
    cfg = dl.cfg
    codes, sc, bi = dl.q4_router
    s = synth._sb_to_f32(sc, cfg.sb_dtype).astype(np.float64).reshape(cfg.experts, -1)
    b = synth._sb_to_f32(bi, cfg.sb_dtype).astype(np.float64).reshape(cfg.experts, -1)
    wabs = np.repeat(15.0 * np.abs(s) + np.abs(b), cfg.group, axis=1)
    return 2 * (cfg.hidden + 64) * U * (np.abs(xh.astype(np.float64)) @ wabs.T)


@pytest.mark.parametrize("cfg,T,order", [(C2, 1, abi.ORDER_REFERENCE_SLOT), (C2, 8, abi.ORDER_CANONICAL),
                                         (C1, 4, abi.ORDER_CANONICAL), (C1_BF, 1, abi.ORDER_REFERENCE_SLOT),
                                         (C1_BF, 40, abi.ORDER_CANONICAL), (C2, 40, abi.ORDER_REFERENCE_SLOT),
                                         (C2_SIG, 1, abi.ORDER_REFERENCE_SLOT), (C2_SIG, 40, abi.ORDER_CANONICAL),
                                         (C5W, 1, abi.ORDER_REFERENCE_SLOT), (C5W, 2, abi.ORDER_CANONICAL),
                                         (C5W_BF, 1, abi.ORDER_CANONICAL), (C5W_BF, 2, abi.ORDER_REFERENCE_SLOT)])
def test_q4_router_logits_and_routes(ctx, cfg, T, order):
    """pbmoe_route with a Q4 router: T <= 16 through the decode router stage
    (rows of 7168 columns through its LDS-staged form), T = 40 through the
    many-token router kernel; f16 and bf16 scale/bias; softmax and sigmoid
    (with selection bias) routing."""
    _say(f"[test] q4 router {cfg.name} T={T} order={order}")
    dl = DeviceLayer(ctx, cfg, 40 + T, order, index=600, q4_router=True)
    xh, _ = synth.activations(SEED, 800 + T, T, cfg.hidden)
    x = ctx.to_device(xh)
    ids = ctx.array((T, cfg.k), np.uint32)
    w = ctx.array((T, cfg.k), np.float32)
    logits = ctx.array((T, cfg.experts), np.float32)
    dl.moe.route(x, ids, w, logits)
    ctx.sync()
    got = logits.download()
    ref = dl.oracle_logits(xh)
    bound = _bound(dl, xh)
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) / bound))
    assert float(np.std(ref)) > 0.1  # the seeded router spreads the logits
    ref_ids, ref_w = orc.route_rows(got, cfg.k, _kind(cfg), order, bias=dl.host.selection_bias,
                                    routed_scale=cfg.routed_scale)
    np.testing.assert_array_equal(ids.download().astype(np.int32), ref_ids)
    np.testing.assert_allclose(w.download(), ref_w, rtol=4e-6, atol=0)
    dl.moe.unbind()


@pytest.mark.parametrize("T", [1, 4])
def test_q4_router_and_gate_fused_layer(ctx, T):
    """pbmoe_moe_layer on C2 (gated shared expert) with a Q4 router and a Q4
    shared gate row: routes bit-exact against the oracle's routing of the
    oracle's logits wherever the K/K+1 gap exceeds the logit bound, the
    hidden state and next-layer norm within the bar of the oracle block with
    the Q4 gate."""
    _say(f"[test] q4 router+gate layer T={T}")
    c = ctx
    cfg = C2
    dl = DeviceLayer(c, cfg, 50 + T, abi.ORDER_REFERENCE_SLOT, index=601, q4_router=True)
    assert dl.q4_gate is not None
    xh, rh = synth.activations(SEED, 820 + T, T, cfg.hidden)
    nw = synth.uniform_f32(SEED, 96, 0, 0, 0, cfg.hidden, 0.5, 1.0)
    x, r = c.to_device(xh), c.to_device(rh)
    out = c.array((T, cfg.hidden), np.float32)
    nn = c.array((T, cfg.hidden), np.float32)
    ids = c.array((T, cfg.k), np.uint32)
    w = c.array((T, cfg.k), np.float32)
    dl.moe.forward(x, r, out, ids, w, c.to_device(nw), nn)
    c.sync()
    gi, gw = ids.download().astype(np.int32), w.download()
    ref_l = dl.oracle_logits(xh)
    ref_ids, ref_w = orc.route_rows(ref_l, cfg.k, orc.ROUTING_SOFTMAX, orc.ORDER_REFERENCE_SLOT)
    bound = _bound(dl, xh)
    for t in range(T):
        srt = np.sort(ref_l[t])[::-1]
        if srt[cfg.k - 1] - srt[cfg.k] > bound[t].max():
            np.testing.assert_array_equal(gi[t], ref_ids[t])
            np.testing.assert_allclose(gw[t], ref_w[t], rtol=1e-4)
    ref_h, ref_n = dl.oracle_block(xh, rh, gi, gw, next_norm=nw)
    mx, rel = assert_layer_tolerance(out.download(), ref_h)
    assert_layer_tolerance(nn.download(), ref_n, "next_normed")
    _say(f"[result] q4 router+gate T={T}: max_abs={mx:.3e} rel_l2={rel:.3e}")
    # the Q4 gate replaced the dense gate bound with the shared expert:
    # the output is nearer the Q4-gate block than the dense-gate block
    slots, rid, n = dl.compact_slots(gi)
    ref_dense, _ = orc.moe_block(dl.oracle_layout(), slots, n, xh, rh, rid, gw,
                                 shared_layout=dl.oracle_shared_layout(), shared_slot=dl.host.shared_slot,
                                 shared_gate_w=dl.host.shared_gate_f16, shared_gate_dtype=orc.DT_F16)
    assert mx < float(np.max(np.abs(out.download() - ref_dense)))
    dl.moe.unbind()


@pytest.mark.parametrize("cfg,T", [(C5W, 1), (C5W_BF, 2)])
def test_q4_router_fused_norm_at_c5_width(ctx, cfg, T):
    """pbmoe_moe_layer_norm with a Q4 router of 7168 columns: the router
    stage stages x times the norm weight in LDS (one token per workgroup at
    this width) and reduces each token's sum of squares there.  Routes
    equal those of pbmoe_moe_layer on the host-normalised rows wherever the
    K/K+1 logit gap exceeds the summation bound; hidden and next-normed rows
    within the bar of the oracle on rows normalised in f64."""
    _say(f"[test] q4 router fused norm {cfg.name} T={T}")
    dl = DeviceLayer(ctx, cfg, 70 + T, abi.ORDER_CANONICAL, index=604, q4_router=True)
    _, hh = synth.activations(SEED, 860 + T, T, cfg.hidden)
    rng = np.random.default_rng(100 + T)
    nw = rng.uniform(0.5, 1.5, cfg.hidden).astype(np.float32)
    nn = rng.uniform(0.5, 1.5, cfg.hidden).astype(np.float32)
    h64 = hh.astype(np.float64)
    xh = (h64 / np.sqrt(np.mean(h64 * h64, axis=1, keepdims=True) + 1e-6) * nw).astype(np.float32)
    h, nw_d, nn_d = ctx.to_device(hh), ctx.to_device(nw), ctx.to_device(nn)
    ids = ctx.array((T, cfg.k), np.uint32)
    w = ctx.array((T, cfg.k), np.float32)
    out = ctx.array((T, cfg.hidden), np.float32)
    nxt = ctx.array((T, cfg.hidden), np.float32)
    dl.moe.forward_norm(h, nw_d, out, ids, w, nn_d, nxt)
    ids_s = ctx.array((T, cfg.k), np.uint32)
    w_s = ctx.array((T, cfg.k), np.float32)
    out_s = ctx.array((T, cfg.hidden), np.float32)
    dl.moe.forward(ctx.to_device(xh), h, out_s, ids_s, w_s)
    ctx.sync()
    gi, gw = ids.download().astype(np.int32), w.download()
    ref_l = dl.oracle_logits(xh)
    bound = _bound(dl, xh)
    checked = 0
    for t in range(T):
        srt = np.sort(ref_l[t])[::-1]
        if srt[cfg.k - 1] - srt[cfg.k] > 2 * bound[t].max():
            np.testing.assert_array_equal(gi[t], ids_s.download().astype(np.int32)[t])
            np.testing.assert_array_equal(np.sort(gi[t]), np.sort(np.argsort(-ref_l[t], kind="stable")[:cfg.k]))
            checked += 1
    ref_h, ref_n = dl.oracle_block(xh, hh, gi, gw, next_norm=nn)
    if np.max(np.abs(ref_h)) > 1e3:
        # large outputs amplify the f32 rounding of the normalised rows, which
        # the device and the host norm round differently: the bar is the
        # oracle's own response to a one-ulp perturbation of every element
        pr = np.random.default_rng(1)
        xp = np.where(pr.random(xh.shape) < 0.5, np.nextafter(xh, np.inf), np.nextafter(xh, -np.inf))
        ref_p, _ = dl.oracle_block(xp.astype(np.float32), hh, gi, gw)
        sens = float(np.max(np.abs(ref_p.astype(np.float64) - ref_h)))
        mx, rel = max_abs_rel_l2(out.download(), ref_h)
        assert rel <= 2e-3 and mx <= max(1e-2, 4.0 * sens), f"max_abs={mx:.3e} rel_l2={rel:.3e} sens={sens:.3e}"
        assert max_abs_rel_l2(nxt.download(), ref_n)[1] <= 2e-3
    else:
        mx, rel = assert_layer_tolerance(out.download(), ref_h)
        assert_layer_tolerance(nxt.download(), ref_n, "next normed")
    _say(f"[result] q4 fused norm {cfg.name} T={T}: ids checked on {checked}/{T} tokens, "
         f"max_abs={mx:.3e} rel_l2={rel:.3e}")
    dl.moe.unbind()


def test_q4_gate_prefill_matches_oracle(ctx):
    """Layer-major prefill (pbmoe_moe_prefill) of 64 tokens with the Q4
    shared gate row, on routes from the Q4 many-token router."""
    _say("[test] q4 gate prefill T=64")
    cfg, T = C2, 64
    dl = DeviceLayer(ctx, cfg, 60, abi.ORDER_CANONICAL, index=602, q4_router=True)
    xh, rh = synth.activations(SEED, 840, T, cfg.hidden)
    x, r = ctx.to_device(xh), ctx.to_device(rh)
    ids = ctx.array((T, cfg.k), np.uint32)
    w = ctx.array((T, cfg.k), np.float32)
    out = ctx.array((T, cfg.hidden), np.float32)
    dl.moe.route(x, ids, w)
    dl.moe.qwen_layer_major_experts(x, r, ids, w, out)
    ctx.sync()
    gi, gw = ids.download().astype(np.int32), w.download()
    ref_h, _ = dl.oracle_block(xh, rh, gi, gw)
    mx, rel = assert_layer_tolerance(out.download(), ref_h)
    _say(f"[result] q4 gate prefill: max_abs={mx:.3e} rel_l2={rel:.3e}")
    dl.moe.unbind()


def test_q4_router_bind_errors(ctx):
    """Refusals at bind time: a scale/bias dtype other than the experts', a
    group size the kernels do not take, missing arrays, a gate before the
    shared expert is bound; a refused bind leaves the router bound before it."""
    _say("[test] q4 router bind errors")
    cfg = C2
    L = abi.lib()
    lay = abi.q4_layout_fixed(cfg.hidden, cfg.intermediate, cfg.group, cfg.sb_dtype)
    slots = ctx.array(cfg.experts * lay.expert_bytes, np.uint8)
    from pb_amd.flashmoe import layer_desc
    desc = layer_desc(cfg)
    abi.check(L.pbmoe_bind_layer(ctx.handle, 603, C.byref(desc), C.byref(lay), slots.ptr, slots.nbytes,
                                 abi.MEM_DEVICE))
    dense = ctx.to_device(np.zeros((cfg.experts, cfg.hidden), np.uint16))
    abi.check(L.pbmoe_bind_router(ctx.handle, 603, dense.ptr, abi.DTYPE_F16, None, abi.MEM_DEVICE))
    codes = ctx.array(cfg.experts * cfg.hidden // 2, np.uint8)
    sb = ctx.array(cfg.experts * cfg.hidden // 32, np.uint16)
    m = abi.Q4Matrix()
    m.codes, m.scales, m.biases = codes.ptr, sb.ptr, sb.ptr
    assert L.pbmoe_bind_router_q4(ctx.handle, 603, C.byref(m), cfg.group, abi.DTYPE_BF16, None,
                                  abi.MEM_DEVICE) == abi.ERR_UNSUPPORTED
    assert b"scale/bias" in L.pbmoe_last_error()
    assert L.pbmoe_bind_router_q4(ctx.handle, 603, C.byref(m), 16, cfg.sb_dtype, None,
                                  abi.MEM_DEVICE) == abi.ERR_UNSUPPORTED
    assert b"group" in L.pbmoe_last_error()
    bad = abi.Q4Matrix()
    bad.codes, bad.scales, bad.biases = codes.ptr, sb.ptr, None
    assert L.pbmoe_bind_router_q4(ctx.handle, 603, C.byref(bad), cfg.group, cfg.sb_dtype, None,
                                  abi.MEM_DEVICE) == abi.ERR_INVALID_ARGUMENT
    assert L.pbmoe_bind_shared_gate_q4(ctx.handle, 603, C.byref(m), cfg.group, cfg.sb_dtype,
                                       abi.MEM_DEVICE) == abi.ERR_NOT_BOUND
    # the refusals left the dense router bound: routing still runs
    x = ctx.to_device(np.ones((1, cfg.hidden), np.float32))
    ids = ctx.array((1, cfg.k), np.uint32)
    w = ctx.array((1, cfg.k), np.float32)
    abi.check(L.pbmoe_route(ctx.handle, 603, x.ptr, 1, ids.ptr, w.ptr, None))
    ctx.sync()
    np.testing.assert_array_equal(ids.download()[0], np.arange(cfg.k))  # all-zero logits: the lowest ids
    abi.check(L.pbmoe_bind_router_q4(ctx.handle, 603, C.byref(m), cfg.group, cfg.sb_dtype, None,
                                     abi.MEM_DEVICE))
    abi.check(L.pbmoe_unbind_layer(ctx.handle, 603))
