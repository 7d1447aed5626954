"""GPU: binding lifecycle of a layer index through the C ABI.  Rebinding an
index starts from an empty binding (router, selection bias and shared
expert must be bound again), and shapes the decode kernels are not built
for are refused at bind time."""
from __future__ import annotations

import ctypes as C
import sys
from dataclasses import replace

import numpy as np
import pytest

from pb_amd import abi, synth
from pb_amd.configs import C1, C2
from pb_amd.flashmoe import MoeLayer, layer_desc
from tests.gpu_common import SEED, DeviceLayer

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = abi.Context(0)
    yield c
    c.close()


def _decode(ctx, moe: MoeLayer, xh, rh):
    T, H = xh.shape
    x, r = ctx.to_device(xh), ctx.to_device(rh)
    out = ctx.array((T, H), np.float32)
    ids = ctx.array((T, moe.cfg.k), np.uint32)
    w = ctx.array((T, moe.cfg.k), np.float32)
    moe.forward(x, r, out, ids, w)
    ctx.sync()
    return out.download(), ids.download()


def test_rebind_resets_router_and_shared(ctx):
    """Index 7 first holds a C1 layer; rebinding it with the larger C2
    descriptor (4x the experts, a gated shared expert) leaves no router or
    shared expert behind: routing and the layer report NOT_BOUND until both
    are bound again, then the layer gives bitwise the result of a fresh
    binding of the same weights."""
    _say("[test] rebind resets router and shared expert")
    small = DeviceLayer(ctx, C1, 3, index=7)
    xh, rh = synth.activations(SEED, 9, 1, C2.hidden)
    _decode(ctx, small.moe, xh[:, :C1.hidden], rh[:, :C1.hidden])
    big = DeviceLayer(ctx, C2, 4, index=8)  # reference result from a fresh index
    ref, ref_ids = _decode(ctx, big.moe, xh, rh)

    desc = layer_desc(C2)
    L = abi.lib()
    abi.check(L.pbmoe_bind_layer(ctx.handle, 7, C.byref(desc), C.byref(big.layout), big.slots.ptr,
                                 big.slots.nbytes, abi.MEM_DEVICE))
    x = ctx.to_device(xh)
    ids = ctx.array((1, C2.k), np.uint32)
    w = ctx.array((1, C2.k), np.float32)
    assert L.pbmoe_route(ctx.handle, 7, x.ptr, 1, ids.ptr, w.ptr, None) == abi.ERR_NOT_BOUND
    assert b"router" in L.pbmoe_last_error()
    abi.check(L.pbmoe_bind_router(ctx.handle, 7, big.router.ptr, abi.DTYPE_F16, None, abi.MEM_DEVICE))
    out = ctx.array((1, C2.hidden), np.float32)
    r = ctx.to_device(rh)
    rc = L.pbmoe_moe_layer(ctx.handle, 7, x.ptr, r.ptr, 1, ids.ptr, w.ptr, None, out.ptr, None)
    assert rc == abi.ERR_NOT_BOUND and b"shared expert" in L.pbmoe_last_error()
    abi.check(L.pbmoe_bind_shared(ctx.handle, 7, C.byref(big.host.shared_layout), big.shared.ptr, big.gate.ptr,
                                  abi.DTYPE_F16, abi.MEM_DEVICE))
    rebound = MoeLayer(ctx, 7, C2, big.layout)
    got, got_ids = _decode(ctx, rebound, xh, rh)
    np.testing.assert_array_equal(got_ids, ref_ids)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    abi.check(L.pbmoe_unbind_layer(ctx.handle, 7))
    assert L.pbmoe_unbind_layer(ctx.handle, 7) == abi.ERR_NOT_BOUND
    big.moe.unbind()


@pytest.mark.parametrize("inter", [1280, 1792, 2304])
def test_unsupported_intermediate_rejected_at_bind(ctx, inter):
    """Intermediate sizes without a decode down-kernel instance are refused
    by pbmoe_bind_layer with UNSUPPORTED, before anything is launched."""
    _say(f"[test] intermediate {inter} rejected")
    cfg = replace(C1, name=f"c1_i{inter}", intermediate=inter, experts=2, k=2)
    desc = layer_desc(cfg)
    lay = abi.q4_layout_fixed(cfg.hidden, inter, cfg.group, cfg.sb_dtype)
    slots = ctx.array(2 * lay.expert_bytes, np.uint8)
    rc = abi.lib().pbmoe_bind_layer(ctx.handle, 60, C.byref(desc), C.byref(lay), slots.ptr, slots.nbytes,
                                    abi.MEM_DEVICE)
    assert rc == abi.ERR_UNSUPPORTED
    assert b"intermediate" in abi.lib().pbmoe_last_error()
    assert abi.lib().pbmoe_unbind_layer(ctx.handle, 60) == abi.ERR_NOT_BOUND


def test_stream_read_xor_of_buffer(ctx):
    """pbmoe_stream_read (the traffic-counter calibration launch) reads every
    16-byte chunk: its XOR of all 32-bit words equals the host's; a size that
    is not a multiple of 16 is refused."""
    _say("[test] stream read")
    rng = np.random.default_rng(3)
    h = rng.integers(0, 2**32, (1 << 20) + 4 * 37, dtype=np.uint32)
    d = ctx.to_device(h)
    out = ctx.array(1, np.uint32)
    L = abi.lib()
    abi.check(L.pbmoe_stream_read(ctx.handle, d.ptr, h.nbytes, out.ptr))
    ctx.sync()
    assert int(out.download()[0]) == int(np.bitwise_xor.reduce(h))
    assert L.pbmoe_stream_read(ctx.handle, d.ptr, h.nbytes - 4, out.ptr) == abi.ERR_ALIGNMENT
