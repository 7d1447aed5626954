"""GPU: the allocation-free layer entry point (pbmoe_moe_layer_noalloc)
against pbmoe_moe_layer on the same bound layer and inputs: routes and
hidden state bitwise equal, on two calls in a row (the second with fewer
tokens, so stale scratch from the first call would show), with and without
caller-provided route buffers and the next-layer norm."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from pb_amd import abi, synth
from pb_amd.configs import C1, C2
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


def _run(ctx, fn, layer, cfg, xh, rh, with_routes, next_norm):
    T, H = xh.shape
    x, r = ctx.to_device(xh), ctx.to_device(rh)
    out = ctx.array((T, H), np.float32)
    ids = ctx.array((T, cfg.k), np.uint32) if with_routes else None
    w = ctx.array((T, cfg.k), np.float32) if with_routes else None
    nn = ctx.array((T, H), np.float32) if next_norm is not None else None
    abi.check(fn(ctx.handle, layer, x.ptr, r.ptr, T, ids.ptr if ids else None, w.ptr if w else None,
                 next_norm.ptr if next_norm is not None else None, out.ptr, nn.ptr if nn else None))
    ctx.sync()
    return (out.download(), ids.download() if ids else None, w.download() if w else None,
            nn.download() if nn else None)


@pytest.mark.parametrize("cfg,tokens", [(C2, (8, 1)), (C1, (16, 3)), (C2, (1, 1))])
def test_noalloc_layer_matches_allocating_layer(ctx, cfg, tokens):
    _say(f"[test] noalloc {cfg.name} tokens={tokens}")
    dl = DeviceLayer(ctx, cfg, 2, index=40)
    L = abi.lib()
    norm_w = ctx.to_device(synth.activations(SEED, 77, 1, cfg.hidden)[0].ravel())
    for call, T in enumerate(tokens):
        xh, rh = synth.activations(SEED, 60 + call, T, cfg.hidden)
        for with_routes in (True, False):
            for nn in (None, norm_w):
                ref = _run(ctx, L.pbmoe_moe_layer, 40, cfg, xh, rh, with_routes, nn)
                got = _run(ctx, L.pbmoe_moe_layer_noalloc, 40, cfg, xh, rh, with_routes, nn)
                np.testing.assert_array_equal(got[0].view(np.uint32), ref[0].view(np.uint32))
                for g, rf in zip(got[1:], ref[1:]):
                    if rf is not None:
                        np.testing.assert_array_equal(g.view(np.uint32), rf.view(np.uint32))
        _say(f"[result] call {call}: T={T} bitwise equal")
    dl.moe.unbind()


def test_noalloc_layer_reports_errors_like_the_allocating_one(ctx):
    _say("[test] noalloc error paths")
    L = abi.lib()
    x = ctx.array((17, C2.hidden), np.float32)
    out = ctx.array((17, C2.hidden), np.float32)
    assert L.pbmoe_moe_layer_noalloc(ctx.handle, 999, x.ptr, x.ptr, 1, None, None, None, out.ptr,
                                     None) == abi.ERR_NOT_BOUND
    dl = DeviceLayer(ctx, C2, 2, index=41)
    assert L.pbmoe_moe_layer_noalloc(ctx.handle, 41, x.ptr, x.ptr, 17, None, None, None, out.ptr,
                                     None) == abi.ERR_UNSUPPORTED
    dl.moe.unbind()
