"""GPU parity of the layer-major prefill path (grouped Q4 GEMM on the matrix
cores) against the CPU oracle: chunks of more than 16 tokens through
pbmoe_moe_prefill, outputs within max-abs <= 1e-2 and relative L2 <= 2e-3 of
the fp32 oracle (fp64 evaluation deciding where outputs are too large for
1e-2 to be above f32 rounding)."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

from pb_amd import abi, synth
from pb_amd.configs import C1, C2, C3, C5
from pb_amd.synth import MoeConfig
from tests.gpu_common import SEED, DeviceLayer, assert_layer_tolerance

pytestmark = pytest.mark.gpu

# small shapes that cover the other group sizes, bf16 scale/bias and a
# bf16 shared expert
T_G32 = MoeConfig("t_g32", hidden=512, intermediate=256, experts=16, k=4, group=32,
                  sb_dtype=abi.DTYPE_F16)
T_G128 = MoeConfig("t_g128_bf16", hidden=1024, intermediate=512, experts=32, k=6, group=128,
                   sb_dtype=abi.DTYPE_BF16)
T_SHARED = MoeConfig("t_shared_bf16", hidden=512, intermediate=256, experts=16, k=4,
                     shared_intermediate=256, shared_gated=True, sb_dtype=abi.DTYPE_BF16)
# the largest expert count (1024): up to 1024 + 1 items in the tile table,
# and more than 2048 routes, so the multi-workgroup dispatch plan
T_E1024 = MoeConfig("t_e1024", hidden=512, intermediate=256, experts=1024, k=8,
                    shared_intermediate=256, shared_gated=True, sb_dtype=abi.DTYPE_F16)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = abi.Context(0)
    yield c
    c.close()


_layers: dict = {}


def _layer(ctx, cfg):
    if cfg.name not in _layers:
        _say(f"[setup] binding {cfg.name}")
        _layers[cfg.name] = DeviceLayer(ctx, cfg, 0, index=len(_layers))
    return _layers[cfg.name]


def _routes(ctx, dl, xh):
    T = xh.shape[0]
    x = ctx.to_device(xh)
    ids = ctx.array((T, dl.cfg.k), np.uint32)
    w = ctx.array((T, dl.cfg.k), np.float32)
    dl.moe.route(x, ids, w)
    ctx.sync()
    return x, ids, w


def _prefill(ctx, dl, x, rh, ids, w, norm=None):
    T = rh.shape[0]
    res = ctx.to_device(rh)
    out = ctx.array((T, dl.cfg.hidden), np.float32)
    nn = ctx.array((T, dl.cfg.hidden), np.float32) if norm is not None else None
    dl.moe.qwen_layer_major_experts(x, res, ids, w, out, norm, nn)
    ctx.sync()
    return out.download(), (nn.download() if nn is not None else None)


THREADS = max(1, min(16, os.cpu_count() or 1))  # the oracle's OpenMP threads


def _check_rows(dl, xh, rh, ids_h, w_h, got, rows, norm_h=None, got_n=None, tag=""):
    ref_h, ref_n = dl.oracle_block(xh[rows], rh[rows], ids_h[rows], w_h[rows], next_norm=norm_h,
                                   threads=THREADS)
    exact = None
    if np.max(np.abs(ref_h)) > 1e3:
        exact = dl.exact_block(xh[rows], rh[rows], ids_h[rows], w_h[rows], threads=THREADS)
    mx, rel = assert_layer_tolerance(got[rows], ref_h, exact=exact)
    _say(f"[result] prefill {tag}: rows={len(rows)} max_abs={mx:.3e} rel_l2={rel:.3e}")
    if norm_h is not None:
        assert_layer_tolerance(got_n[rows], ref_n, "next_normed")


@pytest.mark.parametrize("cfg,T,with_norm", [(C1, 17, False), (C1, 200, True), (C2, 64, True),
                                             (T_G32, 100, False), (T_G128, 150, True),
                                             (T_SHARED, 80, True), (T_E1024, 600, False)])
def test_prefill_matches_oracle(ctx, cfg, T, with_norm):
    _say(f"[test] prefill {cfg.name} T={T} norm={with_norm}")
    dl = _layer(ctx, cfg)
    xh, rh = synth.activations(SEED, 200 + T, T, cfg.hidden)
    x, ids, w = _routes(ctx, dl, xh)
    norm_h = synth.uniform_f32(SEED, 99, 0, 0, 0, cfg.hidden, 0.5, 1.0) if with_norm else None
    got, got_n = _prefill(ctx, dl, x, rh, ids, w, ctx.to_device(norm_h) if with_norm else None)
    _check_rows(dl, xh, rh, ids.download().astype(np.int32), w.download(), got, np.arange(T), norm_h, got_n,
                f"{cfg.name} T={T}")


def test_prefill_full_mantissa_inputs(ctx):
    """Inputs that are not f16 numbers exercise the lo part of the split."""
    _say("[test] prefill full-mantissa inputs")
    dl = _layer(ctx, C1)
    T = 96
    xh, rh = synth.activations(SEED, 301, T, C1.hidden)
    u = synth.uniform_f32(SEED, 98, 0, 0, 0, T * C1.hidden, -1.0, 2.0).reshape(T, C1.hidden)
    xh = (xh * np.float32(1.0 + 1e-3 * np.pi) + np.float32(1e-4) * u).astype(np.float32)
    x, ids, w = _routes(ctx, dl, xh)
    got, _ = _prefill(ctx, dl, x, rh, ids, w)
    _check_rows(dl, xh, rh, ids.download().astype(np.int32), w.download(), got, np.arange(T), tag="full mantissa")


def test_prefill_tile_boundaries(ctx):
    """Experts with 1, 63, 64, 65 and 130 tokens: partial and multiple tiles."""
    _say("[test] prefill tile boundaries")
    cfg = T_G32
    dl = _layer(ctx, cfg)
    T, K, E = 130, cfg.k, cfg.experts
    ids_h = np.zeros((T, K), np.uint32)
    ids_h[:, 0] = 0                                  # 130 tokens
    ids_h[:, 1] = np.where(np.arange(T) < 65, 1, 2)  # 65 and 65
    ids_h[:, 2] = np.where(np.arange(T) < 64, 3, 4)  # 64 and 66
    ids_h[:, 3] = 5 + (np.arange(T) % 11)            # ragged
    ids_h[0, 3] = 15                                 # 1 token
    ids_h[1:64, 3] = np.where(np.arange(1, 64) % 2 == 0, 6, 7)
    w_h = np.full((T, K), 1.0 / K, np.float32)
    w_h[:, 0] = 0.4
    w_h[:, 1:] = 0.2
    xh, rh = synth.activations(SEED, 302, T, cfg.hidden)
    x = ctx.to_device(xh)
    got, _ = _prefill(ctx, dl, x, rh, ctx.to_device(ids_h), ctx.to_device(w_h))
    assert len(set(ids_h.ravel().tolist())) <= E
    _check_rows(dl, xh, rh, ids_h.astype(np.int32), w_h, got, np.arange(T), tag="tile boundaries")


def test_prefill_c3_zipf(ctx):
    """C3: 2048 tokens, Zipf(1.1)-drawn router logits, routed on the device;
    every row against the oracle; a second call is bitwise identical."""
    _say("[test] prefill C3 zipf")
    dl = _layer(ctx, C1)
    T = C3.tokens
    logits_h, hist = synth.drawn_logits_zipf(SEED, 0, T, C3.experts, C3.k, 1.1)
    xh, rh = synth.activations(SEED, 303, T, C3.hidden)
    ids = ctx.array((T, C3.k), np.uint32)
    w = ctx.array((T, C3.k), np.float32)
    dl.moe.route_logits(ctx.to_device(logits_h), ids, w)
    ctx.sync()
    x = ctx.to_device(xh)
    got, _ = _prefill(ctx, dl, x, rh, ids, w)
    again, _ = _prefill(ctx, dl, x, rh, ids, w)
    np.testing.assert_array_equal(got.view(np.uint32), again.view(np.uint32))
    ids_h, w_h = ids.download().astype(np.int32), w.download()
    counts = np.bincount(ids_h.ravel(), minlength=C3.experts)
    _say(f"[info] C3 expert load max={counts.max()} min={counts.min()} used={np.count_nonzero(counts)}")
    _check_rows(dl, xh, rh, ids_h, w_h, got, np.arange(T), tag="C3 zipf")


def test_prefill_c5_shape(ctx):
    """DeepSeek-V3 shape: H7168, I2048, 256 experts, ungated shared expert."""
    _say("[test] prefill C5")
    dl = _layer(ctx, C5)
    T = 24
    xh, rh = synth.activations(SEED, 304, T, C5.hidden)
    x, ids, w = _routes(ctx, dl, xh)
    got, _ = _prefill(ctx, dl, x, rh, ids, w)
    _check_rows(dl, xh, rh, ids.download().astype(np.int32), w.download(), got, np.arange(T), tag="C5")


def test_prefill_c5_full_chunk(ctx):
    """C5 at its benchmark size: 1024 tokens through the DeepSeek-V3-shaped
    layer (group-limited sigmoid routing on the device); every row against
    the oracle and its fp64 evaluation, and a second call bitwise identical."""
    _say("[test] prefill C5 1024 tokens")
    dl = _layer(ctx, C5)
    T = 1024
    xh, rh = synth.activations(SEED, 306, T, C5.hidden)
    x, ids, w = _routes(ctx, dl, xh)
    got, _ = _prefill(ctx, dl, x, rh, ids, w)
    again, _ = _prefill(ctx, dl, x, rh, ids, w)
    np.testing.assert_array_equal(got.view(np.uint32), again.view(np.uint32))
    ids_h, w_h = ids.download().astype(np.int32), w.download()
    counts = np.bincount(ids_h.ravel(), minlength=C5.experts)
    _say(f"[info] C5 expert load max={counts.max()} min={counts.min()} used={np.count_nonzero(counts)}")
    _check_rows(dl, xh, rh, ids_h, w_h, got, np.arange(T), tag="C5 1024")


def test_prefill_out_of_range_route_is_reported(ctx):
    _say("[test] prefill bad route")
    dl = _layer(ctx, C1)
    T = 20
    xh, rh = synth.activations(SEED, 305, T, C1.hidden)
    ids_h = np.tile(np.arange(C1.k, dtype=np.uint32), (T, 1))
    ids_h[7, 2] = C1.experts + 1
    w_h = np.full((T, C1.k), 1.0 / C1.k, np.float32)
    res = ctx.to_device(rh)
    out = ctx.array((T, C1.hidden), np.float32)
    dl.moe.qwen_layer_major_experts(ctx.to_device(xh), res, ctx.to_device(ids_h), ctx.to_device(w_h), out)
    with pytest.raises(abi.PbmoeError) as e:
        ctx.sync()
    assert e.value.status == abi.ERR_ROUTE
    ctx.sync()


@pytest.mark.parametrize("case", ["x_group_offset", "constant_rows"])
def test_prefill_group_sums_beyond_f16(ctx, case):
    """Rows whose elements fit the f16 operands but whose sums over a
    quantisation group do not: "x_group_offset" adds 1100 to one group of
    64 columns (x group sum >= 70400; the split then scales the row by a
    power of two until its group sums fit), "constant_rows" sets three rows
    to 0.25 everywhere, so that each of their SwiGLU activations is about
    2300 and a group of 64 of them sums to about 147000, beyond the f16 hi
    part of the down GEMM's bias-term operand.  Either the result matches
    the oracle or the call reports PBMOE_ERR_NONFINITE (an activation or a
    sum of 64 activations beyond f16); a non-finite output without that
    report fails.  (The synthetic expert weights have a group mean of about
    0.09, so an x group sum beyond f16 drives the activations beyond f16 as
    well: the first case ends in the report, like the second.)"""
    _say(f"[test] prefill group sums beyond f16: {case}")
    dl = _layer(ctx, C1)
    T = 40
    xh, rh = synth.activations(SEED, 307, T, C1.hidden)
    for r in (3, 17, 38):
        if case == "x_group_offset":
            xh[r, 64 * (r % 32):64 * (r % 32) + 64] += np.float32(1100.0)
        else:
            xh[r, :] = np.float32(0.25)
    x, ids, w = _routes(ctx, dl, xh)
    res = ctx.to_device(rh)
    out = ctx.array((T, C1.hidden), np.float32)
    dl.moe.qwen_layer_major_experts(x, res, ids, w, out)
    try:
        ctx.sync()
    except abi.PbmoeError as e:
        assert e.status == abi.ERR_NONFINITE, e
        _say(f"[result] {case}: f16-range error reported")
        ctx.sync()
        return
    got = out.download()
    assert np.all(np.isfinite(got)), f"{np.count_nonzero(~np.isfinite(got))} non-finite outputs, no error"
    _check_rows(dl, xh, rh, ids.download().astype(np.int32), w.download(), got, np.arange(T),
                tag=f"group sums beyond f16: {case}")
