"""GPU parity of the decode stack's GQA attention layer (pbmoe_attention_decode)
against the CPU oracle (or_attention_decode: full_attention_output_values,
runtime/mod.rs:2215-2367, causal_attention math.rs:671-707, q/k norm + RoPE
math.rs:252-325), and of a whole decoder layer (attention + MoE) of the C4
stack."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc
from pb_amd import abi, synth
from pb_amd.configs import C1, C4_ATTN
from pb_amd.flashmoe import AttentionLayer
from tests.gpu_common import SEED, DeviceLayer, assert_layer_tolerance, max_abs_rel_l2

pytestmark = pytest.mark.gpu

F = np.float32


@pytest.fixture(scope="module")
def ctx():
    c = abi.Context(0)
    yield c
    c.close()


def _oracle(acfg, layer):
    mats = synth.attn_host_mats(acfg, SEED, layer, abi.q4_layout_fixed)
    qn, kn, _, _ = synth.attn_norms(acfg, SEED, layer)
    return orc.AttnOracle(mats, qn, kn, acfg.hidden, acfg.q_heads, acfg.kv_heads, acfg.head_dim,
                          acfg.rope_theta, acfg.group, acfg.sb_dtype, acfg.max_context)


def _check_attention(att, ref_att, what):
    # f32 arithmetic on both sides, different summation orders: tight bar
    mx, rel = max_abs_rel_l2(att, ref_att)
    assert rel <= 1e-4 and mx <= 1e-3 * max(1.0, float(np.max(np.abs(ref_att)))), f"{what}: {mx:.3e} {rel:.3e}"


SHAPES = [
    synth.AttnConfig("t_q8_kv8", hidden=512, q_heads=8, kv_heads=8, max_context=200),
    synth.AttnConfig("t_q16_kv4", hidden=512, q_heads=16, kv_heads=4, max_context=200),
    synth.AttnConfig("t_q16_kv8_bf16", hidden=1024, q_heads=16, kv_heads=8, max_context=200, sb_dtype=2),
    synth.AttnConfig("t_q8_kv1_g32", hidden=512, q_heads=8, kv_heads=1, max_context=200, group=32),
    synth.AttnConfig("c4_attention_short", hidden=2048, q_heads=32, kv_heads=4, max_context=200),
]


@pytest.mark.parametrize("acfg", SHAPES, ids=[s.name for s in SHAPES])
def test_attention_decode_sequence_matches_oracle(ctx, acfg):
    """Decode positions 0..140 one token at a time (the cache fills as it
    goes, chunks 64/128 are crossed); every position checked."""
    layer = 50
    dev = AttentionLayer(ctx, layer, acfg).bind_synth(SEED, layer)
    orc_l = _oracle(acfg, layer)
    H = acfg.hidden
    rng = np.random.default_rng(acfg.q_heads * 7 + acfg.kv_heads)
    x_d, r_d = ctx.array((H,), F), ctx.array((H,), F)
    h_d, a_d = ctx.array((H,), F), ctx.array((acfg.q_width,), F)
    for pos in range(141):
        x = rng.standard_normal(H).astype(F)
        r = rng.standard_normal(H).astype(F)
        x_d.upload(x), r_d.upload(r)
        dev.decode(x_d, r_d, pos, h_d, attn_out=a_d)
        ctx.sync()
        ref_att, ref_o = orc_l.decode(x, pos)
        _check_attention(a_d.download(), ref_att, f"{acfg.name} pos {pos}")
        assert_layer_tolerance(h_d.download(), r + ref_o, f"{acfg.name} hidden pos {pos}")
    check = abi.lib().pbmoe_unbind_attention(ctx.handle, layer)
    assert check == 0


@pytest.mark.parametrize("pos", [1000, 4095])
def test_attention_long_context_matches_oracle(ctx, pos):
    """C4 shape at a long context: the cache rows 0..pos-1 are filled with
    the same f16 values on both sides, then one decode at `pos` (64 chunks at
    4095), with the post-attention RMSNorm."""
    acfg, layer = C4_ATTN, 51
    dev = AttentionLayer(ctx, layer, acfg).bind_synth(SEED, layer)
    orc_l = _oracle(acfg, layer)
    rng = np.random.default_rng(pos)
    kw = acfg.kv_width
    keys = (rng.standard_normal((pos, kw)) * 1.5).astype(np.float16)
    vals = rng.standard_normal((pos, kw)).astype(np.float16)
    kp, vp = dev.kv_cache()
    abi.check(abi.lib().pbmoe_upload(ctx.handle, kp, keys.ctypes.data, keys.nbytes))
    abi.check(abi.lib().pbmoe_upload(ctx.handle, vp, vals.ctypes.data, vals.nbytes))
    orc_l.cache_k[:pos] = keys.astype(F)
    orc_l.cache_v[:pos] = vals.astype(F)
    H = acfg.hidden
    x = rng.standard_normal(H).astype(F)
    r = rng.standard_normal(H).astype(F)
    x_d, r_d = ctx.to_device(x), ctx.to_device(r)
    h_d, n_d, a_d = ctx.array((H,), F), ctx.array((H,), F), ctx.array((acfg.q_width,), F)
    dev.decode(x_d, r_d, pos, h_d, post_norm=dev.post_norm, post_normed=n_d, attn_out=a_d)
    ctx.sync()
    ref_att, ref_o = orc_l.decode(x, pos)
    _check_attention(a_d.download(), ref_att, f"pos {pos}")
    ref_h = r + ref_o
    assert_layer_tolerance(h_d.download(), ref_h, "hidden")
    assert_layer_tolerance(n_d.download(), orc.rms_norm(ref_h, dev.post_norm_h, acfg.eps), "post_normed")
    # this position's key/value rows were written to the cache as f16
    kc = np.empty(kw, np.float16)
    abi.check(abi.lib().pbmoe_download(ctx.handle, kc.ctypes.data, kp + pos * kw * 2, kc.nbytes))
    assert np.max(np.abs(kc.astype(F) - orc_l.cache_k[pos])) <= 2e-3 * max(1.0, float(np.max(np.abs(kc))))
    abi.check(abi.lib().pbmoe_unbind_attention(ctx.handle, layer))


@pytest.mark.parametrize("acfg", [SHAPES[1], C4_ATTN], ids=["t_q16_kv4", "c4"])
def test_attention_fused_input_norm_matches_oracle(ctx, acfg):
    """The input RMSNorm formed inside the q/k/v projection kernel
    (input_norm given, the un-normalised hidden state passed): positions
    0..69 against the oracle on oracle-normalised rows, with the hidden state
    also the residual."""
    layer = 54
    dev = AttentionLayer(ctx, layer, acfg).bind_synth(SEED, layer)
    orc_l = _oracle(acfg, layer)
    H = acfg.hidden
    rng = np.random.default_rng(11)
    x_d, h_d = ctx.array((H,), F), ctx.array((H,), F)
    n_d, a_d = ctx.array((H,), F), ctx.array((acfg.q_width,), F)
    for pos in range(70):
        x = (rng.standard_normal(H) * 3.0).astype(F)
        x_d.upload(x)
        dev.decode(x_d, x_d, pos, h_d, post_norm=dev.post_norm, post_normed=n_d, attn_out=a_d,
                   input_norm=dev.input_norm)
        ctx.sync()
        ref_att, ref_o = orc_l.decode(orc.rms_norm(x, dev.input_norm_h, acfg.eps), pos)
        _check_attention(a_d.download(), ref_att, f"{acfg.name} pos {pos}")
        ref_h = x + ref_o
        assert_layer_tolerance(h_d.download(), ref_h, f"{acfg.name} hidden pos {pos}")
        assert_layer_tolerance(n_d.download(), orc.rms_norm(ref_h, dev.post_norm_h, acfg.eps), "post_normed")
    abi.check(abi.lib().pbmoe_unbind_attention(ctx.handle, layer))


@pytest.mark.parametrize("pos", [4096, 6000, 20479])
def test_attention_beyond_the_merge_block_matches_oracle(ctx, pos):
    """Contexts past 64 chunks (4096 positions): the merge kernel loads the
    first 64 chunks' values up front and folds the rest in a second loop;
    65, 94 and 320 chunks, C4 head shape with a 20480-position cache."""
    acfg = synth.AttnConfig("c4_long", hidden=2048, q_heads=32, kv_heads=4, max_context=20480)
    layer = 55
    dev = AttentionLayer(ctx, layer, acfg).bind_synth(SEED, layer)
    orc_l = _oracle(acfg, layer)
    rng = np.random.default_rng(pos)
    kw = acfg.kv_width
    keys = (rng.standard_normal((pos, kw)) * 1.5).astype(np.float16)
    vals = rng.standard_normal((pos, kw)).astype(np.float16)
    kp, vp = dev.kv_cache()
    abi.check(abi.lib().pbmoe_upload(ctx.handle, kp, keys.ctypes.data, keys.nbytes))
    abi.check(abi.lib().pbmoe_upload(ctx.handle, vp, vals.ctypes.data, vals.nbytes))
    orc_l.cache_k[:pos] = keys.astype(F)
    orc_l.cache_v[:pos] = vals.astype(F)
    H = acfg.hidden
    x = rng.standard_normal(H).astype(F)
    r = rng.standard_normal(H).astype(F)
    x_d, r_d = ctx.to_device(x), ctx.to_device(r)
    h_d, a_d = ctx.array((H,), F), ctx.array((acfg.q_width,), F)
    dev.decode(x_d, r_d, pos, h_d, attn_out=a_d)
    ctx.sync()
    ref_att, ref_o = orc_l.decode(x, pos)
    _check_attention(a_d.download(), ref_att, f"pos {pos}")
    assert_layer_tolerance(h_d.download(), r + ref_o, "hidden")
    abi.check(abi.lib().pbmoe_unbind_attention(ctx.handle, layer))


def test_attention_rejects_position_beyond_cache(ctx):
    acfg = synth.AttnConfig("t_small", hidden=512, q_heads=8, kv_heads=2, max_context=16)
    layer = 52
    dev = AttentionLayer(ctx, layer, acfg).bind_synth(SEED, layer)
    H = acfg.hidden
    x_d, h_d = ctx.array((H,), F), ctx.array((H,), F)
    rc = abi.lib().pbmoe_attention_decode(ctx.handle, layer, x_d.ptr, None, x_d.ptr, 16, h_d.ptr, None, None, None)
    assert rc == abi.ERR_SHAPE
    abi.check(abi.lib().pbmoe_unbind_attention(ctx.handle, layer))


def test_attention_phase_events_time_each_kernel(ctx):
    """pbmoe_set_phase_events with 14 events also times the attention
    kernels (q/k/v, chunk partials, merge, o_proj): every pair brackets a
    dispatch of positive duration; counts other than 0, 6 and 14 are
    rejected."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    hip.hipEventSynchronize.argtypes = [C.c_void_p]
    hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    hip.hipEventDestroy.argtypes = [C.c_void_p]
    evs = []
    for _ in range(14):
        e = C.c_void_p()
        assert hip.hipEventCreate(C.byref(e)) == 0
        evs.append(e)
    arr = (C.c_void_p * 14)(*[e.value for e in evs])
    assert abi.lib().pbmoe_set_phase_events(ctx.handle, arr, 7) == abi.ERR_INVALID_ARGUMENT
    acfg = synth.AttnConfig("t_events", hidden=512, q_heads=16, kv_heads=4, max_context=200)
    layer = 54
    dev = AttentionLayer(ctx, layer, acfg).bind_synth(SEED, layer)
    H = acfg.hidden
    rng = np.random.default_rng(11)
    x_d, r_d, h_d = ctx.array((H,), F), ctx.array((H,), F), ctx.array((H,), F)
    x_d.upload(rng.standard_normal(H).astype(F))
    r_d.upload(rng.standard_normal(H).astype(F))
    abi.check(abi.lib().pbmoe_set_phase_events(ctx.handle, arr, 14))
    try:
        dev.decode(x_d, r_d, 150, h_d)
        ctx.sync()
    finally:
        abi.check(abi.lib().pbmoe_set_phase_events(ctx.handle, None, 0))
    for i in range(4):
        ms = C.c_float()
        assert hip.hipEventSynchronize(evs[7 + 2 * i]) == 0
        assert hip.hipEventElapsedTime(C.byref(ms), evs[6 + 2 * i], evs[7 + 2 * i]) == 0
        assert ms.value > 0.0, f"attention kernel {i}"
    for e in evs:
        hip.hipEventDestroy(e)
    abi.check(abi.lib().pbmoe_unbind_attention(ctx.handle, layer))


def test_attention_rejects_unsupported_shapes(ctx):
    d = abi.AttnDesc()
    d.hidden, d.q_heads, d.kv_heads, d.head_dim, d.rotary_dim = 512, 8, 3, 128, 128
    d.rope_theta, d.max_context, d.group_size, d.scale_bias_dtype = 1e6, 8, 64, 1
    w = abi.AttnWeights()
    assert abi.lib().pbmoe_bind_attention(ctx.handle, 53, C.byref(d), C.byref(w)) == abi.ERR_SHAPE
    d.kv_heads, d.head_dim, d.rotary_dim = 2, 64, 64
    assert abi.lib().pbmoe_bind_attention(ctx.handle, 53, C.byref(d), C.byref(w)) == abi.ERR_UNSUPPORTED


def test_decoder_layers_of_the_c4_stack_match_oracle(ctx):
    """Two C4 decoder layers (attention -> o_proj + residual -> post-attention
    RMSNorm -> C1 MoE block with the next layer's input RMSNorm fused) for
    three positions, with zero-mean (centred) expert weights as in the bench
    stack.  Each kernel phase is checked against the oracle given
    the device's own inputs for that phase (the oracle's KV cache is built
    from the device's normed inputs), so every layer is checked in isolation;
    routes are the device's, checked bit-exact against the oracle's
    selection on the device logits."""
    acfg, moe_cfg = C4_ATTN, C1
    H = acfg.hidden
    layers = []
    for l in range(2):
        att = AttentionLayer(ctx, 60 + l, acfg).bind_synth(SEED, 60 + l)
        moe = DeviceLayer(ctx, moe_cfg, 60 + l, abi.ORDER_REFERENCE_SLOT, index=60 + l, centred=True)
        layers.append((att, moe, _oracle(acfg, 60 + l)))
    rng = np.random.default_rng(4)
    h = rng.standard_normal(H).astype(F)
    h_d = ctx.to_device(h.reshape(1, H))
    x_d = ctx.to_device(orc.rms_norm(h, layers[0][0].input_norm_h, acfg.eps).reshape(1, H))
    mid_d, post_d = ctx.array((1, H), F), ctx.array((1, H), F)
    out_d, nxt_d = ctx.array((1, H), F), ctx.array((1, H), F)
    ids = ctx.array((1, moe_cfg.k), np.uint32)
    w = ctx.array((1, moe_cfg.k), np.float32)
    logits = ctx.array((1, moe_cfg.experts), np.float32)
    for pos in range(3):
        for l, (att, moe, orc_att) in enumerate(layers):
            nxt = layers[(l + 1) % 2][0]
            x_in, h_in = x_d.download().ravel(), h_d.download().ravel()
            att.decode(x_d, h_d, pos, mid_d, post_norm=att.post_norm, post_normed=post_d)
            moe.moe.route(post_d, ids, w, logits)
            moe.moe.submit_scheduled_expert_command(post_d, mid_d, ids, w, out_d, nxt.input_norm, nxt_d)
            ctx.sync()
            _, o = orc_att.decode(x_in, pos)
            mid = mid_d.download().ravel()
            assert_layer_tolerance(mid, h_in + o, f"pos {pos} layer {l} attention hidden")
            post = post_d.download().ravel()
            assert_layer_tolerance(post, orc.rms_norm(mid, att.post_norm_h, acfg.eps), f"pos {pos} layer {l} post")
            got_ids = ids.download().astype(np.int32)
            ref_ids, _ = orc.route_rows(logits.download(), moe_cfg.k, orc.ROUTING_SOFTMAX, orc.ORDER_REFERENCE_SLOT)
            assert (got_ids == ref_ids).all()
            ref_out, ref_next = moe.oracle_block(post.reshape(1, H), mid.reshape(1, H), got_ids, w.download(),
                                                 next_norm=nxt.input_norm_h)
            out = out_d.download().ravel()
            assert_layer_tolerance(out, ref_out.ravel(), f"pos {pos} layer {l} hidden")
            assert_layer_tolerance(nxt_d.download().ravel(), orc.rms_norm(out, nxt.input_norm_h, acfg.eps),
                                   f"pos {pos} layer {l} next normed")
            h_d, out_d = out_d, h_d
            x_d, nxt_d = nxt_d, x_d
    for att, moe, _ in layers:
        abi.check(abi.lib().pbmoe_unbind_attention(ctx.handle, att.index))
        moe.moe.unbind()


@pytest.mark.parametrize("sb", [abi.DTYPE_F16, abi.DTYPE_BF16])
def test_device_centring_matches_host(ctx, sb):
    """pbmoe_synth_center_q4 on the device == synth.center_q4_slots on the
    host, bit for bit (the stack's oracle relies on it)."""
    H, I, E = 256, 128, 3
    lay = abi.q4_layout_fixed(H, I, 64, sb)
    dev = ctx.array(E * lay.expert_bytes, np.uint8)
    abi.check(abi.lib().pbmoe_synth_fill_q4(ctx.handle, dev.ptr, C.byref(lay), H, I, SEED, synth.T_EXPERT, 7, 0, E))
    abi.check(abi.lib().pbmoe_synth_center_q4(ctx.handle, dev.ptr, C.byref(lay), H, I, E))
    host = synth.q4_experts(SEED, synth.T_EXPERT, 7, 0, E, H, I, 64, sb, lay.offsets, int(lay.expert_bytes))
    ref = synth.center_q4_slots(host, lay, E, sb)
    got = dev.download()
    assert np.array_equal(got, ref)
    assert not np.array_equal(got, host)
