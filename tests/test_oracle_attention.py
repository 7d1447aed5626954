"""Pin the oracle's GQA attention layer (decode stack row): the reference's
golden vectors, closed forms, f64 brute force, and properties chosen so that
a wrong head mapping, a dropped scale or a swapped rotation sign fails.
Reference paths are relative to src/inference/flashmoe/ of Jc2k/pb.  CPU
only."""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from pb_amd import abi, synth
from pb_amd.configs import C4_ATTN

F = np.float32


def test_causal_attention_golden():
    # tests/scheduler.rs:826-851: one head, width 2, two positions
    out = orc.causal_attention([1.0, 0.0], [[1.0, 0.0], [0.0, 1.0]], [[2.0, 1.0], [-1.0, 3.0]], 1, 1, 2)
    assert np.max(np.abs(out - np.array([1.0092846, 1.6604769], F))) <= 1e-6


def test_residual_rms_norm_golden():
    # tests/scheduler.rs:852-860: residual + attention, then RMSNorm (weights 1)
    att = orc.causal_attention([1.0, 0.0], [[1.0, 0.0], [0.0, 1.0]], [[2.0, 1.0], [-1.0, 3.0]], 1, 1, 2)
    normed = orc.rms_norm(np.array([0.5, -1.0], F) + att, np.ones(2, F))
    assert np.max(np.abs(normed - np.array([1.2955897, 0.5669620], F))) <= 1e-6


def _gqa_f64(q, keys, values, qh, kvh, hd):
    """Textbook grouped-query attention in float64: kv heads repeated
    q_heads / kv_heads times (consecutive q heads share a kv head)."""
    n = keys.shape[0]
    Q = q.reshape(qh, hd).astype(np.float64)
    K = np.repeat(keys.reshape(n, kvh, hd).astype(np.float64), qh // kvh, axis=1)  # [n][qh][hd]
    V = np.repeat(values.reshape(n, kvh, hd).astype(np.float64), qh // kvh, axis=1)
    s = np.einsum("hd,nhd->hn", Q, K) / math.sqrt(hd)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return np.einsum("hn,nhd->hd", p, V).ravel()


@pytest.mark.parametrize("qh,kvh,n", [(4, 2, 1), (4, 2, 17), (8, 1, 33), (6, 3, 5), (4, 4, 9)])
def test_causal_attention_matches_f64_gqa(qh, kvh, n):
    rng = np.random.default_rng(qh * 100 + kvh * 10 + n)
    hd = 8
    q = rng.standard_normal(qh * hd).astype(F)
    k = rng.standard_normal((n, kvh * hd)).astype(F)
    v = rng.standard_normal((n, kvh * hd)).astype(F)
    got = orc.causal_attention(q, k, v, qh, kvh, hd)
    ref = _gqa_f64(q, k, v, qh, kvh, hd)
    assert np.max(np.abs(got - ref)) <= 2e-6 * max(1.0, np.max(np.abs(ref)))


def test_causal_attention_properties():
    rng = np.random.default_rng(5)
    qh, kvh, hd = 4, 2, 8
    q = rng.standard_normal(qh * hd).astype(F)
    # one position: every head returns its kv head's value row
    v1 = rng.standard_normal((1, kvh * hd)).astype(F)
    out = orc.causal_attention(q, rng.standard_normal((1, kvh * hd)).astype(F), v1, qh, kvh, hd)
    for h in range(qh):
        kv = h // (qh // kvh)
        assert np.array_equal(out[h * hd:(h + 1) * hd], v1[0, kv * hd:(kv + 1) * hd])
    # identical keys: uniform weights, the mean of the values
    n = 7
    k = np.tile(rng.standard_normal((1, kvh * hd)).astype(F), (n, 1))
    v = rng.standard_normal((n, kvh * hd)).astype(F)
    out = orc.causal_attention(q, k, v, qh, kvh, hd)
    for h in range(qh):
        kv = h // (qh // kvh)
        assert np.allclose(out[h * hd:(h + 1) * hd], v[:, kv * hd:(kv + 1) * hd].mean(axis=0), atol=1e-6)


def test_rope_split_half_closed_forms():
    rng = np.random.default_rng(11)
    heads, hd, theta = 3, 8, 1e6
    x = rng.standard_normal(heads * hd).astype(F)
    # position 0 (no norm weight): identity
    assert np.array_equal(orc.qk_norm_rope(x, heads, hd, None, 0, hd, theta), x)
    pos = 5
    y = orc.qk_norm_rope(x, heads, hd, None, pos, hd, theta)
    half = hd // 2
    for h in range(heads):
        a, b = x[h * hd:(h + 1) * hd].astype(np.float64), y[h * hd:(h + 1) * hd].astype(np.float64)
        for i in range(half):
            # each (i, i + half) pair is rotated: its norm is preserved
            assert math.isclose(a[i] ** 2 + a[i + half] ** 2, b[i] ** 2 + b[i + half] ** 2, rel_tol=1e-5)
            ang = pos * theta ** (-(2 * i) / hd)  # frequency 0 turns by exactly `position` radians
            exp0 = a[i] * math.cos(ang) - a[i + half] * math.sin(ang)
            exp1 = a[i] * math.sin(ang) + a[i + half] * math.cos(ang)
            assert abs(b[i] - exp0) <= 1e-5 and abs(b[i + half] - exp1) <= 1e-5


def test_rope_partial_rotary_leaves_tail():
    # math_parity_tests.rs:196-227: position 3, head_dim 8, rotary_dim 4,
    # theta 1e7 (the non-rotary tail stays untouched)
    x = np.array([1.0, 2.0, 3.0, 4.0, 100.0, 200.0, 300.0, 400.0], F)
    y = orc.qk_norm_rope(x, 1, 8, None, 3, 4, 1e7)
    assert np.array_equal(y[4:], x[4:])
    for i in range(2):
        ang = 3 * (1e7 ** (-(2 * i) / 4))
        assert abs(y[i] - (x[i] * math.cos(ang) - x[i + 2] * math.sin(ang))) <= 1e-5
        assert abs(y[i + 2] - (x[i] * math.sin(ang) + x[i + 2] * math.cos(ang))) <= 1e-5


def test_qk_norm_is_per_head_rms_times_weight():
    rng = np.random.default_rng(3)
    heads, hd = 4, 16
    x = (rng.standard_normal(heads * hd) * 3.0).astype(F)
    w = rng.uniform(0.5, 1.5, hd).astype(F)
    y = orc.qk_norm_rope(x, heads, hd, w, 0, hd, 1e6)  # position 0: norm only
    for h in range(heads):
        a = x[h * hd:(h + 1) * hd].astype(np.float64)
        exp = a / math.sqrt(np.mean(a * a) + 1e-6) * w
        assert np.max(np.abs(y[h * hd:(h + 1) * hd] - exp)) <= 1e-5


def test_attention_layer_oracle_against_f64_pipeline():
    """or_attention_decode against a float64 restatement built from
    independent pieces (explicit dequantisation, numpy norms, the textbook
    GQA above) on a small seeded layer over 5 positions."""
    acfg = synth.AttnConfig("t", hidden=256, q_heads=4, kv_heads=2, head_dim=128, group=64, max_context=8)
    mats = synth.attn_host_mats(acfg, 77, 0, abi.q4_layout_fixed)
    qn, kn, _, _ = synth.attn_norms(acfg, 77, 0)
    orc_layer = orc.AttnOracle(mats, qn, kn, acfg.hidden, acfg.q_heads, acfg.kv_heads, acfg.head_dim,
                               acfg.rope_theta, acfg.group, orc.DT_F16, acfg.max_context)

    def deq(name, rows, cols):
        c, s, b = mats[name]
        return orc.q4_dequantize_rows(c, s, b, rows, cols, acfg.group, orc.DT_F16).astype(np.float64)

    H, qw, kw, hd = acfg.hidden, acfg.q_width, acfg.kv_width, acfg.head_dim
    Wq, Wk, Wv, Wo = deq("q", qw, H), deq("k", kw, H), deq("v", kw, H), deq("o", H, qw)

    def norm_rope(x, heads, w, pos):
        x = x.reshape(heads, hd).copy()
        x = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6) * w
        half = hd // 2
        ang = pos * acfg.rope_theta ** (-(2 * np.arange(half)) / hd)
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = x[:, :half].copy(), x[:, half:].copy()
        x[:, :half], x[:, half:] = x0 * c - x1 * s, x0 * s + x1 * c
        return x.ravel()

    rng = np.random.default_rng(1)
    ks, vs = [], []
    for pos in range(5):
        x = rng.standard_normal(H).astype(F)
        att, o = orc_layer.decode(x, pos)
        xd = x.astype(np.float64)
        q = norm_rope(Wq @ xd, acfg.q_heads, qn, pos)
        ks.append(norm_rope(Wk @ xd, acfg.kv_heads, kn, pos).astype(np.float16).astype(np.float64))
        vs.append((Wv @ xd).astype(np.float16).astype(np.float64))
        ref_att = _gqa_f64(q, np.array(ks), np.array(vs), acfg.q_heads, acfg.kv_heads, hd)
        ref_o = Wo @ ref_att
        assert np.max(np.abs(att - ref_att)) <= 2e-3 * max(1.0, np.max(np.abs(ref_att))), pos
        assert np.max(np.abs(o - ref_o)) <= 2e-3 * max(1.0, np.max(np.abs(ref_o))), pos


def test_f16_cache_rows_are_f16_values():
    # the KV cache stores f16 (round to nearest even): after a decode step the
    # oracle's cache rows equal numpy's float16 rounding of themselves
    rng = np.random.default_rng(9)
    acfg = synth.AttnConfig("t", hidden=128, q_heads=1, kv_heads=1, head_dim=128, group=64, max_context=2)
    mats = synth.attn_host_mats(acfg, 5, 0, abi.q4_layout_fixed)
    qn, kn, _, _ = synth.attn_norms(acfg, 5, 0)
    layer = orc.AttnOracle(mats, qn, kn, 128, 1, 1, 128, 1e6, 64, orc.DT_F16, 2)
    layer.decode(rng.standard_normal(128).astype(F), 0)
    for row in (layer.cache_k[0], layer.cache_v[0]):
        assert np.array_equal(row, row.astype(np.float16).astype(F))
        assert np.any(row != 0)
