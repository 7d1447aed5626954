"""Pin the CPU oracle against the reference's own golden vectors and against
closed forms / brute force.  Reference paths are relative to
src/inference/flashmoe/ of Jc2k/pb.  CPU only."""
import math

import numpy as np
import pytest

from oracle import oracle as orc

F = np.float32


# ---------------------------------------------------------------- routing ----
def test_top_k_stable_tie_break_golden():
    # math.rs:1231-1238
    ids, vals = orc.top_k_sorted([0.1, 0.9, 0.9, -1.0], 2)
    assert ids == [1, 2] and vals == [F(0.9), F(0.9)]
    w = orc.softmax_in_place(vals)
    assert abs(float(w.sum()) - 1.0) < 1e-6


def test_routing_top_k_replacement_slot_order_golden():
    # math.rs:1257-1279
    scores = [0.1, 2.0, -1.0, 3.0, 0.5, 2.5, -0.2, 1.5, 4.0]
    ids, _ = orc.routing_top_k(scores, 4)
    assert ids == [5, 1, 8, 3]
    ids2, _ = orc.routing_softmax_top_k(scores, 4, orc.ORDER_REFERENCE_SLOT)
    assert ids2 == [5, 1, 8, 3]


def test_routing_softmax_below_sentinel_golden():
    # math.rs:1292-1305
    ids, p = orc.routing_softmax_top_k([-2.0e30, -3.0e30, -4.0e30], 2, orc.ORDER_REFERENCE_SLOT)
    assert ids == [0, 1]
    assert np.all(np.isfinite(p))
    assert abs(float(p.sum()) - 1.0) < 1e-6


def test_top_k_non_four_k_golden():
    # math_parity_tests.rs:12-28
    ids, vals = orc.top_k_sorted([0.2, 1.0, 0.9, -1.0, 3.0, 2.0, 3.0, 1.5], 5)
    assert ids == [4, 6, 5, 7, 1]
    w = orc.softmax_in_place(vals)
    assert abs(float(w.sum()) - 1.0) < 1e-6 and np.all(w > 0)


def test_topk_then_softmax_matches_softmax_then_topk_renorm_golden():
    # math_parity_tests.rs:30-57
    scores = [0.25, -1.0, 3.5, 3.5, 0.0, 2.25, -0.5, 1.75]
    ids, vals = orc.top_k_sorted(scores, 4)
    pb = orc.softmax_in_place(vals)
    probs = orc.softmax_in_place(scores)
    rids, rvals = orc.top_k_sorted(probs, 4)
    ref = np.asarray(rvals, F) / F(sum(rvals))
    assert ids == rids
    assert np.max(np.abs(pb - ref)) <= 1e-6


def test_selection_from_logits_equals_topk_of_probabilities_golden():
    # tests/scheduler.rs:2208-2226 (exact equality of ids and scores)
    logits = [0.0, 2.0, 2.0, -1.0, 1.0]
    ids, p = orc.routing_softmax_top_k(logits, 3, orc.ORDER_REFERENCE_SLOT)
    probs = orc.softmax_in_place(logits)
    rids, rvals = orc.routing_top_k(probs, 3)
    assert ids == rids
    assert p.tolist() == rvals


def test_noaux_sigmoid_golden():
    # math.rs:1521-1532
    ids, w = orc.routing_sigmoid_noaux_top_k([0.0, 2.0, -2.0], [1.0, -1.0, 0.0], 2)
    pairs = sorted(zip(ids, w.tolist()))
    assert [e for e, _ in pairs] == [0, 2]
    assert abs(pairs[0][1] - 0.5) < 1e-6
    assert abs(pairs[1][1] - 1.0 / (1.0 + math.exp(2.0))) < 1e-6


def _brute_slot_scan(scores, k):
    """Independent restatement of the replacement scan used as brute force."""
    slots = [(0, -math.inf)] * k
    for e, s in enumerate(scores):
        m = min(range(k), key=lambda i: (slots[i][1], i))
        if s > slots[m][1]:
            slots[m] = (e, s)
    return [e for e, _ in slots]


@pytest.mark.parametrize("seed", range(20))
def test_topk_orders_against_brute_force(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(8, 300))
    k = int(rng.integers(1, min(n, 16) + 1))
    # ties on purpose: values from a small integer grid
    scores = rng.integers(-6, 6, size=n).astype(F) / F(4)
    ids, _ = orc.top_k_sorted(scores, k)
    brute = sorted(range(n), key=lambda e: (-float(scores[e]), e))[:k]
    assert ids == brute
    ids2, _ = orc.routing_top_k(scores, k)
    assert ids2 == _brute_slot_scan(scores.tolist(), k)
    # the replacement scan keeps the same multiset of values as the sorted top-k
    assert sorted(scores[ids2].tolist()) == sorted(scores[ids].tolist())


def test_replacement_scan_differs_from_lower_index_rule_on_boundary_tie():
    # [1, 1, 2] with K=2: the scan evicts slot 0 (expert 0) for expert 2;
    # the stable sort keeps expert 0.  The HIP router offers both orders.
    assert orc.routing_top_k([1.0, 1.0, 2.0], 2)[0] == [2, 1]
    assert orc.top_k_sorted([1.0, 1.0, 2.0], 2)[0] == [2, 0]


@pytest.mark.parametrize("seed", range(10))
def test_grouped_routing_reduces_to_noaux_at_one_group(seed):
    rng = np.random.default_rng(100 + seed)
    n, k = 64, 6
    logits = rng.normal(size=n).astype(F)
    bias = rng.uniform(-0.1, 0.1, size=n).astype(F)
    gids, gw = orc.routing_sigmoid_grouped_top_k(logits, bias, k, 1, 1)
    nids, nw = orc.routing_sigmoid_noaux_top_k(logits, bias, k, orc.ORDER_CANONICAL)
    assert gids == nids
    np.testing.assert_array_equal(gw, nw)
    sids, _ = orc.routing_sigmoid_noaux_top_k(logits, bias, k, orc.ORDER_REFERENCE_SLOT)
    assert sorted(sids) == sorted(nids)


@pytest.mark.parametrize("seed", range(10))
def test_grouped_routing_brute_force(seed):
    rng = np.random.default_rng(200 + seed)
    n, k, ng, tg = 256, 8, 8, 4
    logits = rng.normal(size=n).astype(F)
    bias = rng.uniform(-0.05, 0.05, size=n).astype(F)
    ids, w = orc.routing_sigmoid_grouped_top_k(logits, bias, k, ng, tg)
    sig = (F(1) / (F(1) + np.exp(-logits))).astype(F)
    biased = (sig + bias).astype(F)
    per = n // ng
    gs = [float(np.sort(biased[g * per:(g + 1) * per])[-2:].sum(dtype=F)) for g in range(ng)]
    keep = sorted(range(ng), key=lambda g: (-gs[g], g))[:tg]
    cand = [e for e in range(n) if e // per in keep]
    brute = sorted(cand, key=lambda e: (-float(biased[e]), e))[:k]
    assert ids == brute
    np.testing.assert_allclose(w, sig[ids], rtol=1e-6, atol=0)  # numpy exp vs libm expf: 1 ulp


def test_grouped_routing_exact_ties_brute_force():
    """Every group has the same top-2 sum and experts repeat across groups:
    the lower group index and then the lower expert index win."""
    n, k, ng, tg = 32, 5, 4, 2
    base = np.array([0.3, -1.2, 2.0, 0.7, 2.0, -0.4, 0.3, 1.1], F)
    logits = np.tile(base, ng)
    ids, w = orc.routing_sigmoid_grouped_top_k(logits, np.zeros(n, F), k, ng, tg)
    sig = (F(1) / (F(1) + np.exp(-logits))).astype(F)
    per = n // ng
    gs = [float(np.sort(sig[g * per:(g + 1) * per])[-2:].sum(dtype=F)) for g in range(ng)]
    keep = sorted(range(ng), key=lambda g: (-gs[g], g))[:tg]
    assert keep == [0, 1]
    cand = [e for e in range(n) if e // per in keep]
    brute = sorted(cand, key=lambda e: (-float(sig[e]), e))[:k]
    assert ids == brute == [2, 4, 10, 12, 7]


# ---------------------------------------------------------- renormalise ----
def test_renormalize_scale_golden():
    # tests/scheduler.rs:4100-4128
    rc, w = orc.renormalize([0.2, 0.6, 0.1], orc.NORM_RENORMALIZE, 0.25)
    assert rc == 0
    exp = [0.25 * 2 / 9, 0.25 * 6 / 9, 0.25 * 1 / 9]
    assert np.max(np.abs(w - np.asarray(exp))) < 1e-6


def test_renormalize_deepseek_floor_golden():
    # tests/scheduler.rs:4131-4152
    rc, w = orc.renormalize([1.0e-6, 2.0e-6], orc.NORM_DEEPSEEK_FLOOR, 1.5)
    assert rc == 0
    assert abs(w[0] - 1.5e-6 / 6.103515625e-5) < 1e-7
    assert abs(w[1] - 3.0e-6 / 6.103515625e-5) < 1e-7
    rc, w = orc.renormalize([1.0e-6, 2.0e-6], orc.NORM_RENORMALIZE, 1.5)
    assert rc == 0 and abs(w[0] - 0.5) < 1e-6 and abs(w[1] - 1.0) < 1e-6


def test_renormalize_rejections():
    # tests/scheduler.rs:4154-4166 (PreserveFullSoftmax), expert_access.rs:93-118
    assert orc.renormalize([1.0, 2.0], orc.NORM_PRESERVE_FULL, 1.0)[0] != 0
    assert orc.renormalize([0.0, 0.0], orc.NORM_RENORMALIZE, 1.0)[0] != 0
    assert orc.renormalize([0.5, -0.1], orc.NORM_RENORMALIZE, 1.0)[0] != 0
    assert orc.renormalize([0.5, 0.5], orc.NORM_RENORMALIZE, 0.0)[0] != 0
    assert orc.renormalize([float("nan"), 0.5], orc.NORM_RENORMALIZE, 1.0)[0] != 0


def test_validate_preselected():
    # protocol.rs:1044-1081
    assert orc.validate_preselected([1, 2], [0.5, 0.5], 2, 4) == 0
    assert orc.validate_preselected([1, 1], [0.5, 0.5], 2, 4) != 0
    assert orc.validate_preselected([1, 4], [0.5, 0.5], 2, 4) != 0
    assert orc.validate_preselected([1], [0.5], 2, 4) != 0
    assert orc.validate_preselected([1, 2], [0.5, float("inf")], 2, 4) != 0


# ------------------------------------------------------ dequant / matvec ----
def test_dequantize_variable_groups_golden():
    # math.rs:1503-1519
    packed = [0x10, 0x32, 0x04, 0x65, 0x87, 0x09]
    out = orc.q4_dequantize_rows(packed, [0.5, -0.25, 0.125, 0.75], [1.0, 2.0, -1.5, 0.25], 2, 5, 3)
    assert out.ravel().tolist() == [1.0, 1.5, 2.0, 1.25, 1.0, -0.875, -0.75, -0.625, 6.25, 7.0]


def test_q4_matvec_nibble_golden():
    # math_parity_tests.rs:96-108
    out = orc.q4_fma_matvec([0x21, 0x43], [1, 2, 3, 4], [0.5], [1.0], 1, 4, 64)
    exp = (1 * 0.5 + 1) * 1 + (2 * 0.5 + 1) * 2 + (3 * 0.5 + 1) * 3 + (4 * 0.5 + 1) * 4
    assert abs(out[0] - exp) < 1e-6


def test_q4_matvec_odd_shapes_golden():
    # math_parity_tests.rs:110-145
    packed = [0x10, 0x32, 0x04, 0x65, 0x87, 0x09, 0xBA, 0xDC, 0x0E]
    x = [0.25, -1.0, 2.0, 0.5, -0.75]
    scales = [0.5, -0.25, 0.125, 0.75, -0.5, 0.25]
    biases = [1.0, 2.0, -1.5, 0.25, 0.0, -0.5]
    out = orc.q4_fma_matvec(packed, x, scales, biases, 3, 5, 3)
    # fp64 brute force over the nibble table q[r][c] = 5r + c
    exp = [sum((5 * r + c) * scales[r * 2 + c // 3] * x[c] + biases[r * 2 + c // 3] * x[c] for c in range(5))
           for r in range(3)]
    assert np.max(np.abs(out - np.asarray(exp))) < 1e-6


def test_q4_matvec_fma_vs_explicit_dequant_golden():
    # math_parity_tests.rs:147-186
    packed = [0xF0, 0x21, 0x43, 0x06, 0x75, 0x98, 0xBA, 0x0D]
    x = [0.5, -2.0, 1.25, 0.0, -0.75, 3.0, -1.5]
    s = [0.03125, -0.125, 0.5, -0.25]
    b = [-1.0, 2.0, 0.25, -0.5]
    a = orc.q4_fma_matvec(packed, x, s, b, 2, 7, 4)
    e = orc.q4_explicit_matvec(packed, x, s, b, 2, 7, 4)
    assert np.max(np.abs(a - e)) <= 1e-6


def test_q4_uint32_word_bf16_golden():
    # experts/parity_tests.rs:1428-1495: word 0x76543210, bf16 s=0.5 b=1.0
    x = [1.0, -2.0, 0.5, 3.0, -1.0, 0.25, 2.0, -0.75]
    packed = list((0x76543210).to_bytes(4, "little"))
    out = orc.q4_fma_matvec(packed, x, [0x3F00], [0x3F80], 1, 8, 8, orc.DT_BF16)
    exp = sum((n * 0.5 + 1.0) * xv for n, xv in enumerate(x))
    assert abs(out[0] - exp) <= 1e-6


def test_tiny_expert_pack_mlp_golden():
    # experts/parity_tests.rs:93-150: gate [30,15], up [45,45], down = 15*a
    lay = orc.make_layout(2, 2, 64, orc.DT_F32, [0, 2, 10, 18, 20, 28, 36, 38, 46], 54)
    slot = np.zeros(64, np.uint8)

    def put(off, vals, dt):
        a = np.asarray(vals, dtype=dt).view(np.uint8)
        slot[off:off + a.size] = a

    put(0, [0xF0, 0x0F], np.uint8)            # gate q = [[0,15],[15,0]]
    put(2, [1.0, 1.0], np.float32)
    put(10, [0.0, 0.0], np.float32)
    put(18, [0x00, 0x00], np.uint8)           # up q = 0, bias 15
    put(20, [1.0, 1.0], np.float32)
    put(28, [15.0, 15.0], np.float32)
    put(36, [0x0F, 0xF0], np.uint8)           # down = diag(15)
    put(38, [1.0, 1.0], np.float32)
    put(46, [0.0, 0.0], np.float32)
    hidden = [1.0, 2.0]
    g = orc.q4_fma_matvec(slot[0:2], hidden, slot[2:10].view(np.float32), slot[10:18].view(np.float32), 2, 2, 64)
    u = orc.q4_fma_matvec(slot[18:20], hidden, slot[20:28].view(np.float32), slot[28:36].view(np.float32), 2, 2, 64)
    assert g.tolist() == [30.0, 15.0] and u.tolist() == [45.0, 45.0]
    y = orc.expert_mlp(lay, slot, hidden)
    a = orc.swiglu(g, u)
    assert np.max(np.abs(y - 15.0 * a)) <= 1e-5 * max(1.0, float(np.max(np.abs(15 * a))))


@pytest.mark.parametrize("seed", range(6))
def test_q4_matvec_fp64_brute_force(seed):
    rng = np.random.default_rng(300 + seed)
    rows, cols, group = int(rng.integers(1, 6)), 64 * int(rng.integers(1, 5)), 64
    packed = rng.integers(0, 256, size=rows * cols // 2, dtype=np.uint8)
    gpr = cols // group
    s = rng.uniform(0.005, 0.02, size=rows * gpr).astype(F)
    b = rng.uniform(-0.1, 0.1, size=rows * gpr).astype(F)
    x = rng.normal(size=cols).astype(F)
    out = orc.q4_fma_matvec(packed, x, s, b, rows, cols, group)
    q = np.stack([packed & 15, packed >> 4], axis=1).reshape(rows, cols).astype(np.float64)
    w = q * np.repeat(s.reshape(rows, gpr), group, 1) + np.repeat(b.reshape(rows, gpr), group, 1)
    exp = w @ x.astype(np.float64)
    bound = 4 * cols * 2.0**-24 * (np.abs(w) @ np.abs(x.astype(np.float64))) + 1e-30
    assert np.all(np.abs(out - exp) <= bound)


def test_dequant_closed_form_exact():
    # q*s+b with q <= 15 and an 11-bit scale is exact before the final rounding:
    # fma(q, s, b) == fp64(q*s+b) rounded once to f32
    rng = np.random.default_rng(7)
    packed = rng.integers(0, 256, size=4 * 32, dtype=np.uint8)
    s16 = rng.uniform(0.005, 0.02, size=4).astype(np.float16)
    b16 = rng.uniform(-0.1, 0.1, size=4).astype(np.float16)
    out = orc.q4_dequantize_rows(packed, s16.view(np.uint16), b16.view(np.uint16), 4, 64, 64, orc.DT_F16)
    q = np.stack([packed & 15, packed >> 4], axis=1).reshape(4, 64).astype(np.float64)
    exp = (q * s16.astype(np.float64)[:, None] + b16.astype(np.float64)[:, None]).astype(F)
    np.testing.assert_array_equal(out, exp)


def test_rms_norm_closed_form():
    x = np.asarray([3.0, 4.0], F)
    out = orc.rms_norm(x, [1.0, 0.5], 0.0)
    r = math.sqrt((9 + 16) / 2)
    assert abs(out[0] - 3 / r) < 1e-6 and abs(out[1] - 0.5 * 4 / r) < 1e-6


# --------------------------------------------------------- layer goldens ----
def _identity_slot_layout():
    """tiny_fixed_q4_layout (tests/scheduler.rs:134-187) + identity slot bytes
    (tests/scheduler.rs:268-282): 2x2 identity, group 2, bf16 scale 1, bias 0."""
    lay = orc.make_layout(2, 2, 2, orc.DT_BF16, [0, 8, 12, 16, 24, 28, 32, 40, 44], 48)
    slot = np.zeros(48, np.uint8)
    for w, s in ((0, 8), (16, 24), (32, 40)):
        slot[w], slot[w + 1] = 0x01, 0x10
        slot[s:s + 4] = [0x80, 0x3F, 0x80, 0x3F]
    return lay, slot


NORMED = [1.2955897, 0.5669620]
ATTN = [1.0092846, 1.6604769]
SCORES = [0.1, 2.0, -1.0, 3.0, 0.5, 2.5, -0.2, 1.5, 4.0]


def _residual():
    return np.asarray([F(0.5) + F(ATTN[0]), F(-1.0) + F(ATTN[1])], F)


def test_k4_layer_golden():
    # tests/scheduler.rs:826-1011
    residual = _residual()
    normed = orc.rms_norm(residual, [1.0, 1.0])
    assert np.max(np.abs(normed - np.asarray(NORMED))) <= 1e-6
    probs = orc.softmax_in_place(SCORES)
    ids, p = orc.routing_top_k(probs, 4)
    assert ids == [5, 1, 8, 3]
    rc, w = orc.renormalize(p, orc.NORM_RENORMALIZE, 1.0)
    assert rc == 0
    assert np.max(np.abs(w - np.asarray([0.12925005, 0.07839412, 0.57925856, 0.2130973]))) <= 1e-6
    # production routing (softmax top-k on raw logits) gives the same routes
    ids2, p2 = orc.routing_softmax_top_k(SCORES, 4, orc.ORDER_REFERENCE_SLOT)
    assert ids2 == ids and np.max(np.abs(p2 - np.asarray(p))) <= 1e-7
    lay, slot = _identity_slot_layout()
    ys = np.stack([orc.expert_mlp(lay, slot, normed) for _ in ids])
    hidden = orc.combine(residual, ys, w, shared=[0.25, -0.5], shared_weight=1.0)
    assert np.max(np.abs(hidden - np.asarray([3.0771027, 0.36557937]))) <= 1e-5
    nn = orc.rms_norm(hidden, [1.0, 0.5])
    assert np.max(np.abs(nn - np.asarray([1.404337, 0.08342209]))) <= 1e-5


def test_k8_no_shared_layer_golden_through_block():
    # tests/scheduler.rs:1013-1176, through the whole-block oracle
    residual = _residual()
    normed = orc.rms_norm(residual, [1.0, 1.0])
    probs = orc.softmax_in_place(SCORES)
    ids, p = orc.routing_top_k(probs, 8)
    assert ids == [0, 1, 8, 3, 4, 5, 6, 7]
    rc, w = orc.renormalize(p, orc.NORM_RENORMALIZE, 1.0)
    exp_w = [0.010802226, 0.072222546, 0.5336564, 0.19632123, 0.016115028, 0.11907485, 0.008002486, 0.04380519]
    assert rc == 0 and np.max(np.abs(w - np.asarray(exp_w))) <= 1e-6
    lay, slot = _identity_slot_layout()
    slots = np.tile(slot, 9)
    hidden, nn = orc.moe_block(lay, slots, 9, normed[None, :], residual[None, :], np.asarray([ids], np.int32),
                               w[None, :], next_norm_w=np.asarray([1.0, 0.5], F))
    assert np.max(np.abs(hidden[0] - np.asarray([2.8271027, 0.86557925]))) <= 1e-5
    assert np.max(np.abs(nn[0] - np.asarray([1.3522521, 0.20701078]))) <= 1e-5


def test_shared_gate_combine_closed_form():
    # qwen_layer_major_combine: sigma only applies with a shared router;
    # without a gate projection the constant 80.0 gives sigma = 1 exactly
    # (metal/mod.rs:4666-4669).
    assert F(1) / (F(1) + np.exp(F(-80))) == F(1)
    r = np.asarray([1.0, 2.0], F)
    ys = np.asarray([[1.0, 1.0], [3.0, -1.0]], F)
    out = orc.combine(r, ys, [0.25, 0.75], shared=[4.0, 8.0], shared_weight=0.5)
    assert out.tolist() == [1.0 + (0.25 + 2.25) + 2.0, 2.0 + (0.25 - 0.75) + 4.0]


# ------------------------------------------------------------ group plan ----
def test_group_plan_golden():
    # tests/metal.rs:536-547
    src, out, groups = orc.group_plan([1, 0, 0, 1], 2, 2)
    assert src.tolist() == [0, 1, 0, 1]
    assert out.tolist() == [2, 0, 1, 3]
    assert groups == [(0, 2), (2, 2)]
    for bad in (([0, 0], 2, 1), ([2], 2, 1), ([], 0, 0)):
        with pytest.raises(ValueError):
            orc.group_plan(*bad)


@pytest.mark.parametrize("seed", range(8))
def test_group_plan_is_stable_sort(seed):
    rng = np.random.default_rng(400 + seed)
    T, K, E = int(rng.integers(1, 200)), int(rng.integers(1, 11)), 64
    ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(T)]).astype(np.int32)
    uniq, slots = orc.layer_major_union(ids, E)
    assert uniq.tolist() == sorted(set(ids.ravel().tolist()))
    assert np.all(uniq[slots] == ids.ravel())
    src, out, groups = orc.group_plan(slots, len(uniq), K)
    order = sorted(range(T * K), key=lambda r: (slots[r], r))   # stable sort by slot
    assert src.tolist() == [r // K for r in order]
    assert [order[i] for i in out] == list(range(T * K))
    assert sum(c for _, c in groups) == T * K


def test_fp64_block_agrees_with_f32_golden():
    # the fp64 evaluation reproduces the K8 golden (tests/scheduler.rs:1013-1176)
    residual = _residual()
    normed = orc.rms_norm(residual, [1.0, 1.0])
    ids, p = orc.routing_top_k(orc.softmax_in_place(SCORES), 8)
    _, w = orc.renormalize(p, orc.NORM_RENORMALIZE, 1.0)
    lay, slot = _identity_slot_layout()
    h = orc.moe_block_f64(lay, np.tile(slot, 9), 9, normed[None, :], residual[None, :], np.asarray([ids], np.int32),
                          w[None, :])
    assert np.max(np.abs(h[0] - np.asarray([2.8271027, 0.86557925]))) <= 1e-5
