"""The oracle's DeepSeek-V4 router (deepseek_v4_router_probabilities +
deepseek_v4_select_routes, deepseek.rs:1300-1394, and the floor
renormalisation x 1.5 of batch_route_rows, metal/deepseek_execution.rs:
3547-3583).  The reference's tests hold no golden vector for it, so the
restatement is pinned by what the mathematics fixes: the three softplus
branches against an f64 evaluation, the selection against an independent
stable sort, exact ties, the optional bias, the floor, and the rejection of
non-finite input."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc

F = np.float32


def ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def f64_sqrt_softplus(l):
    l = np.asarray(l, np.float64)
    sp = np.where(l > 20.0, l, np.where(l < -20.0, np.exp(l), np.log1p(np.exp(l))))
    return np.sqrt(sp)


def test_probability_branches_against_f64():
    l = np.concatenate([np.linspace(-60, 60, 2401),
                        np.array([-20.0, -19.999998, -20.000002, 20.0, 19.999998, 20.000002, 0.0, -0.0,
                                  1e-30, -1e-30, 88.0, -87.0])]).astype(F)
    p = orc.sqrt_softplus(l)
    ref = f64_sqrt_softplus(l).astype(F)
    # two f32 library calls and a correctly rounded sqrt: within 2 ulp
    assert int(ulps(p, ref).max()) <= 2
    # the branch boundaries are strict: 20 and -20 take the log1p branch
    assert orc.sqrt_softplus(np.array([20.0], F))[0] == np.float32(np.sqrt(np.float32(np.log1p(np.exp(np.float32(20.0))))))
    assert orc.sqrt_softplus(np.array([25.0], F))[0] == np.sqrt(np.float32(25.0))
    assert orc.sqrt_softplus(np.array([-30.0], F))[0] == np.sqrt(np.exp(np.float32(-30.0)))
    assert np.all(p >= 0.0)
    assert np.all(np.diff(p[:2401]) >= 0.0)  # monotone in the logit


@pytest.mark.parametrize("seed", range(6))
def test_selection_is_the_stable_descending_sort(seed):
    rng = np.random.default_rng(seed)
    E, K = 256, 6
    logits = (rng.standard_normal(E) * 3).astype(F)
    bias = (rng.standard_normal(E) * 0.1).astype(F) if seed % 2 else None
    ids, w = orc.routing_sqrt_softplus_top_k(logits, bias, K)
    p = f64_sqrt_softplus(logits).astype(F)  # independent evaluation, rounded once
    score = p + (bias if bias is not None else F(0))
    order = sorted(range(E), key=lambda e: (-float(score[e]), e))  # stable: lower index on ties
    gap = np.sort(score)[::-1]
    if gap[K - 1] - gap[K] > 1e-5:  # no near-tie at the cut: the f64 rounding cannot reorder
        assert ids == order[:K]
    assert int(ulps(w, p[ids]).max()) <= 2  # weights are the unbiased probabilities


def test_exact_ties_take_the_lower_index():
    E, K = 256, 6
    logits = np.zeros(E, F)
    ids, _ = orc.routing_sqrt_softplus_top_k(logits, None, K)
    assert ids == [0, 1, 2, 3, 4, 5]
    logits[[200, 7, 100]] = 1.0
    ids, _ = orc.routing_sqrt_softplus_top_k(logits, None, K)
    assert ids == [7, 100, 200, 0, 1, 2]
    # a bias can lift a low probability above a tie, and ties again resolve low
    bias = np.zeros(E, F)
    bias[50] = 10.0
    ids, w = orc.routing_sqrt_softplus_top_k(logits, bias, K)
    assert ids == [50, 7, 100, 200, 0, 1]
    assert w[0] == orc.sqrt_softplus(np.array([0.0], F))[0]  # unbiased


def test_missing_bias_equals_zero_bias():
    rng = np.random.default_rng(11)
    logits = (rng.standard_normal(256) * 4).astype(F)
    a = orc.routing_sqrt_softplus_top_k(logits, None, 6)
    b = orc.routing_sqrt_softplus_top_k(logits, np.zeros(256, F), 6)
    assert a[0] == b[0] and np.array_equal(a[1], b[1])


def test_route_rows_floor_renormalisation_and_scale():
    """batch_route_rows: sum of the six scores in route order (sequential
    f32), inverse = 1 / max(sum, 6.1035156e-5), weight = score * inverse * 1.5."""
    rng = np.random.default_rng(3)
    T, E, K = 5, 256, 6
    logits = (rng.standard_normal((T, E)) * 3).astype(F)
    logits[4] = -60.0  # every probability ~1e-13: the floor decides
    logits[4, [9, 3]] = -50.0
    bias = (rng.standard_normal(E) * 0.05).astype(F)
    ids, w = orc.route_rows(logits, K, orc.ROUTING_SQRT_SOFTPLUS, orc.ORDER_CANONICAL, bias=bias,
                            policy=orc.NORM_DEEPSEEK_FLOOR, routed_scale=1.5)
    for t in range(T):
        sel, p = orc.routing_sqrt_softplus_top_k(logits[t], bias, K)
        assert list(ids[t]) == sel
        s = F(0.0)
        for v in p:
            s = F(s + v)
        inv = F(1.0) / max(s, F(6.103515625e-5))
        np.testing.assert_array_equal(w[t], (p * inv).astype(F) * F(1.5))
    assert np.sum(w[4]) < 1e-6  # floored: the weights do not sum to the scale


def test_non_finite_input_is_rejected():
    logits = np.zeros(256, F)
    logits[17] = np.nan
    with pytest.raises(ValueError):
        orc.routing_sqrt_softplus_top_k(logits, None, 6)
    bias = np.zeros(256, F)
    bias[3] = np.inf
    with pytest.raises(ValueError):
        orc.routing_sqrt_softplus_top_k(np.zeros(256, F), bias, 6)
