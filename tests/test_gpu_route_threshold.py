"""GPU: the workgroup routing of decode token counts (route_token_block,
canonical order) selects through a threshold when it can: the 16 groups of
16 threads publish their key maxima, tau is the K-th largest of them, and
wave 0 sorts the keys >= tau when there are at most 64 of them; otherwise
every wave sorts its 128 keys.  Both paths must give the oracle's ids
bitwise.  Rows are built so that the candidate count is just inside (64)
and just outside (65) the single-wave limit, and so that ties force the
full sort; group g of the threshold holds experts 16g .. 16g + 15 and (for
E = 512) 256 + 16g .. 256 + 16g + 15."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle as orc
from pb_amd import abi
from pb_amd.configs import C1, C2
from tests.gpu_common import DeviceLayer

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = abi.Context(0)
    yield c
    c.close()


def _group_experts(g: int, E: int):
    ex = list(range(16 * g, 16 * g + 16))
    if E > 256:
        ex += list(range(256 + 16 * g, 256 + 16 * g + 16))
    return [e for e in ex if e < E]


def _crafted(E: int, K: int, n_cand: int) -> np.ndarray:
    """Logits whose threshold candidate count is n_cand: groups 0 .. K-1
    peak at 100 - g (tau = 101 - K), n_cand - K more experts of groups
    0 .. K-2 sit just above tau, everything else at 0."""
    l = np.zeros(E, np.float32)
    tau = 100.0 - (K - 1)
    extra = n_cand - K
    for g in range(K):
        ex = _group_experts(g, E)
        l[ex[0]] = 100.0 - g
        if g < K - 1:
            take = min(extra, len(ex) - 1)
            l[ex[1:1 + take]] = tau + 0.5
            extra -= take
    assert extra == 0
    return l


def _rows(cfg, rng):
    E, K = cfg.experts, cfg.k
    rows = [rng.standard_normal(E).astype(np.float32),        # spread scores: threshold path
            _crafted(E, K, 64),                                # exactly the single-wave limit
            _crafted(E, K, 65),                                # one over: the full sort
            np.zeros(E, np.float32)]                           # all tied: the full sort
    r = rng.standard_normal(E).astype(np.float32)
    r[::3] = 1.5                                               # ties at the K boundary
    rows.append(r)
    r = (rng.standard_normal(E) * 1e-3).astype(np.float32)    # narrow spread
    r[rng.integers(0, E, 3)] = 5.0
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("cfg", [C1, C2])
def test_threshold_and_full_sort_select_the_oracle_ids(ctx, cfg):
    _say(f"[test] threshold routing {cfg.name}")
    dl = DeviceLayer(ctx, cfg, 0, abi.ORDER_CANONICAL, index=60 + (cfg is C2))
    rng = np.random.default_rng(77)
    l = _rows(cfg, rng)
    T = l.shape[0]
    assert abi.ORDER_CANONICAL == 0 and T <= 16  # the workgroup routing path
    d = ctx.to_device(l)
    ids = ctx.array((T, cfg.k), np.uint32)
    w = ctx.array((T, cfg.k), np.float32)
    dl.moe.route_logits(d, ids, w)
    ctx.sync()
    ref_ids, ref_w = orc.route_rows(l, cfg.k, orc.ROUTING_SOFTMAX, orc.ORDER_CANONICAL)
    np.testing.assert_array_equal(ids.download().astype(np.int32), ref_ids)
    np.testing.assert_allclose(w.download(), ref_w, rtol=4e-6, atol=0)
    _say(f"[result] {cfg.name}: {T} rows bit-exact")
    dl.moe.unbind()
