"""The C-ABI library loads, exports every symbol include/pbmoe.h declares, and
its host-only entry points (layout, route validation, renormalisation) agree
with the reference rules.  No GPU calls."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from oracle import oracle as orc
from pb_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    text = open(os.path.join(ROOT, "include", "pbmoe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pbmoe_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = _header_functions()
    assert len(names) >= 20
    L = C.CDLL(abi.LIB_PATH)
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/pbmoe.h but not exported"
    assert sorted(abi.exported_symbols()) == names


def test_abi_version():
    assert abi.lib().pbmoe_abi_version() == 1


@pytest.mark.parametrize("h,i,total", [(2048, 768, 2_654_208), (2048, 512, 1_769_472), (7168, 2048, 24_772_608),
                                       (4096, 1024, 7_077_888)])
def test_fixed_layout_sizes(h, i, total):
    # per-expert byte accounting (g=64, 2-byte scale/bias)
    for dt in (abi.DTYPE_F16, abi.DTYPE_BF16):
        lay = abi.q4_layout_fixed(h, i, 64, dt)
        assert lay.expert_bytes == total
        assert abi.lib().pbmoe_q4_layout_validate(C.byref(lay)) == 0


def test_fixed_layout_matches_qwen35_constant_offsets():
    # QwenMoeQ4ExpertLayout::qwen35_a17b (model_family.rs:1070-1122)
    lay = abi.q4_layout_fixed(4096, 1024, 64, abi.DTYPE_BF16)
    assert lay.offsets == [0, 2_097_152, 2_228_224, 2_359_296, 4_456_448, 4_587_520, 4_718_592, 6_815_744,
                           6_946_816]
    assert [c.kind for c in lay.components] == list(range(9))


def test_fixed_layout_rejections():
    out = abi.Q4Layout()
    L = abi.lib()
    assert L.pbmoe_q4_layout_fixed(0, 512, 64, abi.DTYPE_F16, C.byref(out)) == abi.ERR_SHAPE
    assert L.pbmoe_q4_layout_fixed(2048, 500, 64, abi.DTYPE_F16, C.byref(out)) == abi.ERR_SHAPE
    assert b"must be divisible by group_size" in L.pbmoe_last_error()
    assert L.pbmoe_q4_layout_fixed(2048, 512, 64, abi.DTYPE_F32, C.byref(out)) == abi.ERR_DTYPE
    assert b"must be F16 or BF16" in L.pbmoe_last_error()


def test_layout_validate_rejects_gaps_and_totals():
    lay = abi.q4_layout_fixed(2048, 512, 64, abi.DTYPE_F16)
    lay.components[4].offset += 2
    assert abi.lib().pbmoe_q4_layout_validate(C.byref(lay)) == abi.ERR_SHAPE
    lay = abi.q4_layout_fixed(2048, 512, 64, abi.DTYPE_F16)
    lay.expert_bytes += 16
    assert abi.lib().pbmoe_q4_layout_validate(C.byref(lay)) == abi.ERR_SHAPE
    lay = abi.q4_layout_fixed(2048, 512, 64, abi.DTYPE_F16)
    lay.scale_bias_dtype = abi.DTYPE_F32
    assert abi.lib().pbmoe_q4_layout_validate(C.byref(lay)) == abi.ERR_UNSUPPORTED


@pytest.mark.parametrize("seed", range(30))
def test_validate_routes_matches_protocol(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(2, 40))
    K = int(rng.integers(1, min(E, 10) + 1))
    ids = rng.integers(0, E + 2, size=K)
    scores = rng.normal(size=K).astype(np.float32)
    if seed % 5 == 0:
        scores[0] = np.inf
    ok_ref = orc.validate_preselected(ids, scores, K, E) == 0
    ok = abi.validate_routes(ids, scores, K, E) == abi.OK
    assert ok == ok_ref


@pytest.mark.parametrize("policy", [abi.NORM_RENORMALIZE_SELECTED, abi.NORM_DEEPSEEK_FLOOR])
@pytest.mark.parametrize("seed", range(10))
def test_host_renormalize_bitwise_matches_oracle(policy, seed):
    rng = np.random.default_rng(seed)
    p = rng.uniform(0, 1, size=int(rng.integers(1, 11))).astype(np.float32)
    if seed == 3:
        p[:] = 1e-7
    scale = float(rng.choice([1.0, 2.5, 0.25, 1.5]))
    rc, w = abi.renormalize_routes(p, policy, scale)
    rc2, w2 = orc.renormalize(p, policy, scale)
    assert (rc == 0) == (rc2 == 0)
    if rc == 0:
        np.testing.assert_array_equal(w, w2)


def test_host_renormalize_rejects_full_softmax():
    rc, _ = abi.renormalize_routes([0.5, 0.5], abi.NORM_PRESERVE_FULL_SOFTMAX, 1.0)
    assert rc == abi.ERR_UNSUPPORTED
    assert b"full expert softmax" in abi.lib().pbmoe_last_error()
