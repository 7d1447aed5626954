"""Seeded generator: conversions are exact RNE, streams are deterministic and
have the benchmark input distributions.  CPU only."""
import numpy as np
import torch

from pb_amd import abi, synth


def test_f16_rne_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(size=20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, size=20000),
        np.asarray([0.0, -0.0, 65504.0, 65519.996, 65520.0, 70000.0, -1e30, 5.960464477539063e-08,
                    2.9802322387695312e-08, 2.98023259e-08, 6.1035156e-05, 6.0975552e-05, np.inf, -np.inf],
                   np.float32),
    ]).astype(np.float32)
    ours = synth.f32_to_f16(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    back = synth.f16_to_f32(ref)
    np.testing.assert_array_equal(back, ref.view(np.float16).astype(np.float32))


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    vals = (rng.normal(size=20000) * 10.0 ** rng.integers(-20, 20, size=20000)).astype(np.float32)
    ours = synth.f32_to_bf16(vals)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)


def _layout(h, i, dt=abi.DTYPE_F16):
    return abi.q4_layout_fixed(h, i, 64, dt)


def test_q4_experts_deterministic_and_in_range():
    lay = _layout(512, 256)
    a = synth.q4_experts(7, synth.T_EXPERT, 3, 5, 2, 512, 256, 64, abi.DTYPE_F16, lay.offsets, lay.expert_bytes)
    b = synth.q4_experts(7, synth.T_EXPERT, 3, 5, 2, 512, 256, 64, abi.DTYPE_F16, lay.offsets, lay.expert_bytes)
    np.testing.assert_array_equal(a, b)
    # expert 6 generated on its own equals the second slot of the pair
    c = synth.q4_experts(7, synth.T_EXPERT, 3, 6, 1, 512, 256, 64, abi.DTYPE_F16, lay.offsets, lay.expert_bytes)
    np.testing.assert_array_equal(a[lay.expert_bytes:], c)
    slot = a[: lay.expert_bytes]
    o = lay.offsets
    nib = slot[o[0]:o[1]]
    q = np.concatenate([nib & 15, nib >> 4])
    counts = np.bincount(q, minlength=16)
    assert counts.min() > 0.8 * q.size / 16
    s = slot[o[1]:o[2]].view(np.float16).astype(np.float32)
    bb = slot[o[2]:o[3]].view(np.float16).astype(np.float32)
    assert s.min() >= 0.005 - 1e-5 and s.max() <= 0.02 + 1e-5
    assert bb.min() >= -0.1 - 1e-4 and bb.max() <= 0.1 + 1e-4
    assert abs(float(bb.mean())) < 0.01


def test_normal_streams():
    x = synth.f16_to_f32(synth.normal_f16(1, synth.T_INPUT, 0, 0, 0, 200000, 1.0))
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    w = synth.f16_to_f32(synth.normal_f16(1, synth.T_ROUTER, 0, 0, 0, 200000, 0.02))
    assert abs(float(w.std()) - 0.02) < 0.001


def test_drawn_logits_zipf():
    logits, hist = synth.drawn_logits_zipf(5, 0, 2048, 128, 8, 1.1)
    chosen = logits > 2.0
    assert np.all(chosen.sum(axis=1) == 8)
    assert int(hist.sum()) == 2048 * 8
    np.testing.assert_array_equal(hist, chosen.sum(axis=0))
    h = np.sort(hist)[::-1].astype(np.float64)
    assert h[0] > 4 * np.median(h)   # skewed load
