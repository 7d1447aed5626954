"""Host rules the bench prices decode kernels by (no GPU): the algorithmic
bytes of the three decode kernels add up to the whole layer's however the
shared expert's gate/up rows are placed, and one C2 token's shared rows go
with the gate/up launch (its down-prefetch workgroups), as the library's
host rule `shared_rows_in_gateup` decides."""
from dataclasses import replace

from pb_amd.configs import C1, C2, C5, decode_phase_bytes, q4_proj_bytes, shared_rows_in_gateup


def test_shared_rows_follow_the_gate_up_launch_for_one_c2_token():
    assert shared_rows_in_gateup(C2, 1)
    assert not shared_rows_in_gateup(C2, 2)          # several tokens: the router stage
    assert not shared_rows_in_gateup(C1, 1)          # no shared expert
    assert not shared_rows_in_gateup(C5, 1)          # the wide-activation shape
    one = decode_phase_bytes(C2, C2.k, 1)
    shared_gu = 2 * q4_proj_bytes(C2.shared_intermediate, C2.hidden, C2.group) + C2.shared_intermediate * 4
    routed_gu = C2.k * 2 * q4_proj_bytes(C2.intermediate, C2.hidden, C2.group)
    assert one["gateup"] == routed_gu + C2.experts * 4 + C2.hidden * 4 + C2.k * C2.intermediate * 4 + shared_gu


def test_phase_bytes_total_does_not_depend_on_the_placement():
    for cfg in (C2, replace(C2, name="c2_wide_shared", shared_intermediate=4096)):
        for T in (1, 2):
            b = decode_phase_bytes(cfg, cfg.k, T, fused_norm=True)
            moved = shared_rows_in_gateup(cfg, T)
            Is, H, g = cfg.shared_intermediate, cfg.hidden, cfg.group
            shared_gu = 2 * q4_proj_bytes(Is, H, g) + T * Is * 4
            base = decode_phase_bytes(replace(cfg, shared_intermediate=0), cfg.k, T, fused_norm=True)
            # the shared gate/up bytes are in exactly one of the two kernels
            assert b["stage"] + b["gateup"] == base["stage"] + base["gateup"] + shared_gu + (H * 2 if cfg.shared_gated else 0)
            assert (b["gateup"] - base["gateup"] == shared_gu) == moved
