"""The benchmark workload shapes of the MoE block.

C1  CPU-runnable single layer: H2048, E128, K8 softmax renormalised, I768.
C2  Qwen3-Next decode: H2048, E512, K10, I512 + sigmoid-gated shared I512.
C3  prefill of 2048 tokens through the C1 layer with drawn Zipf(1.1) logits.
C4  48 decode layers: GQA attention (C4_ATTN) + the C1 MoE layer, context 4096.
C5  DeepSeek-V3 shape: H7168, E256, K8 sigmoid, 8 groups / topk_group 4,
    per-expert selection bias, I2048 + shared I2048 (ungated), routed
    scale 2.5 (the DeepSeek-V3 routed_scaling_factor; the workload leaves it open).
All: 4-bit affine, group 64, f16 scale/bias.
"""
from __future__ import annotations

from .abi import (NORM_RENORMALIZE_SELECTED, ROUTING_SIGMOID_GROUPED, ROUTING_SOFTMAX_TOPK, DTYPE_F16)
from .synth import AttnConfig, MoeConfig

C1 = MoeConfig("c1_decode", hidden=2048, intermediate=768, experts=128, k=8,
               routing=ROUTING_SOFTMAX_TOPK, normalization=NORM_RENORMALIZE_SELECTED, sb_dtype=DTYPE_F16)
C2 = MoeConfig("c2_qwen3next_decode", hidden=2048, intermediate=512, experts=512, k=10,
               routing=ROUTING_SOFTMAX_TOPK, normalization=NORM_RENORMALIZE_SELECTED,
               shared_intermediate=512, shared_gated=True, sb_dtype=DTYPE_F16)
C3 = MoeConfig("c3_prefill_2048", hidden=2048, intermediate=768, experts=128, k=8,
               routing=ROUTING_SOFTMAX_TOPK, normalization=NORM_RENORMALIZE_SELECTED, sb_dtype=DTYPE_F16,
               tokens=2048)
C5 = MoeConfig("c5_deepseekv3_decode", hidden=7168, intermediate=2048, experts=256, k=8,
               routing=ROUTING_SIGMOID_GROUPED, normalization=NORM_RENORMALIZE_SELECTED, routed_scale=2.5,
               n_group=8, topk_group=4, shared_intermediate=2048, shared_gated=False, sb_dtype=DTYPE_F16)

CONFIGS = {c.name: c for c in (C1, C2, C3, C5)}

# C4: 48-layer decode stack of C1-shaped MoE layers, each preceded by GQA
# attention (32 q heads, 4 kv heads, head_dim 128, f16 KV cache, context
# 4096, RMSNorm eps 1e-6, RoPE theta 1e6), Q4 g64 projections, batch 1.
C4_ATTN = AttnConfig("c4_attention", hidden=2048, q_heads=32, kv_heads=4, head_dim=128, rope_theta=1e6,
                     group=64, sb_dtype=DTYPE_F16, max_context=4096)
C4_LAYERS = 48


def algorithmic_bytes(cfg: MoeConfig, unique_experts: int, tokens: int, fused_norm: bool = False) -> int:
    """HBM bytes a decode call must move at minimum: each selected expert's
    Q4 slot once, the shared slot, the router (f16) and shared gate, and the
    f32 activations in (x, residual) and out (hidden); with the fused input
    RMSNorm (pbmoe_moe_layer_norm) also its f32 weight."""
    def slot(h, i):
        return 3 * (h * i // 2) + 3 * 2 * (h * i // cfg.group) * 2
    b = unique_experts * slot(cfg.hidden, cfg.intermediate)
    if cfg.shared_intermediate:
        b += slot(cfg.hidden, cfg.shared_intermediate)
        if cfg.shared_gated:
            b += cfg.hidden * 2
    b += cfg.experts * cfg.hidden * 2
    b += tokens * cfg.hidden * 4 * 3
    if fused_norm:
        b += cfg.hidden * 4
    return b


def q4_proj_bytes(rows: int, cols: int, group: int) -> int:
    """Bytes of one Q4 projection: packed nibbles + 2-byte scale and bias."""
    return rows * cols // 2 + 2 * (rows * cols // group) * 2


def decode_phase_bytes(cfg: MoeConfig, unique_experts: int, tokens: int, fused_norm: bool = False) -> dict:
    """Algorithmic HBM bytes of each decode kernel (pbmoe_moe_layer):
    stage   router rows (f16), shared gate/up (see below) + gate row, x in,
            logits and shared activations out; with the fused input RMSNorm
            (pbmoe_moe_layer_norm) also the norm weight in and the
            normalised rows out (the gate/up kernel's x);
    gateup  gate/up of the selected experts, logits and x in, act out; the
            shared gate/up rows and shared activations instead of the stage
            when shared_rows_in_gateup;
    down    down of the selected experts + shared down, act in, residual
            in, hidden out."""
    H, I, Is, E, K, g, T = (cfg.hidden, cfg.intermediate, cfg.shared_intermediate, cfg.experts, cfg.k,
                            cfg.group, tokens)
    stage = E * H * 2 + T * H * 4 + T * E * 4
    if fused_norm:
        stage += H * 4 + T * H * 4
    shared_gu = 2 * q4_proj_bytes(Is, H, g) + T * Is * 4 if Is else 0
    gateup = unique_experts * 2 * q4_proj_bytes(I, H, g) + T * E * 4 + T * H * 4 + T * K * I * 4
    if Is:
        if shared_rows_in_gateup(cfg, T):
            gateup += shared_gu
        else:
            stage += shared_gu
        if cfg.shared_gated:
            stage += H * 2
    down = unique_experts * q4_proj_bytes(H, I, g) + T * K * I * 4 + 2 * T * H * 4
    if Is:
        down += q4_proj_bytes(H, Is, g) + T * Is * 4
    return {"stage": stage, "gateup": gateup, "down": down}


def shared_rows_in_gateup(cfg: MoeConfig, tokens: int) -> bool:
    """Whether one token's shared-expert gate/up rows run in the gate/up
    kernel's down-prefetch workgroups instead of the router stage (the host
    rule shared_rows_in_gateup in pbmoe_decode.hip): one token, a shared
    expert, not the wide-activation shape, prefetch workgroups present, at
    most four 32-column chunks per lane, and room in the one round of 768
    resident workgroups for one shared row per prefetch wave."""
    if tokens != 1 or not cfg.shared_intermediate:
        return False
    H, I, K = cfg.hidden, cfg.intermediate, cfg.k
    wide = (K + 1) * I > 12288 and (K + 1) * I <= 18432 and I % 512 == 0 and 1024 <= I <= 2048 and H % 16 == 0
    if wide:
        return False
    pf_base = ((K * (I // 2) + 3) // 4 + 7) // 8 * 8  # the gate/up workgroups before the prefetch ones
    room = (768 - pf_base) // 8 * 8 if pf_base < 768 else 0
    return (down_prefetch_bytes(cfg, K, 1) > 0 and (H // 32 + 63) // 64 <= 4
            and room * 4 >= cfg.shared_intermediate)


def down_prefetch_bytes(cfg: MoeConfig, unique_experts: int, tokens: int) -> int:
    """Bytes of down weights (codes, scales, biases) that route_gateup_kernel
    touches for down_combine_kernel: the selected experts and the shared
    expert, when they total at most 16 MiB and the gate/up grid leaves room
    for the prefetch workgroups (the host rule in pbmoe_decode.hip)."""
    H, I, g = cfg.hidden, cfg.intermediate, cfg.group
    max_items = min(cfg.experts, tokens * cfg.k) if tokens > 1 else tokens * cfg.k
    items_bound = max_items + (1 if cfg.shared_intermediate else 0)
    if items_bound * H * (I // 2 + 4 * (I // g)) > (16 << 20):
        return 0
    wgs = ((max_items * (I // 2) + 3) // 4 + 7) // 8 * 8
    if wgs >= 768:
        return 0
    items = unique_experts + (1 if cfg.shared_intermediate else 0)
    return items * H * (I // 2 + 4 * (I // g))

