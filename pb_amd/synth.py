"""Seeded synthetic MoE layers (host side), shared by tests and the benchmark.

Wraps ``libpbmoe_synth.so`` (pb_amd/csrc/synth_host.c).  Q4 expert bytes are
identical to the device fill kernel's (``pbmoe_synth_fill_q4``); normal draws
are produced on the host only.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpbmoe_synth.so")

T_EXPERT, T_ROUTER, T_SHARED, T_SHARED_GATE, T_INPUT, T_RESIDUAL, T_ROUTER_BIAS, T_LOGITS = range(1, 9)
# attention layer of the decode stack: q and o share one pseudo slot (gate =
# W_q, down = W_o), k and v another (gate = W_k, up = W_v); norm weights
T_ATTN_QO, T_ATTN_KV, T_ATTN_NORM, T_LAYER_NORM, T_KV_FILL = range(9, 14)
T_ROUTER_Q4, T_SHARED_GATE_Q4 = 14, 15

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"synth library missing: {LIB_PATH}; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        L.pbm_fill_q4_experts.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                          C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint64, C.c_void_p,
                                          C.c_int]
        L.pbm_fill_normal_f16.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64,
                                          C.c_double, C.c_void_p, C.c_int]
        L.pbm_f16_to_f32_array.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p]
        L.pbm_f32_to_f16_array.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p]
        L.pbm_f32_to_bf16_array.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p]
        L.pbm_fill_uniform_f32.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64,
                                           C.c_float, C.c_float, C.c_void_p]
        L.pbm_drawn_logits_zipf.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_double,
                                            C.c_void_p, C.c_void_p]
        L.pbm_drawn_logits_zipf.restype = C.c_int
        _lib = L
    return _lib


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def q4_experts(seed: int, tensor: int, layer: int, first: int, count: int, hidden: int, intermediate: int,
               group: int, sb_dtype: int, offsets, expert_bytes: int) -> np.ndarray:
    """`count` fixed-slot Q4 experts back to back (uint8)."""
    out = np.empty(count * expert_bytes, np.uint8)
    off = np.ascontiguousarray(np.asarray(offsets, dtype=np.uint64))
    lib().pbm_fill_q4_experts(seed, tensor, layer, first, count, hidden, intermediate, group, sb_dtype,
                              off.ctypes.data, expert_bytes, out.ctypes.data, _threads())
    return out


def normal_f16(seed: int, tensor: int, layer: int, expert: int, part: int, n: int, sigma: float) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().pbm_fill_normal_f16(seed, tensor, layer, expert, part, n, sigma, out.ctypes.data, _threads())
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().pbm_f16_to_f32_array(h.ctypes.data, h.size, out.ctypes.data)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().pbm_f32_to_f16_array(f.ctypes.data, f.size, out.ctypes.data)
    return out


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().pbm_f32_to_bf16_array(f.ctypes.data, f.size, out.ctypes.data)
    return out


def uniform_f32(seed: int, tensor: int, layer: int, expert: int, part: int, n: int, lo: float, width: float):
    out = np.empty(n, np.float32)
    lib().pbm_fill_uniform_f32(seed, tensor, layer, expert, part, n, lo, width, out.ctypes.data)
    return out


def drawn_logits_zipf(seed: int, layer: int, tokens: int, experts: int, k: int, s: float = 1.1):
    """Prefill router logits with a Zipf(s) expert load; returns (logits, hist)."""
    logits = np.empty((tokens, experts), np.float32)
    hist = np.empty(experts, np.uint32)
    rc = lib().pbm_drawn_logits_zipf(seed, layer, tokens, experts, k, s, logits.ctypes.data, hist.ctypes.data)
    if rc:
        raise ValueError("invalid zipf logits request")
    return logits, hist


@dataclass
class MoeConfig:
    """One benchmark workload shape (see configs in pb_amd.configs)."""
    name: str
    hidden: int
    intermediate: int
    experts: int
    k: int
    routing: int = 0            # pbmoe_routing
    normalization: int = 0      # pbmoe_normalization
    routed_scale: float = 1.0
    n_group: int = 1
    topk_group: int = 1
    shared_intermediate: int = 0
    shared_gated: bool = False
    group: int = 64
    sb_dtype: int = 1           # f16 scale/bias (benchmark shapes); 2 = bf16 (reference artifacts)
    tokens: int = 1


@dataclass
class HostLayer:
    """Host arrays of one seeded layer."""
    cfg: MoeConfig
    layer: int
    layout: object
    slots: np.ndarray
    router_f16: np.ndarray           # [E][H] uint16 (f16 bits)
    selection_bias: np.ndarray | None
    shared_layout: object | None = None
    shared_slot: np.ndarray | None = None
    shared_gate_f16: np.ndarray | None = None
    extra: dict = field(default_factory=dict)


def make_layer(cfg: MoeConfig, seed: int, layer: int, layout_fn, with_slots: bool = True) -> HostLayer:
    """Generate a full layer on the host.  layout_fn(hidden, inter, group, dtype)
    returns a layout object with ``offsets`` and ``expert_bytes``."""
    H, I, E = cfg.hidden, cfg.intermediate, cfg.experts
    lay = layout_fn(H, I, cfg.group, cfg.sb_dtype)
    slots = (q4_experts(seed, T_EXPERT, layer, 0, E, H, I, cfg.group, cfg.sb_dtype, lay.offsets,
                        int(lay.expert_bytes)) if with_slots else np.empty(0, np.uint8))
    router = normal_f16(seed, T_ROUTER, layer, 0, 0, E * H, 0.02).reshape(E, H)
    bias = None
    if cfg.routing != 0:
        bias = uniform_f32(seed, T_ROUTER_BIAS, layer, 0, 0, E, -0.05, 0.1)
    hl = HostLayer(cfg, layer, lay, slots, router, bias)
    if cfg.shared_intermediate:
        sl = layout_fn(H, cfg.shared_intermediate, cfg.group, cfg.sb_dtype)
        hl.shared_layout = sl
        hl.shared_slot = q4_experts(seed, T_SHARED, layer, 0, 1, H, cfg.shared_intermediate, cfg.group,
                                    cfg.sb_dtype, sl.offsets, int(sl.expert_bytes))
        if cfg.shared_gated:
            hl.shared_gate_f16 = normal_f16(seed, T_SHARED_GATE, layer, 0, 0, H, 0.02).reshape(1, H)
    return hl


def activations(seed: int, layer: int, tokens: int, hidden: int):
    """x and residual [tokens][hidden]: f16 N(0,1) draws widened to f32."""
    x = f16_to_f32(normal_f16(seed, T_INPUT, layer, 0, 0, tokens * hidden, 1.0)).reshape(tokens, hidden)
    r = f16_to_f32(normal_f16(seed, T_RESIDUAL, layer, 0, 0, tokens * hidden, 1.0)).reshape(tokens, hidden)
    return x, r


@dataclass
class AttnConfig:
    """The GQA attention layer before each MoE block of the decode stack
    (workload C4: 32 q heads, 4 kv heads, head_dim 128, f16 KV
    cache, RMSNorm eps 1e-6, RoPE theta 1e6, Q4 projections)."""
    name: str
    hidden: int
    q_heads: int
    kv_heads: int
    head_dim: int = 128
    rope_theta: float = 1e6
    group: int = 64
    sb_dtype: int = 1
    max_context: int = 4096
    eps: float = 1e-6

    @property
    def q_width(self) -> int:
        return self.q_heads * self.head_dim

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim


def attn_pseudo_layouts(acfg: AttnConfig, layout_fn):
    """(q/o layout, k/v layout): fixed Q4 slots whose gate/down (resp.
    gate/up) projections hold W_q/W_o (resp. W_k/W_v)."""
    return (layout_fn(acfg.hidden, acfg.q_width, acfg.group, acfg.sb_dtype),
            layout_fn(acfg.hidden, acfg.kv_width, acfg.group, acfg.sb_dtype))


def attn_norms(acfg: AttnConfig, seed: int, layer: int):
    """q_norm, k_norm [head_dim] ~ U(0.5, 1.5); input and post-attention
    RMSNorm weights [hidden] ~ U(0.5, 1.5) (f32)."""
    hd, H = acfg.head_dim, acfg.hidden
    return (uniform_f32(seed, T_ATTN_NORM, layer, 0, 0, hd, 0.5, 1.0),
            uniform_f32(seed, T_ATTN_NORM, layer, 0, 1, hd, 0.5, 1.0),
            uniform_f32(seed, T_LAYER_NORM, layer, 0, 0, H, 0.5, 1.0),
            uniform_f32(seed, T_LAYER_NORM, layer, 0, 1, H, 0.5, 1.0))


def attn_host_mats(acfg: AttnConfig, seed: int, layer: int, layout_fn) -> dict:
    """W_q, W_k, W_v, W_o as (codes u8, scales u16, biases u16): the seeded
    Q4 generator's codes and scales over two pseudo slots, biases centred so
    that every weight row has mean ~0 (the activations of a decoder layer
    then stay O(1-10), as in a trained model)."""
    lqo, lkv = attn_pseudo_layouts(acfg, layout_fn)
    H = acfg.hidden
    qo = q4_experts(seed, T_ATTN_QO, layer, 0, 1, H, acfg.q_width, acfg.group, acfg.sb_dtype, lqo.offsets,
                    int(lqo.expert_bytes))
    kv = q4_experts(seed, T_ATTN_KV, layer, 0, 1, H, acfg.kv_width, acfg.group, acfg.sb_dtype, lkv.offsets,
                    int(lkv.expert_bytes))

    def part(slot, lay, comp):
        c = lay.components[comp]
        return slot[int(c.offset):int(c.offset) + int(c.bytes)]

    def mat(slot, lay, first):
        # zero-mean weights, as an affine quantisation of zero-mean tensors
        # gives: bias' = bias - 7.5 scale (codes uniform over 0..15)
        scales = part(slot, lay, first + 1).view(np.uint16).copy()
        biases = part(slot, lay, first + 2).view(np.uint16)
        return part(slot, lay, first).copy(), scales, centred_bias(biases, scales, acfg.sb_dtype)

    return {"q": mat(qo, lqo, 0), "o": mat(qo, lqo, 6), "k": mat(kv, lkv, 0), "v": mat(kv, lkv, 3)}


def q4_matrix(seed: int, tensor: int, layer: int, rows: int, cols: int, group: int, sb_dtype: int, layout_fn):
    """A Q4 matrix [rows][cols] as (codes u8 [rows*cols/2], scales u16,
    biases u16 [rows][cols/group]): the gate projection of one seeded pseudo
    slot (rows rounded up to the group), biases centred as for the attention
    matrices.  Used for a Q4 router and a Q4 shared-expert gate row."""
    pad = -(-rows // group) * group
    lay = layout_fn(cols, pad, group, sb_dtype)
    slot = q4_experts(seed, tensor, layer, 0, 1, cols, pad, group, sb_dtype, lay.offsets, int(lay.expert_bytes))

    def part(comp):
        c = lay.components[comp]
        return slot[int(c.offset):int(c.offset) + int(c.bytes)]

    codes = part(0)[:rows * cols // 2].copy()
    scales = part(1).view(np.uint16)[:rows * (cols // group)].copy()
    biases = part(2).view(np.uint16)[:rows * (cols // group)]
    return codes, scales, centred_bias(biases, scales, sb_dtype)


def _sb_to_f32(a: np.ndarray, sb_dtype: int) -> np.ndarray:
    if sb_dtype == 2:
        return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)
    return f16_to_f32(a)


def centred_bias(biases: np.ndarray, scales: np.ndarray, sb_dtype: int) -> np.ndarray:
    """bias - 7.5 scale rounded to the scale/bias dtype (7.5 scale is exact
    in f32): the host mirror of pbmoe_synth_center_q4."""
    v = _sb_to_f32(biases, sb_dtype) - np.float32(7.5) * _sb_to_f32(scales, sb_dtype)
    return f32_to_bf16(v) if sb_dtype == 2 else f32_to_f16(v)


def center_q4_slots(slots: np.ndarray, lay, count: int, sb_dtype: int) -> np.ndarray:
    """Copy of `count` fixed Q4 slots with every projection's biases centred
    (pbmoe_synth_center_q4 on the host)."""
    out = np.array(slots, dtype=np.uint8, copy=True)
    stride = int(lay.expert_bytes)
    for e in range(count):
        for p in range(3):
            cs, cb = lay.components[3 * p + 1], lay.components[3 * p + 2]
            so, bo = e * stride + int(cs.offset), e * stride + int(cb.offset)
            sc = out[so:so + int(cs.bytes)].view(np.uint16)
            bi = out[bo:bo + int(cb.bytes)].view(np.uint16)
            bi[:] = centred_bias(bi, sc, sb_dtype)
    return out

