"""ctypes front end of the CPU oracle (TEST INFRASTRUCTURE, not product code).

Loads ``oracle/liboracle_pbmoe.so`` (built by ``oracle/Makefile``), a plain-C
restatement of the reference's CPU arithmetic for the FlashMoE MoE block.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module; the product path never does.

Each wrapper names the reference function it restates (paths relative to
``src/inference/flashmoe/`` of Jc2k/pb).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_pbmoe.so")

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
DT_Q4 = 3  # a Q4 shared gate row in moe_block (shared_gate_w = (codes, scales, biases, group, sb_dtype))
ORDER_CANONICAL, ORDER_REFERENCE_SLOT = 0, 1
NORM_RENORMALIZE, NORM_DEEPSEEK_FLOOR, NORM_PRESERVE_FULL = 0, 1, 2
ROUTING_SOFTMAX, ROUTING_SIGMOID_NOAUX, ROUTING_SIGMOID_GROUPED, ROUTING_SQRT_SOFTPLUS = 0, 1, 2, 3

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        _lib = C.CDLL(LIB_PATH)
    return _lib


def _p(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def router_logits(w: np.ndarray, x: np.ndarray, dtype: int = DT_F16) -> np.ndarray:
    """weights/store.rs:880-897 — sequential mul-then-add per expert row."""
    w = np.ascontiguousarray(w)
    x = _f32(x)
    experts, hidden = w.shape
    out = np.empty(experts, np.float32)
    lib().or_router_logits(_p(w), C.c_int(dtype), _p(x), C.c_int(experts), C.c_int(hidden), _p(out))
    return out


def router_logits_mt(w: np.ndarray, x: np.ndarray, dtype: int = DT_F16, threads: int = 1) -> np.ndarray:
    """router_logits with the rows split over OpenMP threads (bitwise equal)."""
    w = np.ascontiguousarray(w)
    x = _f32(x)
    experts, hidden = w.shape
    out = np.empty(experts, np.float32)
    lib().or_router_logits_mt(_p(w), C.c_int(dtype), _p(x), C.c_int(experts), C.c_int(hidden), _p(out),
                              C.c_int(threads))
    return out


def routing_top_k(scores, k: int):
    """math.rs:746-769 — replacement-slot scan, slot order."""
    s = _f32(scores)
    ids = np.empty(max(k, 1), np.int32)
    vals = np.empty(max(k, 1), np.float32)
    n = lib().or_routing_top_k(_p(s), C.c_int(s.size), C.c_int(k), _p(ids), _p(vals))
    return ids[:n].tolist(), vals[:n].tolist()


def top_k_sorted(scores, k: int):
    """math.rs:710-726 — stable sort, score desc then index asc."""
    s = _f32(scores)
    ids = np.empty(max(k, 1), np.int32)
    vals = np.empty(max(k, 1), np.float32)
    n = lib().or_top_k_sorted(_p(s), C.c_int(s.size), C.c_int(k), _p(ids), _p(vals))
    return ids[:n].tolist(), vals[:n].tolist()


def softmax_in_place(values) -> np.ndarray:
    """math.rs:728-744."""
    v = _f32(values).copy()
    lib().or_softmax_in_place(_p(v), C.c_int(v.size))
    return v


def routing_softmax_top_k(logits, k: int, order: int = ORDER_REFERENCE_SLOT):
    """math.rs:771-783."""
    s = _f32(logits)
    ids = np.empty(max(k, 1), np.int32)
    p = np.empty(max(k, 1), np.float32)
    n = lib().or_routing_softmax_top_k(_p(s), C.c_int(s.size), C.c_int(k), C.c_int(order), _p(ids), _p(p))
    return ids[:n].tolist(), p[:n].copy()


def routing_sigmoid_noaux_top_k(logits, bias, k: int, order: int = ORDER_REFERENCE_SLOT):
    """math.rs:788-819."""
    s = _f32(logits)
    b = _f32(bias)
    assert s.size == b.size
    ids = np.empty(max(k, 1), np.int32)
    w = np.empty(max(k, 1), np.float32)
    n = lib().or_routing_sigmoid_noaux_top_k(_p(s), _p(b), C.c_int(s.size), C.c_int(k), C.c_int(order), _p(ids), _p(w))
    return ids[:n].tolist(), w[:n].copy()


def sqrt_softplus(logits) -> np.ndarray:
    """deepseek_v4_router_probabilities (deepseek.rs:1300-1324), element-wise."""
    s = _f32(logits).ravel()
    out = np.empty_like(s)
    for i, v in enumerate(s):
        out[i] = lib().or_sqrt_softplus(C.c_float(float(v)))
    return out


def routing_sqrt_softplus_top_k(logits, bias, k: int):
    """deepseek_v4_router_probabilities + deepseek_v4_select_routes
    (deepseek.rs:1300-1394); bias None = no correction bias."""
    s = _f32(logits)
    b = _f32(bias) if bias is not None else None
    ids = np.empty(max(k, 1), np.int32)
    w = np.empty(max(k, 1), np.float32)
    n = lib().or_routing_sqrt_softplus_top_k(_p(s), _p(b) if b is not None else None, C.c_int(s.size), C.c_int(k),
                                             _p(ids), _p(w))
    if n < 0:
        raise ValueError("non-finite DeepSeek-V4 router input")
    return ids[:n].tolist(), w[:n].copy()


def routing_sigmoid_grouped_top_k(logits, bias, k: int, n_group: int, topk_group: int):
    """DeepSeek-V3 group-limited noaux routing.  No reference implementation
    exists: pinned by the n_group=1 reduction to math.rs:788-819 and by a
    brute-force restatement of the published definition.  The selection
    bias is required (e_score_correction_bias)."""
    if bias is None:
        raise ValueError("grouped sigmoid routing needs the selection bias")
    s = _f32(logits)
    b = _f32(bias)
    ids = np.empty(max(k, 1), np.int32)
    w = np.empty(max(k, 1), np.float32)
    n = lib().or_routing_sigmoid_grouped_top_k(_p(s), _p(b), C.c_int(s.size), C.c_int(k), C.c_int(n_group),
                                               C.c_int(topk_group), _p(ids), _p(w))
    if n < 0:
        raise ValueError("invalid grouped routing shape")
    return ids[:n].tolist(), w[:n].copy()


def renormalize(p, policy: int, routed_scale: float):
    """scheduler/expert_access.rs:80-135; returns (status, weights)."""
    pp = _f32(p)
    w = np.zeros(max(pp.size, 1), np.float32)
    rc = lib().or_renormalize(_p(pp), C.c_int(pp.size), C.c_int(policy), C.c_float(routed_scale), _p(w))
    return rc, w[: pp.size].copy()


def validate_preselected(ids, scores, active_experts: int, experts: int) -> int:
    """scheduler/protocol.rs:1044-1081; 0 = ok."""
    i = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
    s = _f32(scores)
    return lib().or_validate_preselected(_p(i), _p(s), C.c_int(i.size), C.c_int(active_experts), C.c_int(experts))


def q4_dequantize_rows(packed, scales, biases, rows: int, cols: int, group: int, sb_dtype: int = DT_F32):
    """math.rs:913-954 — w = fma(q, s, b)."""
    pk = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    sc, bi = _sb(scales, sb_dtype), _sb(biases, sb_dtype)
    out = np.empty(rows * cols, np.float32)
    rc = lib().or_q4_dequantize_rows(_p(pk), _p(sc), _p(bi), C.c_int(sb_dtype), C.c_int(rows), C.c_int(cols),
                                     C.c_int(group), _p(out))
    assert rc == 0
    return out.reshape(rows, cols)


def _sb(a, dtype):
    if dtype == DT_F32:
        return _f32(a)
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint16))


def q4_fma_matvec(packed, x, scales, biases, rows: int, cols: int, group: int, sb_dtype: int = DT_F32):
    """math.rs:861-911 — acc += fma(q, s*x, b*x)."""
    pk = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    sc, bi = _sb(scales, sb_dtype), _sb(biases, sb_dtype)
    xx = _f32(x)
    out = np.empty(rows, np.float32)
    rc = lib().or_q4_fma_matvec(_p(pk), _p(xx), _p(sc), _p(bi), C.c_int(sb_dtype), C.c_int(rows), C.c_int(cols),
                                C.c_int(group), _p(out))
    assert rc == 0
    return out


def router_logits_q4(packed, scales, biases, x, experts: int, hidden: int, group: int,
                     sb_dtype: int = DT_F16) -> np.ndarray:
    """Logits [T][experts] of a Q4 router: the resident Q4 projection
    (ResidentMmapMatvecProjection::Q4, metal/projection.rs:232-259, kernel
    q4_mmap_fma_matvec[_bf16_scale_bias], shaders.metal:488-660) in the
    arithmetic of math.rs:861-911 (q4_fma_matvec) for every token row."""
    xx = np.atleast_2d(_f32(x))
    return np.stack([q4_fma_matvec(packed, xx[t], scales, biases, experts, hidden, group, sb_dtype)
                     for t in range(xx.shape[0])])


class _Q4Rows(C.Structure):
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p), ("group", C.c_int),
                ("sb_dtype", C.c_int)]


def q4_explicit_matvec(packed, x, scales, biases, rows: int, cols: int, group: int, sb_dtype: int = DT_F32):
    """tests/scheduler.rs:308-325 — sum of (q*s+b)*x."""
    pk = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    sc, bi = _sb(scales, sb_dtype), _sb(biases, sb_dtype)
    xx = _f32(x)
    out = np.empty(rows, np.float32)
    lib().or_q4_explicit_matvec(_p(pk), _p(xx), _p(sc), _p(bi), C.c_int(sb_dtype), C.c_int(rows), C.c_int(cols),
                                C.c_int(group), _p(out))
    return out


def swiglu(g, u) -> np.ndarray:
    gg, uu = _f32(g), _f32(u)
    out = np.empty_like(gg)
    lib().or_swiglu(_p(gg), _p(uu), C.c_int(gg.size), _p(out))
    return out


def rms_norm(x, w=None, eps: float = 1e-6) -> np.ndarray:
    """math.rs:147-167."""
    xx = _f32(x)
    out = np.empty_like(xx)
    ww = _f32(w) if w is not None else None
    lib().or_rms_norm(_p(xx), _p(ww) if ww is not None else None, C.c_int(xx.size), C.c_float(eps), _p(out))
    return out


def layer_major_union(ids: np.ndarray, experts: int):
    """scheduler/mod.rs:685-769 — sorted unique union + route slots."""
    i = np.ascontiguousarray(ids, dtype=np.int32)
    rows, k = i.shape
    uniq = np.empty(experts, np.int32)
    cnt = C.c_int(0)
    slots = np.empty(rows * k, np.int32)
    rc = lib().or_layer_major_union(_p(i), C.c_int(rows), C.c_int(k), C.c_int(experts), _p(uniq), C.byref(cnt),
                                    _p(slots))
    if rc:
        raise ValueError(f"union failed: {rc}")
    return uniq[: cnt.value].copy(), slots


def group_plan(route_slots, unique: int, active: int):
    """metal/mod.rs:3197-3233 — returns (src_rows, out_idx, groups) or raises."""
    rs = np.ascontiguousarray(np.asarray(route_slots, dtype=np.int32))
    src = np.empty(max(rs.size, 1), np.uint32)
    out = np.empty(max(rs.size, 1), np.uint32)
    groups = np.empty(max(2 * unique, 2), np.uint32)
    rc = lib().or_group_plan(_p(rs), C.c_int(rs.size), C.c_int(unique), C.c_int(active), _p(src), _p(out),
                             _p(groups))
    if rc:
        raise ValueError(f"group plan rejected: {rc}")
    return src[: rs.size].copy(), out[: rs.size].copy(), [tuple(g) for g in groups[: 2 * unique].reshape(-1, 2).tolist()]


class Q4Layout(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32),
        ("intermediate", C.c_uint32),
        ("group_size", C.c_uint32),
        ("sb_dtype", C.c_uint32),
        ("expert_bytes", C.c_uint64),
        ("offset", C.c_uint64 * 9),
    ]


def make_layout(hidden: int, intermediate: int, group: int, sb_dtype: int, offsets, expert_bytes: int) -> Q4Layout:
    lay = Q4Layout()
    lay.hidden, lay.intermediate, lay.group_size, lay.sb_dtype = hidden, intermediate, group, sb_dtype
    lay.expert_bytes = expert_bytes
    for i, o in enumerate(offsets):
        lay.offset[i] = int(o)
    return lay


def expert_mlp(layout: Q4Layout, slot: np.ndarray, x) -> np.ndarray:
    """One expert's Q4 SwiGLU chain (reference_q4_swiglu, tests/scheduler.rs:327-336)."""
    xx = _f32(x)
    y = np.empty(layout.hidden, np.float32)
    rc = lib().or_expert_mlp(C.byref(layout), _p(np.ascontiguousarray(slot)), _p(xx), _p(y))
    assert rc == 0
    return y


def combine(residual, ys, weights, shared=None, shared_weight: float = 0.0) -> np.ndarray:
    """qwen_layer_major_combine for one row (shaders.metal:1756-1786)."""
    r = _f32(residual)
    y = _f32(ys)
    w = _f32(weights)
    s = _f32(shared) if shared is not None else None
    out = np.empty_like(r)
    lib().or_combine(_p(r), _p(y), _p(w), C.c_int(w.size), _p(s) if s is not None else None,
                     C.c_float(shared_weight), C.c_int(r.size), _p(out))
    return out


def _gate_arg(shared_gate_w, shared_gate_dtype: int):
    """The shared-gate argument of or_moe_block[_f64]: a dense row, or for
    DT_Q4 a (codes, scales, biases, group, sb_dtype) tuple passed as an
    or_q4_rows struct; plus the arrays it points into (kept alive)."""
    if shared_gate_w is None:
        return None, []
    if shared_gate_dtype == DT_Q4:
        codes, scales, biases, group, sbt = shared_gate_w
        keep = [np.ascontiguousarray(codes, dtype=np.uint8), _sb(scales, sbt), _sb(biases, sbt)]
        q = _Q4Rows(keep[0].ctypes.data, keep[1].ctypes.data, keep[2].ctypes.data, group, sbt)
        keep.append(q)
        return C.byref(q), keep
    keep = [np.ascontiguousarray(shared_gate_w)]
    return _p(keep[0]), keep


def moe_block(layout: Q4Layout, slots: np.ndarray, experts: int, x: np.ndarray, residual: np.ndarray,
              ids: np.ndarray, weights: np.ndarray, shared_layout: Q4Layout | None = None,
              shared_slot: np.ndarray | None = None, shared_gate_w: np.ndarray | None = None,
              shared_gate_dtype: int = DT_F16, next_norm_w: np.ndarray | None = None, eps: float = 1e-6,
              threads: int = 1):
    """CMD3 per-row arithmetic (metal/mod.rs:4289-4765, shaders.metal:1756-1786).
    Returns (hidden[T][H], next_normed[T][H] or None)."""
    xx = _f32(x)
    rr = _f32(residual)
    rows, hidden = xx.shape
    ii = np.ascontiguousarray(ids, dtype=np.int32)
    ww = _f32(weights)
    k = ii.shape[1]
    out = np.empty((rows, hidden), np.float32)
    nn = np.empty((rows, hidden), np.float32) if next_norm_w is not None else None
    nw = _f32(next_norm_w) if next_norm_w is not None else None
    gate_arg, keep = _gate_arg(shared_gate_w, shared_gate_dtype)
    rc = lib().or_moe_block(
        C.byref(layout), _p(slots), C.c_int(experts),
        C.byref(shared_layout) if shared_layout is not None else None,
        _p(shared_slot) if shared_slot is not None else None,
        gate_arg, C.c_int(shared_gate_dtype),
        _p(xx), _p(rr), C.c_int(rows), C.c_int(k), _p(ii), _p(ww),
        _p(nw) if nw is not None else None, C.c_float(eps), _p(out),
        _p(nn) if nn is not None else None, C.c_int(threads))
    if rc:
        raise ValueError(f"oracle moe_block failed: {rc}")
    return out, nn


def moe_block_f64(layout: Q4Layout, slots: np.ndarray, experts: int, x: np.ndarray, residual: np.ndarray,
                  ids: np.ndarray, weights: np.ndarray, shared_layout: Q4Layout | None = None,
                  shared_slot: np.ndarray | None = None, shared_gate_w: np.ndarray | None = None,
                  shared_gate_dtype: int = DT_F16, threads: int = 1) -> np.ndarray:
    """fp64 evaluation of the block (the exact value the f32 paths round);
    the shared gate as for moe_block (dense row, or a DT_Q4 tuple)."""
    xx = _f32(x)
    rr = _f32(residual)
    rows, hidden = xx.shape
    ii = np.ascontiguousarray(ids, dtype=np.int32)
    ww = _f32(weights)
    out = np.empty((rows, hidden), np.float64)
    gate_arg, keep = _gate_arg(shared_gate_w, shared_gate_dtype)
    rc = lib().or_moe_block_f64(
        C.byref(layout), _p(slots), C.c_int(experts),
        C.byref(shared_layout) if shared_layout is not None else None,
        _p(shared_slot) if shared_slot is not None else None,
        gate_arg, C.c_int(shared_gate_dtype),
        _p(xx), _p(rr), C.c_int(rows), C.c_int(ii.shape[1]), _p(ii), _p(ww), _p(out), C.c_int(threads))
    if rc:
        raise ValueError(f"oracle moe_block_f64 failed: {rc}")
    return out


def route_rows(logits: np.ndarray, k: int, kind: int = ROUTING_SOFTMAX, order: int = ORDER_REFERENCE_SLOT,
               bias: np.ndarray | None = None, n_group: int = 1, topk_group: int = 1,
               policy: int = NORM_RENORMALIZE, routed_scale: float = 1.0):
    """Routing stage for T rows: selection (math.rs:771-819) then
    renormalisation (expert_access.rs:80-135)."""
    ll = _f32(logits)
    rows, experts = ll.shape
    bb = _f32(bias) if bias is not None else np.zeros(experts, np.float32)
    ids = np.empty((rows, k), np.int32)
    w = np.empty((rows, k), np.float32)
    rc = lib().or_route_rows(_p(ll), _p(bb), C.c_int(rows), C.c_int(experts), C.c_int(k), C.c_int(kind),
                             C.c_int(order), C.c_int(n_group), C.c_int(topk_group), C.c_int(policy),
                             C.c_float(routed_scale), _p(ids), _p(w))
    if rc:
        raise ValueError(f"oracle routing failed: {rc}")
    return ids, w


# ---- GQA attention of the decode stack ----------------------------------------

def qk_norm_rope(values, heads: int, head_dim: int, weight, position: int, rotary_dim: int,
                 theta: float) -> np.ndarray:
    """apply_optional_per_head_rms_norm_and_split_half_rope (math.rs:252-325)."""
    v = _f32(values).copy()
    w = _f32(weight) if weight is not None else None
    lib().or_qk_norm_rope(_p(v), C.c_int(heads), C.c_int(head_dim), _p(w) if w is not None else None,
                          C.c_int(position), C.c_int(rotary_dim), C.c_float(theta))
    return v


def causal_attention(q, keys, values, q_heads: int, kv_heads: int, head_dim: int) -> np.ndarray:
    """causal_attention (math.rs:671-707); keys/values [n][kv_heads*head_dim]."""
    qq, kk, vv = _f32(q), _f32(keys), _f32(values)
    n = kk.size // (kv_heads * head_dim) if kv_heads * head_dim else 0
    out = np.zeros(q_heads * head_dim, np.float32)
    lib().or_causal_attention(_p(qq), _p(kk), _p(vv), C.c_int(n), C.c_int(q_heads), C.c_int(kv_heads),
                              C.c_int(head_dim), _p(out))
    return out


class AttnOracle:
    """One attention layer of the decode stack with its own f32 copy of the
    f16 KV cache (or_attention_decode: runtime/mod.rs:2215-2367 + o_proj).
    mats: dict q/k/v/o -> (codes u8, scales u16, biases u16)."""

    def __init__(self, mats: dict, q_norm, k_norm, hidden: int, q_heads: int, kv_heads: int,
                 head_dim: int, theta: float, group: int, sb_dtype: int, max_context: int):
        self.mats = {k: tuple(np.ascontiguousarray(a) for a in v) for k, v in mats.items()}
        self.q_norm, self.k_norm = _f32(q_norm), _f32(k_norm)
        self.H, self.qh, self.kvh, self.hd = hidden, q_heads, kv_heads, head_dim
        self.theta, self.group, self.sb = theta, group, sb_dtype
        self.cache_k = np.zeros((max_context, kv_heads * head_dim), np.float32)
        self.cache_v = np.zeros((max_context, kv_heads * head_dim), np.float32)

    def decode(self, normed, position: int):
        """Returns (attention values [q_heads*head_dim], o [H])."""
        order = ("q", "k", "v", "o")
        codes = (C.c_void_p * 4)(*[self.mats[n][0].ctypes.data for n in order])
        scales = (C.c_void_p * 4)(*[self.mats[n][1].ctypes.data for n in order])
        biases = (C.c_void_p * 4)(*[self.mats[n][2].ctypes.data for n in order])
        x = _f32(normed)
        att = np.zeros(self.qh * self.hd, np.float32)
        o = np.zeros(self.H, np.float32)
        rc = lib().or_attention_decode(codes, scales, biases, C.c_int(self.sb), C.c_int(self.group),
                                       _p(self.q_norm), _p(self.k_norm), C.c_int(self.H), C.c_int(self.qh),
                                       C.c_int(self.kvh), C.c_int(self.hd), C.c_int(self.hd),
                                       C.c_float(self.theta), C.c_int(position), _p(x), _p(self.cache_k),
                                       _p(self.cache_v), _p(att), _p(o))
        if rc != 0:
            raise RuntimeError(f"or_attention_decode failed ({rc})")
        return att, o


def _declare():
    L = lib()
    L.or_routing_top_k.restype = C.c_int
    L.or_top_k_sorted.restype = C.c_int
    L.or_routing_softmax_top_k.restype = C.c_int
    L.or_routing_sigmoid_noaux_top_k.restype = C.c_int
    L.or_routing_sigmoid_grouped_top_k.restype = C.c_int
    L.or_routing_sqrt_softplus_top_k.restype = C.c_int
    L.or_sqrt_softplus.restype = C.c_float
    L.or_sqrt_softplus.argtypes = [C.c_float]
    L.or_renormalize.restype = C.c_int


if os.path.exists(LIB_PATH):
    _declare()
