"""Host-side mirror of the reference's MoE operator seam, over the C ABI.

The reference drives the MoE block through ``MetalExecutionFacade``
(src/inference/flashmoe/runtime/mod.rs:648-1410): a router prep whose logits
feed the CPU top-k (metal/mod.rs:2864-3036), ``submit_scheduled_expert_command``
for decode CMD3 (runtime/mod.rs:922-961) and ``qwen_layer_major_experts`` for
layer-major prefill (runtime/mod.rs:1151-1161).  ``MoeLayer`` keeps those
operations and their argument meaning; each call goes straight to
libpbmoe.so on the device.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import abi
from .abi import Context, DeviceArray, LayerDesc, check, lib
from .synth import HostLayer, MoeConfig


def layer_desc(cfg: MoeConfig, route_order: int = abi.ORDER_CANONICAL) -> LayerDesc:
    d = LayerDesc()
    d.hidden, d.intermediate, d.experts, d.active_experts = cfg.hidden, cfg.intermediate, cfg.experts, cfg.k
    d.routing, d.normalization, d.route_order = cfg.routing, cfg.normalization, route_order
    d.routed_scale = cfg.routed_scale
    d.n_group, d.topk_group = cfg.n_group, cfg.topk_group
    d.shared_intermediate = cfg.shared_intermediate
    d.shared_gated = 1 if cfg.shared_gated else 0
    d.norm_epsilon = 1e-6
    return d


class MoeLayer:
    """One bound MoE layer (resident experts, router, optional shared expert)."""

    def __init__(self, ctx: Context, index: int, cfg: MoeConfig, layout, route_order: int = abi.ORDER_CANONICAL):
        self.ctx, self.index, self.cfg, self.layout = ctx, index, cfg, layout
        self.desc = layer_desc(cfg, route_order)
        self._keep: list = []

    # -- residency (prepare_resident_expert_backing, metal/mod.rs:1382-1402) --
    def bind_host(self, host: HostLayer) -> "MoeLayer":
        cfg = self.cfg
        check(lib().pbmoe_bind_layer(self.ctx.handle, self.index, C.byref(self.desc), C.byref(self.layout),
                                     host.slots.ctypes.data, host.slots.nbytes, abi.MEM_HOST))
        bias = host.selection_bias
        check(lib().pbmoe_bind_router(self.ctx.handle, self.index, host.router_f16.ctypes.data, abi.DTYPE_F16,
                                      bias.ctypes.data if bias is not None else None, abi.MEM_HOST))
        if cfg.shared_intermediate:
            g = host.shared_gate_f16
            check(lib().pbmoe_bind_shared(self.ctx.handle, self.index, C.byref(host.shared_layout),
                                          host.shared_slot.ctypes.data, g.ctypes.data if g is not None else None,
                                          abi.DTYPE_F16, abi.MEM_HOST))
        return self

    def bind_device(self, slots: DeviceArray, router: DeviceArray, selection_bias: DeviceArray | None = None,
                    shared_layout=None, shared_slot: DeviceArray | None = None,
                    shared_gate: DeviceArray | None = None) -> "MoeLayer":
        self._keep = [slots, router, selection_bias, shared_slot, shared_gate]
        check(lib().pbmoe_bind_layer(self.ctx.handle, self.index, C.byref(self.desc), C.byref(self.layout),
                                     slots.ptr, slots.nbytes, abi.MEM_DEVICE))
        check(lib().pbmoe_bind_router(self.ctx.handle, self.index, router.ptr, abi.DTYPE_F16,
                                      selection_bias.ptr if selection_bias is not None else None, abi.MEM_DEVICE))
        if shared_slot is not None:
            check(lib().pbmoe_bind_shared(self.ctx.handle, self.index, C.byref(shared_layout), shared_slot.ptr,
                                          shared_gate.ptr if shared_gate is not None else None, abi.DTYPE_F16,
                                          abi.MEM_DEVICE))
        return self

    def bind_file(self, root: str, file_layer: int, router: DeviceArray, selection_bias: DeviceArray | None = None,
                  shared_layout=None, shared_slot: DeviceArray | None = None,
                  shared_gate: DeviceArray | None = None) -> "MoeLayer":
        """Experts from root/layer_NN.bin + .json (pbmoe_bind_layer_file), the
        dense router and shared expert from device arrays."""
        self._keep = [router, selection_bias, shared_slot, shared_gate]
        check(lib().pbmoe_bind_layer_file(self.ctx.handle, self.index, C.byref(self.desc), C.byref(self.layout),
                                          str(root).encode(), file_layer))
        check(lib().pbmoe_bind_router(self.ctx.handle, self.index, router.ptr, abi.DTYPE_F16,
                                      selection_bias.ptr if selection_bias is not None else None, abi.MEM_DEVICE))
        if shared_slot is not None:
            check(lib().pbmoe_bind_shared(self.ctx.handle, self.index, C.byref(shared_layout), shared_slot.ptr,
                                          shared_gate.ptr if shared_gate is not None else None, abi.DTYPE_F16,
                                          abi.MEM_DEVICE))
        return self

    def bind_router_q4(self, codes: DeviceArray, scales: DeviceArray, biases: DeviceArray, group: int,
                       selection_bias: DeviceArray | None = None) -> "MoeLayer":
        """A resident Q4 router [experts][hidden] in place of the dense one
        (pbmoe_bind_router_q4; the Q4 arm of encode_resident_projection_rows,
        metal/projection.rs:232-259).  Scale/bias dtype = the experts'."""
        self._keep += [codes, scales, biases, selection_bias]
        m = abi.Q4Matrix()
        m.codes, m.scales, m.biases = codes.ptr, scales.ptr, biases.ptr
        check(lib().pbmoe_bind_router_q4(self.ctx.handle, self.index, C.byref(m), group, self.cfg.sb_dtype,
                                         selection_bias.ptr if selection_bias is not None else None,
                                         abi.MEM_DEVICE))
        return self

    def bind_shared_gate_q4(self, codes: DeviceArray, scales: DeviceArray, biases: DeviceArray,
                            group: int) -> "MoeLayer":
        """A resident Q4 shared-expert gate row [1][hidden] in place of the
        dense one given to the shared binding (pbmoe_bind_shared_gate_q4)."""
        self._keep += [codes, scales, biases]
        m = abi.Q4Matrix()
        m.codes, m.scales, m.biases = codes.ptr, scales.ptr, biases.ptr
        check(lib().pbmoe_bind_shared_gate_q4(self.ctx.handle, self.index, C.byref(m), group, self.cfg.sb_dtype,
                                              abi.MEM_DEVICE))
        return self

    def slots(self):
        """(device address, bytes) of the bound expert slots."""
        p, n = C.c_void_p(), C.c_size_t()
        check(lib().pbmoe_layer_slots(self.ctx.handle, self.index, C.byref(p), C.byref(n)))
        return p.value, n.value

    # -- router prep + routing stage (metal/mod.rs:2943-3013) ----------------
    def route(self, x: DeviceArray, ids: DeviceArray, weights: DeviceArray, logits: DeviceArray | None = None):
        tokens = x.shape[0]
        check(lib().pbmoe_route(self.ctx.handle, self.index, x.ptr, tokens, ids.ptr, weights.ptr,
                                logits.ptr if logits is not None else None))

    def route_logits(self, logits: DeviceArray, ids: DeviceArray, weights: DeviceArray):
        check(lib().pbmoe_route_logits(self.ctx.handle, self.index, logits.ptr, logits.shape[0], ids.ptr,
                                       weights.ptr))

    # -- CMD3 decode (submit_scheduled_expert_command) ------------------------
    def submit_scheduled_expert_command(self, x: DeviceArray, residual: DeviceArray, ids: DeviceArray,
                                        weights: DeviceArray, hidden_out: DeviceArray,
                                        next_norm: DeviceArray | None = None,
                                        next_normed: DeviceArray | None = None):
        check(lib().pbmoe_moe_decode(self.ctx.handle, self.index, x.ptr, residual.ptr, x.shape[0], ids.ptr,
                                     weights.ptr, next_norm.ptr if next_norm is not None else None, hidden_out.ptr,
                                     next_normed.ptr if next_normed is not None else None))

    # -- whole block: routing stage + CMD3 in one call ------------------------
    def forward(self, x: DeviceArray, residual: DeviceArray, hidden_out: DeviceArray,
                ids: DeviceArray | None = None, weights: DeviceArray | None = None,
                next_norm: DeviceArray | None = None, next_normed: DeviceArray | None = None):
        check(lib().pbmoe_moe_layer(self.ctx.handle, self.index, x.ptr, residual.ptr, x.shape[0],
                                    ids.ptr if ids is not None else None,
                                    weights.ptr if weights is not None else None,
                                    next_norm.ptr if next_norm is not None else None, hidden_out.ptr,
                                    next_normed.ptr if next_normed is not None else None))

    # -- whole block from the un-normalised hidden state (CMD2's fused
    #    post-attention RMSNorm, metal/mod.rs:2864-2917) --------------------
    def forward_norm(self, hidden: DeviceArray, norm_weight: DeviceArray, hidden_out: DeviceArray,
                     ids: DeviceArray | None = None, weights: DeviceArray | None = None,
                     next_norm: DeviceArray | None = None, next_normed: DeviceArray | None = None):
        check(lib().pbmoe_moe_layer_norm(self.ctx.handle, self.index, hidden.ptr, norm_weight.ptr,
                                         hidden.shape[0], ids.ptr if ids is not None else None,
                                         weights.ptr if weights is not None else None,
                                         next_norm.ptr if next_norm is not None else None, hidden_out.ptr,
                                         next_normed.ptr if next_normed is not None else None))

    # -- layer-major prefill (qwen_layer_major_experts) -----------------------
    def qwen_layer_major_experts(self, x: DeviceArray, residual: DeviceArray, ids: DeviceArray,
                                 weights: DeviceArray, hidden_out: DeviceArray,
                                 next_norm: DeviceArray | None = None, next_normed: DeviceArray | None = None):
        check(lib().pbmoe_moe_prefill(self.ctx.handle, self.index, x.ptr, residual.ptr, x.shape[0], ids.ptr,
                                      weights.ptr, next_norm.ptr if next_norm is not None else None,
                                      hidden_out.ptr, next_normed.ptr if next_normed is not None else None))

    def unbind(self):
        check(lib().pbmoe_unbind_layer(self.ctx.handle, self.index))


def dispatch_plan(ctx: Context, ids: DeviceArray, experts: int):
    """resolve_layer_major_experts + qwen_layer_major_group_plan on the device;
    returns host arrays (unique_ids, route_slots, src_rows, out_idx, groups)."""
    tokens, k = ids.shape
    n = tokens * k
    uniq = ctx.array(experts, np.uint32)
    cnt = ctx.array(1, np.uint32)
    slots = ctx.array(n, np.uint32)
    src = ctx.array(n, np.uint32)
    out = ctx.array(n, np.uint32)
    groups = ctx.array((experts, 2), np.uint32)
    check(lib().pbmoe_dispatch_plan(ctx.handle, experts, k, tokens, ids.ptr, uniq.ptr, cnt.ptr, slots.ptr, src.ptr,
                                    out.ptr, groups.ptr))
    ctx.sync()
    u = int(cnt.download()[0])
    return (uniq.download()[:u], slots.download(), src.download(), out.download(),
            [tuple(int(v) for v in g) for g in groups.download()[:u]])


class AttentionLayer:
    """One bound GQA attention layer of the decode stack with its KV cache:
    the reference's Qwen full-attention step (full_attention_output_values,
    runtime/mod.rs:2215-2367) followed by o_proj, the residual add and the
    post-attention RMSNorm (runtime/mod.rs:2979-2996)."""

    def __init__(self, ctx: Context, index: int, acfg):
        self.ctx, self.index, self.acfg = ctx, index, acfg
        d = abi.AttnDesc()
        d.hidden, d.q_heads, d.kv_heads, d.head_dim = acfg.hidden, acfg.q_heads, acfg.kv_heads, acfg.head_dim
        d.rotary_dim = acfg.head_dim
        d.rope_theta = acfg.rope_theta
        d.norm_epsilon = acfg.eps
        d.max_context = acfg.max_context
        d.group_size = acfg.group
        d.scale_bias_dtype = acfg.sb_dtype
        self.desc = d
        self._keep: list = []

    def bind_synth(self, seed: int, layer: int) -> "AttentionLayer":
        """Seeded Q4 projections (synth.attn_host_mats) and norm weights,
        uploaded to the device."""
        from . import synth
        mats = synth.attn_host_mats(self.acfg, seed, layer, abi.q4_layout_fixed)
        qn, kn, self.input_norm_h, self.post_norm_h = synth.attn_norms(self.acfg, seed, layer)
        return self.bind_host(mats, qn, kn)

    def bind_host(self, mats: dict, q_norm: np.ndarray, k_norm: np.ndarray) -> "AttentionLayer":
        """mats: q/k/v/o -> (codes u8, scales u16, biases u16) host arrays."""
        ctx = self.ctx
        keep = []
        w = abi.AttnWeights()
        for name in ("q", "k", "v", "o"):
            parts = [ctx.to_device(np.ascontiguousarray(a)) for a in mats[name]]
            keep += parts
            m = abi.Q4Matrix()
            m.codes, m.scales, m.biases = parts[0].ptr, parts[1].ptr, parts[2].ptr
            setattr(w, name, m)
        qn, kn = ctx.to_device(np.asarray(q_norm, np.float32)), ctx.to_device(np.asarray(k_norm, np.float32))
        keep += [qn, kn]
        w.q_norm, w.k_norm = qn.ptr, kn.ptr
        if getattr(self, "input_norm_h", None) is not None:
            self.input_norm, self.post_norm = ctx.to_device(self.input_norm_h), ctx.to_device(self.post_norm_h)
        self._keep = keep
        check(lib().pbmoe_bind_attention(ctx.handle, self.index, C.byref(self.desc), C.byref(w)))
        return self

    def kv_cache(self):
        k, v = C.c_void_p(), C.c_void_p()
        check(lib().pbmoe_attention_kv_cache(self.ctx.handle, self.index, C.byref(k), C.byref(v)))
        return k.value, v.value

    def decode(self, normed: DeviceArray, residual: DeviceArray, position: int, hidden_out: DeviceArray,
               post_norm: DeviceArray | None = None, post_normed: DeviceArray | None = None,
               attn_out: DeviceArray | None = None, input_norm: DeviceArray | None = None):
        """input_norm given: `normed` is the hidden state before input_layernorm."""
        check(lib().pbmoe_attention_decode(self.ctx.handle, self.index, normed.ptr,
                                           input_norm.ptr if input_norm is not None else None, residual.ptr,
                                           position, hidden_out.ptr,
                                           post_norm.ptr if post_norm is not None else None,
                                           post_normed.ptr if post_normed is not None else None,
                                           attn_out.ptr if attn_out is not None else None))

