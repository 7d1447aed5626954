"""ctypes binding of the C ABI in include/pbmoe.h (libpbmoe.so).

This is the same binding a Rust ``extern "C"`` crate makes; tests, smoke and
the benchmark drive the library only through it.  Loading fails loudly when
the native library is missing: there is no Python or CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpbmoe.so")

# pbmoe_status
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_SHAPE = 2
ERR_DTYPE = 3
ERR_ALIGNMENT = 4
ERR_ROUTE = 5
ERR_UNSUPPORTED = 6
ERR_DEVICE = 7
ERR_TIMEOUT = 8
ERR_NOT_BOUND = 9
ERR_OUT_OF_MEMORY = 10
ERR_NONFINITE = 11
ERR_IO = 12
ERR_FORMAT = 13

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
ROUTING_SOFTMAX_TOPK, ROUTING_SIGMOID_NOAUX, ROUTING_SIGMOID_GROUPED, ROUTING_SQRT_SOFTPLUS = 0, 1, 2, 3
NORM_RENORMALIZE_SELECTED, NORM_DEEPSEEK_FLOOR, NORM_PRESERVE_FULL_SOFTMAX = 0, 1, 2
ORDER_CANONICAL, ORDER_REFERENCE_SLOT = 0, 1
MEM_HOST, MEM_DEVICE = 0, 1


class PbmoeError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"pbmoe status {status}: {message}")
        self.status = status
        self.message = message


class Component(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("reserved", C.c_uint32), ("offset", C.c_uint64), ("bytes", C.c_uint64)]


class Q4Layout(C.Structure):
    _fields_ = [
        ("expert_bytes", C.c_uint64),
        ("group_size", C.c_uint32),
        ("scale_bias_dtype", C.c_uint32),
        ("components", Component * 9),
    ]

    @property
    def offsets(self) -> list[int]:
        return [int(c.offset) for c in self.components]


class LayerDesc(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32),
        ("intermediate", C.c_uint32),
        ("experts", C.c_uint32),
        ("active_experts", C.c_uint32),
        ("routing", C.c_uint32),
        ("normalization", C.c_uint32),
        ("route_order", C.c_uint32),
        ("routed_scale", C.c_float),
        ("n_group", C.c_uint32),
        ("topk_group", C.c_uint32),
        ("shared_intermediate", C.c_uint32),
        ("shared_gated", C.c_uint32),
        ("norm_epsilon", C.c_float),
    ]


_P = C.c_void_p
_U32 = C.c_uint32
class PackInfo(C.Structure):
    """pbmoe_pack_info: metadata of root/layer_NN.json."""
    _fields_ = [("format", C.c_char * 48), ("layer", C.c_uint32), ("experts", C.c_uint32),
                ("expert_size", C.c_uint64), ("file_bytes", C.c_uint64), ("packs", C.c_uint32),
                ("records", C.c_uint32)]


class AttnDesc(C.Structure):
    """pbmoe_attn_desc."""
    _fields_ = [("hidden", C.c_uint32), ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("rotary_dim", C.c_uint32), ("rope_theta", C.c_float),
                ("norm_epsilon", C.c_float), ("max_context", C.c_uint32), ("group_size", C.c_uint32),
                ("scale_bias_dtype", C.c_uint32)]


class Q4Matrix(C.Structure):
    """pbmoe_q4_matrix (device pointers)."""
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p)]


class AttnWeights(C.Structure):
    """pbmoe_attn_weights (device pointers)."""
    _fields_ = [("q", Q4Matrix), ("k", Q4Matrix), ("v", Q4Matrix), ("o", Q4Matrix),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p)]


_SIG = {
    "pbmoe_abi_version": ([], C.c_int),
    "pbmoe_last_error": ([], C.c_char_p),
    "pbmoe_q4_layout_fixed": ([_U32, _U32, _U32, _U32, C.POINTER(Q4Layout)], C.c_int),
    "pbmoe_q4_layout_validate": ([C.POINTER(Q4Layout)], C.c_int),
    "pbmoe_validate_routes": ([_P, _P, _U32, _U32, _U32], C.c_int),
    "pbmoe_renormalize_routes": ([_P, _U32, _U32, C.c_float, _P], C.c_int),
    "pbmoe_ctx_create": ([C.c_int, C.POINTER(_P)], C.c_int),
    "pbmoe_ctx_destroy": ([_P], C.c_int),
    "pbmoe_ctx_stream": ([_P, C.POINTER(_P)], C.c_int),
    "pbmoe_sync": ([_P], C.c_int),
    "pbmoe_set_phase_events": ([_P, C.POINTER(_P), _U32], C.c_int),
    "pbmoe_device_alloc": ([_P, C.c_size_t, C.POINTER(_P)], C.c_int),
    "pbmoe_device_free": ([_P, _P], C.c_int),
    "pbmoe_upload": ([_P, _P, _P, C.c_size_t], C.c_int),
    "pbmoe_download": ([_P, _P, _P, C.c_size_t], C.c_int),
    "pbmoe_bind_layer": ([_P, _U32, C.POINTER(LayerDesc), C.POINTER(Q4Layout), _P, C.c_size_t, _U32], C.c_int),
    "pbmoe_pack_inspect": ([C.c_char_p, _U32, C.POINTER(PackInfo)], C.c_int),
    "pbmoe_bind_layer_file": ([_P, _U32, C.POINTER(LayerDesc), C.POINTER(Q4Layout), C.c_char_p, _U32], C.c_int),
    "pbmoe_layer_slots": ([_P, _U32, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)], C.c_int),
    "pbmoe_bind_router": ([_P, _U32, _P, _U32, _P, _U32], C.c_int),
    "pbmoe_bind_shared": ([_P, _U32, C.POINTER(Q4Layout), _P, _P, _U32, _U32], C.c_int),
    "pbmoe_stream_read": ([_P, _P, C.c_size_t, _P], C.c_int),
    "pbmoe_bind_router_q4": ([_P, _U32, C.POINTER(Q4Matrix), _U32, _U32, _P, _U32], C.c_int),
    "pbmoe_bind_shared_gate_q4": ([_P, _U32, C.POINTER(Q4Matrix), _U32, _U32, _U32], C.c_int),
    "pbmoe_unbind_layer": ([_P, _U32], C.c_int),
    "pbmoe_route": ([_P, _U32, _P, _U32, _P, _P, _P], C.c_int),
    "pbmoe_route_logits": ([_P, _U32, _P, _U32, _P, _P], C.c_int),
    "pbmoe_moe_decode": ([_P, _U32, _P, _P, _U32, _P, _P, _P, _P, _P], C.c_int),
    "pbmoe_moe_layer": ([_P, _U32, _P, _P, _U32, _P, _P, _P, _P, _P], C.c_int),
    "pbmoe_moe_layer_noalloc": ([_P, _U32, _P, _P, _U32, _P, _P, _P, _P, _P], C.c_int),
    "pbmoe_moe_layer_norm": ([_P, _U32, _P, _P, _U32, _P, _P, _P, _P, _P], C.c_int),
    "pbmoe_moe_prefill": ([_P, _U32, _P, _P, _U32, _P, _P, _P, _P, _P], C.c_int),
    "pbmoe_dispatch_plan": ([_P, _U32, _U32, _U32, _P, _P, _P, _P, _P, _P, _P], C.c_int),
    "pbmoe_q4_dequantize": ([_P, _P, _P, _P, _U32, _U32, _U32, _U32, _P], C.c_int),
    "pbmoe_synth_fill_q4": ([_P, _P, C.POINTER(Q4Layout), _U32, _U32, C.c_uint64, _U32, _U32, _U32, _U32], C.c_int),
    "pbmoe_synth_center_q4": ([_P, _P, C.POINTER(Q4Layout), _U32, _U32, _U32], C.c_int),
    "pbmoe_bind_attention": ([_P, _U32, C.POINTER(AttnDesc), C.POINTER(AttnWeights)], C.c_int),
    "pbmoe_unbind_attention": ([_P, _U32], C.c_int),
    "pbmoe_attention_kv_cache": ([_P, _U32, C.POINTER(_P), C.POINTER(_P)], C.c_int),
    "pbmoe_attention_decode": ([_P, _U32, _P, _P, _P, _U32, _P, _P, _P, _P], C.c_int),
}

_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """Load libpbmoe.so (raises if it is not built: no fallback exists)."""
    global _lib
    if _lib is None:
        path = os.environ.get("PBMOE_LIB", LIB_PATH)  # another build of the library (comparisons)
        if not os.path.exists(path):
            raise RuntimeError(f"native library missing: {path}; run __graft_entry__.build()")
        L = C.CDLL(path)
        for name, (args, res) in _SIG.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIG)


def check(status: int) -> None:
    if status != OK:
        msg = lib().pbmoe_last_error()
        raise PbmoeError(status, msg.decode() if msg else "")


def status_of(fn, *args) -> int:
    """Call an ABI function and return its status without raising."""
    return fn(*args)


def q4_layout_fixed(hidden: int, intermediate: int, group_size: int, sb_dtype: int) -> Q4Layout:
    lay = Q4Layout()
    check(lib().pbmoe_q4_layout_fixed(hidden, intermediate, group_size, sb_dtype, C.byref(lay)))
    return lay


def pack_inspect(root: str, layer: int) -> PackInfo:
    """pbmoe_pack_inspect: parsed and validated root/layer_NN.json."""
    info = PackInfo()
    check(lib().pbmoe_pack_inspect(str(root).encode(), layer, C.byref(info)))
    return info


def validate_routes(ids, scores, active_experts: int, experts: int) -> int:
    i = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
    s = np.ascontiguousarray(np.asarray(scores, dtype=np.float32))
    return lib().pbmoe_validate_routes(i.ctypes.data, s.ctypes.data, i.size, active_experts, experts)


def renormalize_routes(scores, normalization: int, routed_scale: float):
    s = np.ascontiguousarray(np.asarray(scores, dtype=np.float32))
    w = np.zeros(max(s.size, 1), np.float32)
    rc = lib().pbmoe_renormalize_routes(s.ctypes.data, s.size, normalization, routed_scale, w.ctypes.data)
    return rc, w[: s.size]


class DeviceArray:
    """Device allocation owned through the C ABI (pbmoe_device_alloc)."""

    def __init__(self, ctx: "Context", shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib().pbmoe_device_alloc(ctx.handle, max(self.nbytes, 1), C.byref(p)))
        self.ptr = p.value

    def upload(self, host: np.ndarray) -> "DeviceArray":
        h = np.ascontiguousarray(host, dtype=self.dtype)
        assert h.nbytes == self.nbytes, (h.nbytes, self.nbytes)
        check(lib().pbmoe_upload(self.ctx.handle, self.ptr, h.ctypes.data, h.nbytes))
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().pbmoe_download(self.ctx.handle, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib().pbmoe_device_free(self.ctx.handle, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.ctx.handle:
                lib().pbmoe_device_free(self.ctx.handle, self.ptr)
        except Exception:
            pass


class Context:
    """pbmoe_ctx: one device, one HIP stream."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().pbmoe_ctx_create(device, C.byref(h)))
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            lib().pbmoe_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def stream(self) -> int:
        s = C.c_void_p()
        check(lib().pbmoe_ctx_stream(self.handle, C.byref(s)))
        return s.value or 0

    def sync(self) -> None:
        check(lib().pbmoe_sync(self.handle))

    def array(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def to_device(self, host: np.ndarray) -> DeviceArray:
        h = np.ascontiguousarray(host)
        return DeviceArray(self, h.shape, h.dtype).upload(h)
