"""ctypes front end of the CPU oracle (oracle/qq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg.  It is the checker, never the thing measured on
the GPU and never a fallback of the product path.

Each wrapper names the reference function it restates; the C file holds the
file:line citations and how each function is pinned.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libqq_oracle.so")
_lib = None

TYPE_F32 = 0
TYPE_Q8_0 = 8


def build():
    """Compile the oracle in place (gcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        L.qo_f16_to_f64.restype = ctypes.c_double
        L.qo_f16_to_f64.argtypes = [ctypes.c_uint16]
        L.qo_f32_to_f16.restype = ctypes.c_uint16
        L.qo_f32_to_f16.argtypes = [ctypes.c_float]
        for name in ("qo_matmul_q8_0", "qo_matmul_f32"):
            f = getattr(L, name)
            f.restype = None
            f.argtypes = [P, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, P, P]
        L.qo_matmul_generic.restype = ctypes.c_int
        L.qo_matmul_generic.argtypes = [ctypes.c_int, P, ctypes.c_size_t, ctypes.c_int,
                                        ctypes.c_int, P, P]
        L.qo_read_weight_f32.restype = ctypes.c_int
        L.qo_read_weight_f32.argtypes = [ctypes.c_int, P, ctypes.c_size_t, ctypes.c_int, P]
        for name in ("qo_silu_inplace",):
            getattr(L, name).argtypes = [P, ctypes.c_int]
        for name in ("qo_mul_inplace", "qo_add_vec"):
            getattr(L, name).argtypes = [P, P, ctypes.c_int]
        L.qo_rmsnorm_unit.argtypes = [P, P, ctypes.c_int, ctypes.c_double]
        L.qo_moe_ffn.restype = ctypes.c_int
        L.qo_moe_ffn.argtypes = [ctypes.POINTER(MoeLayer), P, P, ctypes.c_int, P, P, P, P]
        L.qo_moe_route.restype = ctypes.c_int
        L.qo_moe_route.argtypes = [ctypes.POINTER(MoeLayer), P, ctypes.c_int, P, P, P]
        _lib = L
    return _lib


GATING_SIGMOID_BIAS = 0   # LFM2: sigmoid, expert bias for selection, 1e-6 in the sum
GATING_SOFTMAX = 1        # Qwen3-MoE: softmax, no bias, sum from 0


class MoeLayer(ctypes.Structure):
    _fields_ = [
        ("H", ctypes.c_int), ("F", ctypes.c_int), ("E", ctypes.c_int), ("K", ctypes.c_int),
        ("router_type", ctypes.c_int),
        ("router", ctypes.c_void_p), ("router_off", ctypes.c_size_t),
        ("bias_type", ctypes.c_int),
        ("bias", ctypes.c_void_p), ("bias_off", ctypes.c_size_t),
        ("gate", ctypes.c_void_p), ("gate_off", ctypes.c_size_t),
        ("up", ctypes.c_void_p), ("up_off", ctypes.c_size_t),
        ("down", ctypes.c_void_p), ("down_off", ctypes.c_size_t),
        ("gating", ctypes.c_int),
    ]


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def f16_to_f64(h):
    return lib().qo_f16_to_f64(int(h))


def f32_to_f16(f):
    return lib().qo_f32_to_f16(float(f))


def matmul_q8_0(buf, in_dim, out_dim, x, offset=0):
    """matmulQ80xF32 (src/tensor.js:26-53) -> float32[out_dim]."""
    buf = np.ascontiguousarray(buf, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(out_dim, np.float32)
    lib().qo_matmul_q8_0(_p(buf), offset, in_dim, out_dim, _p(x), _p(y))
    return y


def matmul_f32(buf, in_dim, out_dim, x, offset=0):
    """matmulF32xF32 (src/tensor.js:469-482) -> float32[out_dim]."""
    buf = np.ascontiguousarray(buf).view(np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(out_dim, np.float32)
    lib().qo_matmul_f32(_p(buf), offset, in_dim, out_dim, _p(x), _p(y))
    return y


def matmul_generic(typ, buf, in_dim, out_dim, x, offset=0):
    """matmulGeneric (src/tensor.js:485-496); raises like `throw new Error`."""
    buf = np.ascontiguousarray(buf).view(np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(out_dim, np.float32)
    if lib().qo_matmul_generic(typ, _p(buf), offset, in_dim, out_dim, _p(x), _p(y)):
        raise ValueError("Unsupported tensor type for matmul: %d" % typ)
    return y


def silu(a):
    a = np.array(a, dtype=np.float32, copy=True)
    lib().qo_silu_inplace(_p(a), a.size)
    return a


def rmsnorm_unit(x, eps=1e-5):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().qo_rmsnorm_unit(_p(x), _p(out), x.size, eps)
    return out


def _layer_struct(layer, keep):
    def ptr(a):
        a = np.ascontiguousarray(a).view(np.uint8)
        keep.append(a)
        return _p(a)

    has_bias = layer.get("bias") is not None
    return MoeLayer(H=layer["H"], F=layer["F"], E=layer["E"], K=layer["K"],
                    router_type=layer["router_type"], router=ptr(layer["router"]), router_off=0,
                    bias_type=layer["bias_type"] if has_bias else -1,
                    bias=ptr(layer["bias"]) if has_bias else None, bias_off=0,
                    gate=ptr(layer["gate"]), gate_off=0,
                    up=ptr(layer["up"]), up_off=0,
                    down=ptr(layer["down"]), down_off=0,
                    gating=GATING_SOFTMAX if layer.get("gating") == "softmax" else GATING_SIGMOID_BIAS)


def moe_route(layer, x):
    """Routing of _moEFFN (src/lfm2-engine.js:417-447) -> (idx, w, probs)."""
    H, E, K = layer["H"], layer["E"], layer["K"]
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H)
    T = x.shape[0]
    idx = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float64)
    probs = np.empty((T, E), np.float32)
    keep = []
    st = _layer_struct(layer, keep)
    if lib().qo_moe_route(ctypes.byref(st), _p(x), T, _p(idx), _p(w), _p(probs)):
        raise ValueError("qo_moe_route rejected the layer")
    return idx, w, probs


def moe_ffn(layer, x, hidden, mask=None):
    """Lfm2Engine._moEFFN (src/lfm2-engine.js:413-487) over T tokens.

    layer: dict from synth.moe_layer().  x, hidden: float32 [T, H].
    Returns (hidden_out, idx int32[T,K], w float64[T,K], probs float32[T,E]).
    """
    H, F, E, K = layer["H"], layer["F"], layer["E"], layer["K"]
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H)
    T = x.shape[0]
    hid = np.array(hidden, dtype=np.float32, copy=True).reshape(T, H)
    idx = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float64)
    probs = np.empty((T, E), np.float32)
    m = None
    if mask is not None:
        m = np.zeros(E, np.uint8)
        for e in mask:
            m[e] = 1
    keep = []
    st = _layer_struct(layer, keep)
    rc = lib().qo_moe_ffn(ctypes.byref(st), _p(x), _p(hid), T, _p(m), _p(idx), _p(w), _p(probs))
    if rc:
        raise ValueError("qo_moe_ffn rejected the layer")
    return hid, idx, w, probs
