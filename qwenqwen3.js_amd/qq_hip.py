"""ctypes binding of libqqmoe.so (include/qq_moe.h) for Python callers.

The product's host language is JavaScript (js/, napi/); this module is the
second binding of the same C ABI, used by the parity tests and bench.py.
It never computes anything itself: when libqqmoe.so is missing or the device
cannot be opened it raises, there is no CPU fallback.

torch bundles a HIP runtime under the same soname (libamdhip64.so.7) as the
one libqqmoe.so links; the first one loaded serves the whole process.  A
process that also uses torch imports torch before this module.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqqmoe.so")

QQ_OK = 0
TYPE_F32 = 0
TYPE_Q8_0 = 8
GATING_SIGMOID_BIAS = 0   # LFM2-MoE
GATING_SOFTMAX = 1        # Qwen3-MoE

# Every symbol include/qq_moe.h declares (tests/test_abi.py keeps them in sync).
EXPORTS = (
    "qq_init", "qq_destroy", "qq_last_error", "qq_set_stream", "qq_synchronize",
    "qq_q8_0_upload", "qq_q8_0_upload_dev", "qq_tensor_release",
    "qq_q8_0_matvec", "qq_q8_0_matvec_dev",
    "qq_moe_create", "qq_moe_release", "qq_moe_forward", "qq_moe_forward_dev",
    "qq_moe_forward_norm_dev", "qq_moe_set_gating",
    "qq_set_mfma_min_tokens", "qq_rmsnorm_dev", "qq_timer_start", "qq_timer_stop",
    "qq_profile_enable", "qq_profile_read", "qq_profile_name", "qq_profile_kernel_count",
    "qq_capture_begin", "qq_capture_end", "qq_graph_launch", "qq_graph_release",
)

_lib = None


class QQError(RuntimeError):
    pass


def load():
    """Load libqqmoe.so and declare its signatures (no device is touched)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise QQError("libqqmoe.so is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    PP = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "qq_init": (I, [I, PP]),
        "qq_destroy": (None, [P]),
        "qq_last_error": (ctypes.c_char_p, [P]),
        "qq_set_stream": (I, [P, P]),
        "qq_synchronize": (I, [P]),
        "qq_q8_0_upload": (I, [P, P, S, I, I, I, PP]),
        "qq_q8_0_upload_dev": (I, [P, P, S, I, I, I, PP]),
        "qq_tensor_release": (I, [P, P]),
        "qq_q8_0_matvec": (I, [P, P, I, P, P, I]),
        "qq_q8_0_matvec_dev": (I, [P, P, I, P, P, I]),
        "qq_moe_create": (I, [P, P, I, P, P, P, P, I, I, I, I, PP]),
        "qq_moe_release": (I, [P, P]),
        "qq_moe_forward": (I, [P, P, P, P, I, P, P, P, P]),
        "qq_moe_forward_dev": (I, [P, P, P, P, I, P, P, P, P]),
        "qq_moe_forward_norm_dev": (I, [P, P, P, P, ctypes.c_double, I, P, P, P, P]),
        "qq_moe_set_gating": (I, [P, P, I]),
        "qq_set_mfma_min_tokens": (I, [P, I]),
        "qq_rmsnorm_dev": (I, [P, P, P, P, I, I, ctypes.c_double]),
        "qq_timer_start": (I, [P]),
        "qq_timer_stop": (I, [P, ctypes.POINTER(ctypes.c_float)]),
        "qq_profile_enable": (I, [P, I]),
        "qq_profile_read": (I, [P, P, P, I]),
        "qq_profile_name": (ctypes.c_char_p, [I]),
        "qq_profile_kernel_count": (I, []),
        "qq_capture_begin": (I, [P]),
        "qq_capture_end": (I, [P, PP]),
        "qq_graph_launch": (I, [P, P]),
        "qq_graph_release": (I, [P, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Graph:
    """A recorded sequence of device-pointer calls (qq_capture_end)."""

    def __init__(self, ctx, h):
        self.ctx = ctx
        self.h = h

    def launch(self):
        self.ctx.check(self.ctx.L.qq_graph_launch(self.ctx.h, self.h), "qq_graph_launch")

    def release(self):
        if self.h:
            self.ctx.check(self.ctx.L.qq_graph_release(self.ctx.h, self.h), "qq_graph_release")
            self.h = None


class Context:
    """One device + stream (qq_init / qq_destroy)."""

    def __init__(self, device=0):
        L = load()
        h = ctypes.c_void_p()
        rc = L.qq_init(device, ctypes.byref(h))
        if rc != QQ_OK:
            raise QQError("qq_init(%d) failed (%d): %s" % (device, rc, L.qq_last_error(None).decode()))
        self.h = h
        self.L = L

    def check(self, rc, what):
        if rc != QQ_OK:
            raise QQError("%s failed (%d): %s" % (what, rc, self.L.qq_last_error(self.h).decode()))

    def close(self):
        if self.h:
            self.L.qq_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def set_stream(self, stream_handle):
        self.check(self.L.qq_set_stream(self.h, stream_handle), "qq_set_stream")

    def synchronize(self):
        self.check(self.L.qq_synchronize(self.h), "qq_synchronize")

    def capture_begin(self):
        """Start recording the device-pointer calls on this context into a graph."""
        self.check(self.L.qq_capture_begin(self.h), "qq_capture_begin")

    def capture_end(self):
        """Close the recording; returns a Graph to replay."""
        g = ctypes.c_void_p()
        self.check(self.L.qq_capture_end(self.h, ctypes.byref(g)), "qq_capture_end")
        return Graph(self, g)

    def rmsnorm_dev(self, x_ptr, weight_ptr, out_ptr, T, H, eps=1e-5):
        """out = rmsnorm(x) * weight (weight_ptr None: unit weight), device pointers."""
        self.check(self.L.qq_rmsnorm_dev(self.h, x_ptr, weight_ptr, out_ptr, int(T), int(H),
                                         float(eps)), "qq_rmsnorm_dev")

    def set_mfma_min_tokens(self, tokens):
        """Token batches of >= tokens rows use the fp16 MFMA path (0: never)."""
        self.check(self.L.qq_set_mfma_min_tokens(self.h, int(tokens)), "qq_set_mfma_min_tokens")

    def timer_start(self):
        self.check(self.L.qq_timer_start(self.h), "qq_timer_start")

    def timer_stop(self):
        ms = ctypes.c_float()
        self.check(self.L.qq_timer_stop(self.h, ctypes.byref(ms)), "qq_timer_stop")
        return ms.value

    def profile_enable(self, max_launches):
        self.check(self.L.qq_profile_enable(self.h, max_launches), "qq_profile_enable")

    def profile_read(self):
        """{kernel name: (summed ms, launches)} since profile_enable, then cleared."""
        n = self.L.qq_profile_kernel_count()
        ms = np.zeros(n, np.float32)
        cnt = np.zeros(n, np.int32)
        self.check(self.L.qq_profile_read(self.h, _ptr(ms), _ptr(cnt), n), "qq_profile_read")
        return {self.L.qq_profile_name(i).decode(): (float(ms[i]), int(cnt[i]))
                for i in range(n) if cnt[i]}

    # ---- tensors ----
    def upload_q8_0(self, gguf_bytes, in_dim, out_dim, n_mats=1):
        buf = np.ascontiguousarray(gguf_bytes).view(np.uint8)
        h = ctypes.c_void_p()
        self.check(self.L.qq_q8_0_upload(self.h, _ptr(buf), buf.nbytes, in_dim, out_dim, n_mats,
                                         ctypes.byref(h)), "qq_q8_0_upload")
        return Tensor(self, h, in_dim, out_dim, n_mats)

    def upload_q8_0_dev(self, dev_ptr, nbytes, in_dim, out_dim, n_mats=1):
        h = ctypes.c_void_p()
        self.check(self.L.qq_q8_0_upload_dev(self.h, ctypes.c_void_p(dev_ptr), nbytes, in_dim,
                                             out_dim, n_mats, ctypes.byref(h)), "qq_q8_0_upload_dev")
        return Tensor(self, h, in_dim, out_dim, n_mats)

    def moe_create(self, router, router_type, bias, gate, up, down, H, F, E, K):
        r = np.ascontiguousarray(router).view(np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        h = ctypes.c_void_p()
        self.check(self.L.qq_moe_create(self.h, _ptr(r), router_type, _ptr(b), gate.h, up.h, down.h,
                                        H, F, E, K, ctypes.byref(h)), "qq_moe_create")
        return MoeLayer(self, h, H, F, E, K, (gate, up, down))


class Tensor:
    def __init__(self, ctx, h, in_dim, out_dim, n_mats):
        self.ctx, self.h = ctx, h
        self.in_dim, self.out_dim, self.n_mats = in_dim, out_dim, n_mats

    def matvec(self, x, mat=0):
        """matmulQ80xF32 on host arrays: x [rows, in_dim] -> y [rows, out_dim]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows = x.size // self.in_dim
        y = np.empty((rows, self.out_dim), np.float32)
        self.ctx.check(self.ctx.L.qq_q8_0_matvec(self.ctx.h, self.h, mat, _ptr(x), _ptr(y), rows),
                       "qq_q8_0_matvec")
        return y

    def matvec_dev(self, x_ptr, y_ptr, rows, mat=0):
        self.ctx.check(self.ctx.L.qq_q8_0_matvec_dev(self.ctx.h, self.h, mat, ctypes.c_void_p(x_ptr),
                                                     ctypes.c_void_p(y_ptr), rows), "qq_q8_0_matvec_dev")

    def release(self):
        if self.h:
            self.ctx.L.qq_tensor_release(self.ctx.h, self.h)
            self.h = None


class MoeLayer:
    def __init__(self, ctx, h, H, F, E, K, keep):
        self.ctx, self.h = ctx, h
        self.H, self.F, self.E, self.K = H, F, E, K
        self._keep = keep

    def set_gating(self, gating):
        """GATING_SIGMOID_BIAS (LFM2-MoE, default) or GATING_SOFTMAX (Qwen3-MoE)."""
        self.ctx.check(self.ctx.L.qq_moe_set_gating(self.ctx.h, self.h, int(gating)), "qq_moe_set_gating")
        return self

    def forward(self, x, hidden, mask=None, want_probs=True):
        """_moEFFN over T tokens on host arrays.  Returns (hidden_out, idx, w, probs)."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.H)
        T = x.shape[0]
        hid = np.array(hidden, dtype=np.float32, copy=True).reshape(T, self.H)
        idx = np.empty((T, self.K), np.int32)
        w = np.empty((T, self.K), np.float64)
        probs = np.empty((T, self.E), np.float32) if want_probs else None
        m = None
        if mask is not None:
            m = np.zeros(self.E, np.uint8)
            for e in mask:
                m[e] = 1
        self.ctx.check(self.ctx.L.qq_moe_forward(self.ctx.h, self.h, _ptr(x), _ptr(hid), T, _ptr(m),
                                                 _ptr(idx), _ptr(w), _ptr(probs)), "qq_moe_forward")
        return hid, idx, w, probs

    def forward_dev(self, x_ptr, hidden_ptr, T, mask=None, idx_ptr=None, w_ptr=None, probs_ptr=None):
        m = None
        if mask is not None:
            m = np.zeros(self.E, np.uint8)
            for e in mask:
                m[e] = 1
        vp = lambda p: None if p is None else ctypes.c_void_p(p)
        self.ctx.check(self.ctx.L.qq_moe_forward_dev(self.ctx.h, self.h, ctypes.c_void_p(x_ptr),
                                                     ctypes.c_void_p(hidden_ptr), T, _ptr(m), vp(idx_ptr),
                                                     vp(w_ptr), vp(probs_ptr)), "qq_moe_forward_dev")

    def forward_norm_dev(self, hidden_ptr, T, norm_w_ptr=None, eps=1e-5, mask=None, idx_ptr=None,
                         w_ptr=None, probs_ptr=None):
        """hidden += MoE(rmsnorm(hidden) * norm_w), device pointers (qq_moe_forward_norm_dev)."""
        m = None
        if mask is not None:
            m = np.zeros(self.E, np.uint8)
            for e in mask:
                m[e] = 1
        vp = lambda p: None if p is None else ctypes.c_void_p(p)
        self.ctx.check(self.ctx.L.qq_moe_forward_norm_dev(
            self.ctx.h, self.h, ctypes.c_void_p(hidden_ptr), vp(norm_w_ptr), float(eps), T, _ptr(m),
            vp(idx_ptr), vp(w_ptr), vp(probs_ptr)), "qq_moe_forward_norm_dev")

    def release(self):
        if self.h:
            self.ctx.L.qq_moe_release(self.ctx.h, self.h)
            self.h = None
