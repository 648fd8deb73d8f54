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
QQ_WAIT_LIMIT_US_DEFAULT = 50000
# the device epoch moves on by this much when a timed-out decode wait is reported
SYNC_EPOCH_SKIP = 1024

# Every symbol include/qq_moe.h declares (tests/test_abi.py keeps them in sync).
EXPORTS = (
    "qq_init", "qq_destroy", "qq_last_error", "qq_set_stream", "qq_synchronize",
    "qq_q8_0_upload", "qq_q8_0_upload_dev", "qq_tensor_release",
    "qq_q8_0_matvec", "qq_q8_0_matvec_dev",
    "qq_moe_create", "qq_moe_release", "qq_moe_forward", "qq_moe_forward_dev",
    "qq_moe_forward_norm_dev", "qq_moe_forward_noalloc_dev", "qq_moe_set_gating",
    "qq_moe_stack_create", "qq_moe_stack_release", "qq_moe_stack_forward_dev",
    "qq_set_mfma_min_tokens", "qq_set_wait_limit", "qq_debug_epoch", "qq_debug_plant_words", "qq_rmsnorm_dev", "qq_timer_start", "qq_timer_stop",
    "qq_profile_enable", "qq_profile_read", "qq_profile_name", "qq_profile_kernel_count",
    "qq_capture_begin", "qq_capture_end", "qq_graph_launch", "qq_graph_release",
    "qq_buffer_alloc", "qq_buffer_free", "qq_buffer_write", "qq_buffer_read", "qq_moe_forward_record_dev",
)
# ... and include/qq_gguf.h
GGUF_EXPORTS = (
    "qq_gguf_open", "qq_gguf_open_memory", "qq_gguf_close", "qq_gguf_last_error", "qq_gguf_header",
    "qq_gguf_find_tensor", "qq_gguf_tensor_info", "qq_gguf_find_key", "qq_gguf_kv_info",
    "qq_gguf_kv_number", "qq_gguf_kv_string", "qq_gguf_kv_array", "qq_gguf_kv_array_number",
    "qq_gguf_moe_params", "qq_gguf_moe_layer",
)


# ... and include/qq_lfm2.h
LFM2_EXPORTS = (
    "qq_lfm2_create", "qq_lfm2_get_info", "qq_lfm2_reset", "qq_lfm2_forward_dev", "qq_lfm2_forward",
    "qq_lfm2_forward_routed_dev", "qq_lfm2_forward_routed",
    "qq_lfm2_release",
)


class Lfm2Info(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "n_layers", "n_embd", "n_heads", "n_head_kv", "head_dim", "n_vocab", "n_ff", "n_experts",
        "n_experts_used", "n_dense_lead", "l_cache", "max_ctx", "n_attn_layers")] + [
        ("eps", ctypes.c_double), ("rope_freq_base", ctypes.c_double)]


class GgufHeader(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("tensor_count", ctypes.c_uint64),
                ("kv_count", ctypes.c_uint64), ("file_size", ctypes.c_uint64),
                ("alignment", ctypes.c_uint64), ("data_offset", ctypes.c_uint64)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_int), ("shape", ctypes.c_uint64 * 4),
                ("type", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


class GgufMoeInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("H", "F", "E", "K", "gating", "router_type", "has_bias")]

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
        "qq_moe_forward_noalloc_dev": (I, [P, P, P, P, I, P, P, P, P]),
        "qq_moe_forward_norm_dev": (I, [P, P, P, P, ctypes.c_double, I, P, P, P, P]),
        "qq_moe_set_gating": (I, [P, P, I]),
        "qq_moe_stack_create": (I, [P, P, P, I, PP]),
        "qq_moe_stack_release": (I, [P, P]),
        "qq_moe_stack_forward_dev": (I, [P, P, P, ctypes.c_double, I, P, P, P, P]),
        "qq_set_mfma_min_tokens": (I, [P, I]),
        "qq_set_wait_limit": (I, [P, I]),
        "qq_debug_epoch": (I, [P, ctypes.POINTER(ctypes.c_uint32)]),
        "qq_debug_plant_words": (I, [P, ctypes.c_uint32]),
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
        "qq_buffer_alloc": (I, [P, S, PP]),
        "qq_buffer_free": (I, [P, P]),
        "qq_buffer_write": (I, [P, P, P, S]),
        "qq_buffer_read": (I, [P, P, P, S]),
        "qq_moe_forward_record_dev": (I, [P, P, P, P, I, P, P]),
        "qq_gguf_open": (I, [ctypes.c_char_p, PP]),
        "qq_gguf_open_memory": (I, [P, S, PP]),
        "qq_gguf_close": (None, [P]),
        "qq_gguf_last_error": (ctypes.c_char_p, []),
        "qq_gguf_header": (I, [P, ctypes.POINTER(GgufHeader)]),
        "qq_gguf_find_tensor": (ctypes.c_int64, [P, ctypes.c_char_p]),
        "qq_gguf_tensor_info": (I, [P, ctypes.c_uint64, ctypes.POINTER(GgufTensor)]),
        "qq_gguf_find_key": (ctypes.c_int64, [P, ctypes.c_char_p]),
        "qq_gguf_kv_info": (I, [P, ctypes.c_uint64, ctypes.POINTER(ctypes.c_char_p),
                                ctypes.POINTER(ctypes.c_uint32)]),
        "qq_gguf_kv_number": (I, [P, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)]),
        "qq_gguf_kv_string": (I, [P, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p),
                                  ctypes.POINTER(ctypes.c_uint64)]),
        "qq_gguf_kv_array": (I, [P, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint32),
                                 ctypes.POINTER(ctypes.c_uint64)]),
        "qq_gguf_kv_array_number": (I, [P, ctypes.c_uint64, ctypes.c_uint64,
                                        ctypes.POINTER(ctypes.c_double)]),
        "qq_gguf_moe_params": (I, [P, I, I, I, ctypes.POINTER(GgufMoeInfo)]),
        "qq_gguf_moe_layer": (I, [P, P, I, I, I, PP]),
        "qq_lfm2_create": (I, [P, P, PP]),
        "qq_lfm2_get_info": (I, [P, ctypes.POINTER(Lfm2Info)]),
        "qq_lfm2_reset": (I, [P, P]),
        "qq_lfm2_forward_dev": (I, [P, P, I, I, P, P]),
        "qq_lfm2_forward_routed_dev": (I, [P, P, I, I, P, P, P, P, P]),
        "qq_lfm2_forward_routed": (I, [P, P, I, I, P, P, P, P, P]),
        "qq_lfm2_forward": (I, [P, P, I, I, P]),
        "qq_lfm2_release": (None, [P, P]),
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

    def buffer_alloc(self, nbytes):
        """Zeroed device memory (qq_buffer_alloc); returns the device address."""
        p = ctypes.c_void_p()
        self.check(self.L.qq_buffer_alloc(self.h, int(nbytes), ctypes.byref(p)), "qq_buffer_alloc")
        return p.value

    def buffer_free(self, ptr):
        self.check(self.L.qq_buffer_free(self.h, ctypes.c_void_p(ptr)), "qq_buffer_free")

    def buffer_write(self, ptr, arr):
        a = np.ascontiguousarray(arr)
        self.check(self.L.qq_buffer_write(self.h, ctypes.c_void_p(ptr), _ptr(a), a.nbytes), "qq_buffer_write")

    def buffer_read(self, ptr, out):
        """Fill the contiguous array `out` from device address `ptr` once enqueued work has run."""
        assert out.flags["C_CONTIGUOUS"]
        self.check(self.L.qq_buffer_read(self.h, ctypes.c_void_p(ptr), _ptr(out), out.nbytes), "qq_buffer_read")
        return out

    def set_wait_limit(self, microseconds):
        """Bound on the decode kernel's device-side waits (qq_set_wait_limit)."""
        self.check(self.L.qq_set_wait_limit(self.h, int(microseconds)), "qq_set_wait_limit")

    def debug_epoch(self):
        """The device epoch of the decode exchange tags (qq_debug_epoch)."""
        v = ctypes.c_uint32()
        self.check(self.L.qq_debug_epoch(self.h, ctypes.byref(v)), "qq_debug_epoch")
        return v.value

    def debug_plant_words(self, tag):
        """Fill every exchange table with words tagged `tag` (qq_debug_plant_words)."""
        self.check(self.L.qq_debug_plant_words(self.h, int(tag) & 0xffffffff), "qq_debug_plant_words")

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

    def moe_stack(self, layers, norm_w_ptrs=None):
        """A stack of MoE layers of one shape (qq_moe_stack_create); norm_w_ptrs:
        one device pointer (or None) per layer, or None for unit weights."""
        n = len(layers)
        arr = (ctypes.c_void_p * n)(*[l.h for l in layers])
        nw = None
        if norm_w_ptrs is not None:
            nw = (ctypes.c_void_p * n)(*[None if p is None else ctypes.c_void_p(p) for p in norm_w_ptrs])
        h = ctypes.c_void_p()
        self.check(self.L.qq_moe_stack_create(self.h, arr, nw, n, ctypes.byref(h)), "qq_moe_stack_create")
        return MoeStack(self, h, list(layers))


class Gguf:
    """Native GGUF reader (include/qq_gguf.h) over a file (memory-mapped) or
    over caller bytes; needs no device."""

    def __init__(self, path=None, data=None):
        self.L = load()
        h = ctypes.c_void_p()
        if path is not None:
            rc = self.L.qq_gguf_open(os.fsencode(path), ctypes.byref(h))
            self._data = None
        else:
            self._data = (ctypes.c_uint8 * len(data)).from_buffer_copy(data) if len(data) else None
            rc = self.L.qq_gguf_open_memory(self._data, len(data), ctypes.byref(h))
        if rc != QQ_OK:
            raise QQError("qq_gguf_open failed (%d): %s" % (rc, self.L.qq_gguf_last_error().decode()))
        self.h = h

    def check(self, rc, what):
        if rc != QQ_OK:
            raise QQError("%s failed (%d): %s" % (what, rc, self.L.qq_gguf_last_error().decode()))

    def close(self):
        if self.h:
            self.L.qq_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def header(self):
        hd = GgufHeader()
        self.check(self.L.qq_gguf_header(self.h, ctypes.byref(hd)), "qq_gguf_header")
        return {f: getattr(hd, f) for f, _ in GgufHeader._fields_}

    def tensors(self):
        out = []
        for i in range(self.header()["tensor_count"]):
            t = GgufTensor()
            self.check(self.L.qq_gguf_tensor_info(self.h, i, ctypes.byref(t)), "qq_gguf_tensor_info")
            out.append(dict(name=t.name.decode("utf-8", "replace"), shape=list(t.shape[:t.n_dims]),
                            type=t.type, offset=t.offset, nbytes=t.nbytes))
        return out

    def find_tensor(self, name):
        return self.L.qq_gguf_find_tensor(self.h, name.encode())

    def find_key(self, key):
        return self.L.qq_gguf_find_key(self.h, key.encode())

    def kv(self, i):
        """(key, type, value): numbers as float, strings as str, arrays as
        (elem_type, n, numeric items or None)."""
        k, t = ctypes.c_char_p(), ctypes.c_uint32()
        self.check(self.L.qq_gguf_kv_info(self.h, i, ctypes.byref(k), ctypes.byref(t)), "qq_gguf_kv_info")
        typ = t.value
        if typ == 8:
            p, n = ctypes.c_void_p(), ctypes.c_uint64()
            self.check(self.L.qq_gguf_kv_string(self.h, i, ctypes.byref(p), ctypes.byref(n)), "kv_string")
            val = ctypes.string_at(p, n.value).decode("utf-8", "replace") if n.value else ""
        elif typ == 9:
            et, n = ctypes.c_uint32(), ctypes.c_uint64()
            self.check(self.L.qq_gguf_kv_array(self.h, i, ctypes.byref(et), ctypes.byref(n)), "kv_array")
            items = None
            if et.value not in (8, 9):
                items = []
                for j in range(n.value):
                    v = ctypes.c_double()
                    self.check(self.L.qq_gguf_kv_array_number(self.h, i, j, ctypes.byref(v)), "kv_array_number")
                    items.append(v.value)
            val = (et.value, n.value, items)
        else:
            v = ctypes.c_double()
            self.check(self.L.qq_gguf_kv_number(self.h, i, ctypes.byref(v)), "qq_gguf_kv_number")
            val = v.value
        return k.value.decode("utf-8", "replace"), typ, val

    def moe_params(self, block, K=0, gating=-1):
        info = GgufMoeInfo()
        self.check(self.L.qq_gguf_moe_params(self.h, block, K, gating, ctypes.byref(info)), "qq_gguf_moe_params")
        return {f: getattr(info, f) for f, _ in GgufMoeInfo._fields_}

    def moe_layer(self, ctx, block, K=0, gating=-1):
        """Upload block `block` to ctx's device (qq_gguf_moe_layer); the layer owns its tensors."""
        p = self.moe_params(block, K, gating)
        h = ctypes.c_void_p()
        ctx.check(self.L.qq_gguf_moe_layer(ctx.h, self.h, block, K, gating, ctypes.byref(h)), "qq_gguf_moe_layer")
        return MoeLayer(ctx, h, p["H"], p["F"], p["E"], p["K"], ())


class Lfm2Model:
    """The LFM2 single-token device forward (include/qq_lfm2.h), built from a Gguf."""

    def __init__(self, ctx, gguf):
        self.ctx, self.L = ctx, ctx.L
        h = ctypes.c_void_p()
        ctx.check(self.L.qq_lfm2_create(ctx.h, gguf.h, ctypes.byref(h)), "qq_lfm2_create")
        self.h = h
        info = Lfm2Info()
        ctx.check(self.L.qq_lfm2_get_info(self.h, ctypes.byref(info)), "qq_lfm2_get_info")
        self.info = {f: getattr(info, f) for f, _ in Lfm2Info._fields_}

    def reset(self):
        self.ctx.check(self.L.qq_lfm2_reset(self.ctx.h, self.h), "qq_lfm2_reset")

    def forward(self, token, position, logits=True):
        """Host logits (float32 [n_vocab]) or None."""
        out = np.empty(self.info["n_vocab"], np.float32) if logits else None
        self.ctx.check(self.L.qq_lfm2_forward(self.ctx.h, self.h, token, position, _ptr(out)),
                       "qq_lfm2_forward")
        return out

    def forward_dev(self, token, position, logits_ptr=None, idx_ptr=None):
        self.ctx.check(self.L.qq_lfm2_forward_dev(self.ctx.h, self.h, token, position, logits_ptr, idx_ptr),
                       "qq_lfm2_forward_dev")

    def forward_routed(self, token, position, mask=None, logits=True):
        """(logits, idx, w, probs) on the host (qq_lfm2_forward_routed): the
        onRouterUpdate payload of every MoE block, with the experts in `mask`
        skipped; rows of dense blocks are -1 / NaN."""
        I = self.info
        nl, K, E = I["n_layers"], I["n_experts_used"], I["n_experts"]
        out = np.empty(I["n_vocab"], np.float32) if logits else None
        idx = np.full((nl, K), -1, np.int32)
        w = np.full((nl, K), np.nan, np.float64)
        probs = np.full((nl, E), np.nan, np.float32)
        m = None
        if mask is not None:
            m = np.zeros(E, np.uint8)
            for e in mask:
                m[e] = 1
        self.ctx.check(self.L.qq_lfm2_forward_routed(self.ctx.h, self.h, token, position, _ptr(out), _ptr(m),
                                                     _ptr(idx), _ptr(w), _ptr(probs)), "qq_lfm2_forward_routed")
        return out, idx, w, probs

    def release(self):
        if self.h:
            self.L.qq_lfm2_release(self.ctx.h, self.h)
            self.h = None


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


class MoeStack:
    """n MoE layers applied in order to residual rows (qq_moe_stack_*)."""

    def __init__(self, ctx, h, layers):
        self.ctx, self.h, self.layers = ctx, h, layers
        self.n = len(layers)

    def forward_dev(self, hidden_ptr, T, eps=1e-5, mask=None, idx_ptr=None, w_ptr=None, probs_ptr=None):
        """For each layer: hidden += MoE_l(rmsnorm(hidden) * norm_w_l), device
        pointers; routing of layer l at l*T*K / l*T*E."""
        m = None
        if mask is not None:
            m = np.zeros(self.layers[0].E, np.uint8)
            for e in mask:
                m[e] = 1
        vp = lambda p: None if p is None else ctypes.c_void_p(p)
        self.ctx.check(self.ctx.L.qq_moe_stack_forward_dev(
            self.ctx.h, self.h, ctypes.c_void_p(hidden_ptr), float(eps), T, _ptr(m), vp(idx_ptr), vp(w_ptr),
            vp(probs_ptr)), "qq_moe_stack_forward_dev")

    def release(self):
        if self.h:
            self.ctx.check(self.ctx.L.qq_moe_stack_release(self.ctx.h, self.h), "qq_moe_stack_release")
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

    def forward_record_dev(self, x_ptr, hidden_ptr, T, mask=None, record_ptr=None):
        """hidden += MoE(x) and the per-row routing record [K idx | K w | E probs] as
        floats (qq_moe_forward_record_dev), device pointers, enqueued."""
        m = None
        if mask is not None:
            m = np.zeros(self.E, np.uint8)
            for e in mask:
                m[e] = 1
        vp = lambda p: None if p is None else ctypes.c_void_p(p)
        self.ctx.check(self.ctx.L.qq_moe_forward_record_dev(self.ctx.h, self.h, ctypes.c_void_p(x_ptr),
                                                            ctypes.c_void_p(hidden_ptr), T, _ptr(m),
                                                            vp(record_ptr)), "qq_moe_forward_record_dev")

    def forward_noalloc_dev(self, x_ptr, hidden_ptr, T, mask=None, idx_ptr=None, w_ptr=None, probs_ptr=None):
        """forward_dev with the fixed per-GPU scratch array (qq_moe_forward_noalloc_dev)."""
        m = None
        if mask is not None:
            m = np.zeros(self.E, np.uint8)
            for e in mask:
                m[e] = 1
        vp = lambda p: None if p is None else ctypes.c_void_p(p)
        self.ctx.check(self.ctx.L.qq_moe_forward_noalloc_dev(self.ctx.h, self.h, ctypes.c_void_p(x_ptr),
                                                             ctypes.c_void_p(hidden_ptr), T, _ptr(m),
                                                             vp(idx_ptr), vp(w_ptr), vp(probs_ptr)),
                       "qq_moe_forward_noalloc_dev")

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
