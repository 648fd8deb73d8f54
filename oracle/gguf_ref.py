"""Python restatement of the reference's GGUF reader (src/gguf.js, GGUFReader).

TEST INFRASTRUCTURE ONLY: tests/ use it as the checker of the library's
native reader (qwenqwen3.js_amd/csrc/gguf.cpp); nothing in the product path
imports it.

Follows, function by function:
  parse_header    GGUFReader._parseHeader      src/gguf.js:37-94
  _skip_value     GGUFReader._skipValue        src/gguf.js:96-131
  _read_value     GGUFReader._readValue        src/gguf.js:177-212
  tensor_nbytes   GGUFReader._tensorNbytes     src/gguf.js:302-343
  tensor_meta     getTensorMeta / ...ByName    src/gguf.js:235-261
  key_value       getKeyValue / findKey        src/gguf.js:215-226
  arch            getArch                      src/gguf.js:264-292
  read_weight_f32 _readWeightF32               src/tensor.js:80-100

Pinned by tests/test_gguf.py: a hand-assembled known-answer file whose every
offset is written out in the test, round trips of files made by
oracle/synth.py's GGUF writer (written from the published GGUF v3 layout, not
from this reader), and the reference's own error messages.
"""
import math
import struct

import numpy as np

SIGNATURE = b"GGUF"
VERSION = 3
KV = dict(UINT8=0, INT8=1, UINT16=2, INT16=3, UINT32=4, INT32=5, FLOAT32=6, BOOL=7,
          STRING=8, ARRAY=9, UINT64=10, INT64=11, FLOAT64=12)
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B",
           10: "<Q", 11: "<q", 12: "<d"}

# bytes per block and elements per block (gguf.js:302-343); unknown -> F32
_BLOCKS = {0: (4, 1), 1: (2, 1), 8: (34, 32), 2: (34, 32), 3: (36, 32), 6: (42, 32), 7: (44, 32),
           10: (84, 256), 11: (110, 256), 12: (144, 256), 13: (176, 256), 14: (210, 256)}


class GGUFError(Exception):
    pass


def tensor_nbytes(shape, typ):
    n = 1
    for d in shape:
        n *= d
    size, per = _BLOCKS.get(typ, (4, 1))
    return -(-n // per) * size


class Reader:
    """GGUFReader over a bytes-like object (the whole file)."""

    def __init__(self, buf):
        self.buf = memoryview(buf).cast("B")
        self.kvs = []        # (key, type, value_offset)
        self.tensors = []    # dicts: name, shape, type, offset (absolute), nbytes (padded)
        self.warnings = []
        self._parse_header()

    # -- low-level reads (DataView semantics: RangeError past the end)
    def _u(self, fmt, off):
        n = struct.calcsize(fmt)
        if off < 0 or off + n > len(self.buf):
            raise GGUFError("Offset is outside the bounds of the DataView")
        return struct.unpack_from(fmt, self.buf, off)[0]

    def _str(self, off, n):
        if off + n > len(self.buf):
            raise GGUFError("Out of bounds string read: offset=%d, len=%d, buffer size=%d"
                            % (off, n, len(self.buf)))
        return bytes(self.buf[off:off + n]).decode("utf-8", errors="replace")

    def _parse_header(self):
        sig = self._str(0, 4) if len(self.buf) >= 4 else bytes(self.buf).decode("latin-1")
        if sig != "GGUF":
            raise GGUFError("Invalid signature: %s" % sig)
        self.version = self._u("<I", 4)
        if self.version != VERSION:
            self.warnings.append("GGUF version %d may not be fully supported" % self.version)
        n_tensors = self._u("<Q", 8)
        n_kv = self._u("<Q", 16)
        off = 24
        for _ in range(n_kv):
            klen = self._u("<Q", off)
            key = self._str(off + 8, klen)
            typ = self._u("<I", off + 8 + klen)
            val = off + 8 + klen + 4
            self.kvs.append((key, typ, val))
            off = self._skip_value(typ, val)
        for _ in range(n_tensors):
            nlen = self._u("<Q", off)
            off += 8
            name = self._str(off, nlen)
            off += nlen
            nd = self._u("<I", off)
            off += 4
            shape = []
            for _ in range(nd):
                shape.append(self._u("<Q", off))
                off += 8
            typ = self._u("<I", off)
            off += 4
            rel = self._u("<Q", off)
            off += 8
            nbytes = -(-tensor_nbytes(shape, typ) // 256) * 256
            self.tensors.append(dict(name=name, shape=shape, type=typ, rel=rel, nbytes=nbytes))
        align = self._js_number(self.key_value("general.alignment"))
        align = int(align) if (align == align and align) else 32   # Number(x) || 32
        self.alignment = align
        self.data_offset = off + (align - off % align) % align
        for t in self.tensors:
            t["offset"] = self.data_offset + t.pop("rel")

    def _skip_value(self, typ, off):
        if typ in _SCALAR:
            return off + struct.calcsize(_SCALAR[typ])
        if typ == KV["STRING"]:
            return off + 8 + self._u("<Q", off)
        if typ == KV["ARRAY"]:
            et = self._u("<I", off)
            n = self._u("<Q", off + 4)
            p = off + 12
            for _ in range(n):
                p = self._skip_value(et, p)
            return p
        raise GGUFError("Unknown KV type: %d" % typ)

    def _read_value(self, typ, off):
        if typ == KV["BOOL"]:
            return self._u("<B", off) != 0
        if typ in _SCALAR:
            return self._u(_SCALAR[typ], off)
        if typ == KV["STRING"]:
            return self._str(off + 8, self._u("<Q", off))
        if typ == KV["ARRAY"]:
            et = self._u("<I", off)
            n = self._u("<Q", off + 4)
            p = off + 12
            out = []
            for _ in range(n):
                out.append(self._read_value(et, p))
                p = self._skip_value(et, p)
            return out
        raise GGUFError("Unsupported KV type: %d" % typ)

    @staticmethod
    def _js_number(v):
        """Number(v) for the value kinds getKeyValue returns."""
        if v is None:
            return math.nan
        if isinstance(v, bool):
            return 1.0 if v else 0.0
        if isinstance(v, (int, float)):
            return float(v)
        if isinstance(v, str):
            s = v.strip()
            if s == "":
                return 0.0
            try:
                return float(int(s, 16)) if s.lower().startswith("0x") else float(s)
            except ValueError:
                return math.nan
        return math.nan

    # -- public API
    def header(self):
        return dict(version=self.version, tensor_count=len(self.tensors), kv_count=len(self.kvs),
                    file_size=len(self.buf))

    def find_key(self, key):
        for i, (k, _, _) in enumerate(self.kvs):
            if k == key:
                return i
        return -1

    def kv_value(self, i):
        _, typ, off = self.kvs[i]
        return self._read_value(typ, off)

    def key_value(self, key, default=None):
        i = self.find_key(key)
        return default if i < 0 else self.kv_value(i)

    def tensor_meta(self, name):
        for t in self.tensors:
            if t["name"] == name:
                return dict(offset=t["offset"], nbytes=t["nbytes"], shape=list(t["shape"]), type=t["type"])
        return None

    def tensor_bytes(self, name, n):
        m = self.tensor_meta(name)
        return np.frombuffer(self.buf, np.uint8, n, m["offset"])

    def arch(self):
        """getArch (gguf.js:264-292), the fields this path reads."""
        a = self.key_value("general.architecture", "unknown")
        p = a + "."
        num = lambda k: self._js_number(self.key_value(p + k))
        return dict(architecture=a, embeddingLength=num("embedding_length"),
                    blockCount=num("block_count"),
                    expertFeedForwardLength=num("expert_feed_forward_length") or 0,
                    expertCount=num("expert_count"), expertUsedCount=num("expert_used_count"))


def read_weight_f32(typ, raw, n):
    """_readWeightF32 (src/tensor.js:80-100): an F32 or Q8_0 vector of n values."""
    raw = np.asarray(raw, np.uint8)
    if typ == 0:
        return raw[:4 * n].view("<f4").astype(np.float32)
    if typ == 8:
        out = np.empty(n, np.float32)
        for b in range(-(-n // 32)):
            d = float(raw[b * 34:b * 34 + 2].view("<f2")[0])
            qs = raw[b * 34 + 2:b * 34 + 34].view(np.int8)
            for i in range(min(32, n - 32 * b)):
                out[32 * b + i] = np.float32(float(qs[i]) * d)
        return out
    raise GGUFError("Unsupported weight type for norm: %d" % typ)


def moe_params(r, block, K=0, gating=-1):
    """The MoE block binding of the engines (src/lfm2-engine.js:129-137,
    src/qwen3-engine.js:41-73) with the engine picked as html/chat.html:206-207
    does: returns (H, F, E, K, gating, router_type, has_bias)."""
    arch = r.key_value("general.architecture", "")
    lfm2 = arch in ("", "lfm2moe", "lfm2")
    if gating < 0:
        gating = 0 if lfm2 else 1
    if K <= 0:
        k = Reader._js_number(r.key_value((arch or "lfm2moe") + ".expert_used_count"))
        K = int(k) if (k == k and k) else (4 if lfm2 else 8)
    g = r.tensor_meta("blk.%d.ffn_gate_exps.weight" % block)
    rt = r.tensor_meta("blk.%d.ffn_gate_inp.weight" % block)
    b = r.tensor_meta("blk.%d.exp_probs_b.bias" % block)
    H, F, E = g["shape"]
    return H, F, E, K, gating, rt["type"], int(gating == 0 and b is not None)


def moe_layer(r, block, K=0, gating=-1):
    """An oracle-format layer dict (as oracle/synth.py's moe_layer makes) read
    from the file: the tensors the engines bind for MoE block `block`."""
    H, F, E, K, gating, rtype, has_bias = moe_params(r, block, K, gating)
    nbH, nbF = -(-H // 32), -(-F // 32)
    rn = E * H * 4 if rtype == 0 else E * nbH * 34
    layer = dict(H=H, F=F, E=E, K=K, router_type=rtype,
                 router=np.array(r.tensor_bytes("blk.%d.ffn_gate_inp.weight" % block, rn)),
                 bias_type=0, bias=None,
                 gate=np.array(r.tensor_bytes("blk.%d.ffn_gate_exps.weight" % block, E * F * nbH * 34)),
                 up=np.array(r.tensor_bytes("blk.%d.ffn_up_exps.weight" % block, E * F * nbH * 34)),
                 down=np.array(r.tensor_bytes("blk.%d.ffn_down_exps.weight" % block, E * H * nbF * 34)),
                 gating="softmax" if gating == 1 else "sigmoid")
    if has_bias:
        m = r.tensor_meta("blk.%d.exp_probs_b.bias" % block)
        nb = E * 4 if m["type"] == 0 else -(-E // 32) * 34
        layer["bias"] = read_weight_f32(m["type"], r.tensor_bytes("blk.%d.exp_probs_b.bias" % block, nb), E)
    return layer
