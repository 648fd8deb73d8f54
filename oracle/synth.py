"""Seeded synthetic inputs in the reference's GGUF byte layout.

TEST INFRASTRUCTURE: used by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg to build identical inputs for the HIP path and the oracle.

Layouts follow the reference:
  * Q8_0 block = {fp16 d (little-endian) @+0, int8 qs[32] @+2}, 34 bytes
    (src/tensor.js:1-2, src/gguf.js:307-309).
  * A 2-D GGUF tensor [in_dim, out_dim] is column-major: column c holds
    ceil(in_dim/32) blocks (src/tensor.js:4-5, 36).
  * A 3-D expert tensor [in_dim, out_dim, E] is E such matrices back to back
    (src/lfm2-engine.js:489-505).
  * The F32 router [H, E] is expert-major: column e is H floats
    (src/tensor.js:469-482).

Value distributions are the benchmark workloads': qs ~ U{-127..127},
d = fp16_RNE(|N(0,1)| * 0.002), router ~ N(0, 0.02), activations ~ N(0, 1).
"""
import numpy as np

QK = 32
BLK = 34
Q8_DTYPE = np.dtype([("d", "<f2"), ("qs", "i1", (QK,))])
assert Q8_DTYPE.itemsize == BLK

TYPE_F32 = 0
TYPE_Q8_0 = 8

# Zipf(s=1.1) expert bias for the skewed prefill workload:
# bias_e = ZIPF_ALPHA * ln(pmf(rank_e)) over a seeded expert permutation.
# With this alpha the hottest experts receive 300+ of the 2048 tokens and the
# coldest fewer than 10 (tests/test_synth.py checks this on the oracle's routing).
ZIPF_S = 1.1
ZIPF_ALPHA = 0.17


def q8_0_tensor(rng, in_dim, out_dim, n_mats=1, scale=0.002):
    """GGUF-layout Q8_0 bytes of n_mats matrices [in_dim, out_dim]."""
    nb = (in_dim + QK - 1) // QK
    n = n_mats * out_dim * nb
    blocks = np.empty(n, Q8_DTYPE)
    blocks["qs"] = rng.integers(-127, 128, size=(n, QK), dtype=np.int8)
    if in_dim % QK:
        # the reference never reads past in_dim (src/tensor.js:44); zero the tail
        blocks["qs"].reshape(n_mats, out_dim, nb, QK)[:, :, -1, in_dim % QK:] = 0
    blocks["d"] = (np.abs(rng.standard_normal(n)) * scale).astype(np.float16)
    return blocks.view(np.uint8)


def q8_0_dequant(buf, in_dim, out_dim, n_mats=1):
    """float64 [n_mats, out_dim, in_dim] dense view of GGUF Q8_0 bytes."""
    nb = (in_dim + QK - 1) // QK
    blocks = np.frombuffer(np.ascontiguousarray(buf).tobytes(), Q8_DTYPE).reshape(n_mats, out_dim, nb)
    w = blocks["qs"].astype(np.float64) * blocks["d"].astype(np.float64)[..., None]
    return w.reshape(n_mats, out_dim, nb * QK)[:, :, :in_dim]


def zipf_bias(rng, E, s=ZIPF_S, alpha=ZIPF_ALPHA):
    k = np.arange(1, E + 1, dtype=np.float64)
    pmf = k ** (-s)
    pmf /= pmf.sum()
    perm = rng.permutation(E)
    return (alpha * np.log(pmf[perm])).astype(np.float32)


def moe_layer(seed, H=2048, F=1792, E=32, K=4, bias="uniform", router_type=TYPE_F32,
              router_std=0.02, gating="sigmoid"):
    """One LFM2-MoE MoE layer's tensors, as Lfm2Engine binds them
    (src/lfm2-engine.js:129-137), or with gating="softmax" a Qwen3-MoE layer
    (src/qwen3-engine.js:48-73: no bias tensor; pass bias=None).

    bias: "uniform" -> U(-0.01, 0.01) F32; "zipf" -> Zipf(1.1) skew; None -> absent.
    router_type: TYPE_F32 (float32 [H, E]) or TYPE_Q8_0.
    """
    rng = np.random.default_rng(seed)
    if router_type == TYPE_F32:
        router = (rng.standard_normal((E, H)) * router_std).astype(np.float32).view(np.uint8).ravel()
    elif router_type == TYPE_Q8_0:
        router = q8_0_tensor(rng, H, E, 1, scale=router_std / 64.0)
    else:
        raise ValueError(router_type)
    if bias is None:
        b = None
    elif bias == "uniform":
        b = rng.uniform(-0.01, 0.01, E).astype(np.float32)
    elif bias == "zipf":
        b = zipf_bias(rng, E)
    else:
        raise ValueError(bias)
    return {
        "H": H, "F": F, "E": E, "K": K,
        "router_type": router_type, "router": router,
        "bias_type": TYPE_F32, "bias": b,
        "gate": q8_0_tensor(rng, H, F, E),
        "up": q8_0_tensor(rng, H, F, E),
        "down": q8_0_tensor(rng, F, H, E),
        "gating": gating,
    }


def activations(seed, T, H):
    """(x, hidden): x is the ffn_norm output fed to the MoE, hidden the residual."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    hidden = rng.standard_normal((T, H)).astype(np.float32)
    return x, hidden


def matvec_case(seed, in_dim=1024, out_dim=3072):
    """Q8_0 matvec workload: GGUF [in_dim, out_dim] weight and x ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    w = q8_0_tensor(rng, in_dim, out_dim)
    x = rng.standard_normal(in_dim).astype(np.float32)
    return w, x


# ---------------------------------------------------------------- GGUF files

# GGUF v3 as published with ggml (docs/gguf.md): little-endian header
# {"GGUF", u32 version, u64 n_tensors, u64 n_kv}; KV = {string key, u32 type,
# value}; string = {u64 len, bytes}; array = {u32 elem type, u64 n, elems};
# tensor info = {string name, u32 n_dims, u64 ne[n_dims], u32 type,
# u64 offset from the data section}; the data section starts at the next
# multiple of general.alignment (32 when the key is absent) and each tensor's
# data is aligned the same way.
GGUF_KV_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?",
               10: "<Q", 11: "<q", 12: "<d"}
GGUF_STRING, GGUF_ARRAY = 8, 9


def _gguf_str(s):
    import struct
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _gguf_value(typ, v):
    import struct
    if typ == GGUF_STRING:
        return _gguf_str(v)
    if typ == GGUF_ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_gguf_value(et, x) for x in items)
    return struct.pack(GGUF_KV_FMT[typ], v)


def gguf_file(kvs, tensors, version=3, alignment=None):
    """Bytes of a GGUF file.

    kvs: [(key, type, value)], array values as (elem_type, [items]);
    tensors: [(name, shape, type, data bytes)];
    alignment: when given, written as general.alignment (u32) ahead of kvs.
    Returns (bytes, {name: absolute data offset})."""
    import struct
    al = 32 if alignment is None else alignment
    kv_list = ([("general.alignment", 4, alignment)] if alignment is not None else []) + list(kvs)
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv_list))
    head += b"".join(_gguf_str(k) + struct.pack("<I", t) + _gguf_value(t, v) for k, t, v in kv_list)
    raw = [np.ascontiguousarray(t[3]).view(np.uint8).tobytes() for t in tensors]
    rel, pos = [], 0
    for data in raw:
        pos = -(-pos // al) * al
        rel.append(pos)
        pos += len(data)
    for (name, shape, typ, _), r in zip(tensors, rel):
        head += _gguf_str(name) + struct.pack("<I", len(shape))
        head += b"".join(struct.pack("<Q", d) for d in shape) + struct.pack("<IQ", typ, r)
    start = -(-len(head) // al) * al
    out = bytearray(head) + bytearray(start - len(head))
    for data, r in zip(raw, rel):
        out += bytearray(start + r - len(out))
        out += data
    return bytes(out), {t[0]: start + r for t, r in zip(tensors, rel)}


def gguf_write(path, kvs, tensors, version=3):
    """gguf_file's layout (default alignment) written to `path` tensor by
    tensor, without building the whole file in memory.  Returns {name: offset}."""
    import struct
    al = 32
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    head += b"".join(_gguf_str(k) + struct.pack("<I", t) + _gguf_value(t, v) for k, t, v in kvs)
    sizes = [np.asarray(t[3]).nbytes for t in tensors]
    rel, pos = [], 0
    for n in sizes:
        pos = -(-pos // al) * al
        rel.append(pos)
        pos += n
    for (name, shape, typ, _), r in zip(tensors, rel):
        head += _gguf_str(name) + struct.pack("<I", len(shape))
        head += b"".join(struct.pack("<Q", d) for d in shape) + struct.pack("<IQ", typ, r)
    start = -(-len(head) // al) * al
    with open(path, "wb") as f:
        f.write(head + bytes(start - len(head)))
        at = 0
        for t, r in zip(tensors, rel):
            f.write(bytes(r - at))
            data = np.ascontiguousarray(t[3])
            f.write(memoryview(data.view(np.uint8).reshape(-1)))
            at = r + data.nbytes
    return {t[0]: start + r for t, r in zip(tensors, rel)}


def moe_gguf(layers, arch="lfm2moe", K=None, alignment=None, extra_kvs=()):
    """A GGUF file holding MoE blocks 0..n-1 built from oracle-format layer
    dicts (moe_layer), with the tensor names the engines bind
    (src/lfm2-engine.js:131-136, src/qwen3-engine.js:49-69) and the arch keys
    they read.  Returns (bytes, {name: offset})."""
    L0 = layers[0]
    kvs = [("general.architecture", GGUF_STRING, arch),
           (arch + ".block_count", 4, len(layers)),
           (arch + ".embedding_length", 4, L0["H"]),
           (arch + ".expert_count", 4, L0["E"]),
           (arch + ".expert_feed_forward_length", 4, L0["F"])]
    if K is not None:
        kvs.append((arch + ".expert_used_count", 4, K))
    kvs += list(extra_kvs)
    tensors = []
    for b, L in enumerate(layers):
        H, F, E = L["H"], L["F"], L["E"]
        p = "blk.%d." % b
        tensors.append((p + "ffn_norm.weight", [H], TYPE_F32, np.ones(H, np.float32)))
        tensors.append((p + "ffn_gate_inp.weight", [H, E], L["router_type"], L["router"]))
        if L.get("bias") is not None:
            tensors.append((p + "exp_probs_b.bias", [E], TYPE_F32, L["bias"]))
        tensors.append((p + "ffn_gate_exps.weight", [H, F, E], TYPE_Q8_0, L["gate"]))
        tensors.append((p + "ffn_up_exps.weight", [H, F, E], TYPE_Q8_0, L["up"]))
        tensors.append((p + "ffn_down_exps.weight", [F, H, E], TYPE_Q8_0, L["down"]))
    return gguf_file(kvs, tensors, alignment=alignment)


# ---------------------------------------------------------------- LFM2 whole model

TYPE_F16 = 1

LFM2_TINY = dict(H=256, n_layers=6, attn_layers=(2, 4), n_dense=2, n_heads=4, n_head_kv=2,
                 head_dim=64, n_ff=512, F=128, E=8, K=2, vocab=300, l_cache=3, ctx=64,
                 rope_base=5000000.0, eps=1e-5)
"""A small LFM2-MoE model: layers 0-1 dense, 2 and 4 attention, the rest short-conv."""

LFM2_8B_A1B = dict(H=2048, n_layers=24, attn_layers=(2, 6, 10, 14, 18, 21), n_dense=2,
                   n_heads=32, n_head_kv=8, head_dim=64, n_ff=7168, F=1792, E=32, K=4,
                   vocab=65536, l_cache=3, ctx=4096, rope_base=5000000.0, eps=1e-5)
"""LFM2-8B-A1B's shapes: 24 blocks (6 attention, 18 short-conv; 2 dense FFN,
22 MoE with 32 experts, top-4), H 2048, 32 query / 8 KV heads of 64, vocab 65536."""


def q8_0_pool(seed, n_blocks, scale=0.005):
    """A pool of random Q8_0 blocks that lfm2_tensors(pool=...) slices its
    matrices from (a fast way to fill a multi-GB model whose values only need
    to be plausible, as for timing)."""
    rng = np.random.default_rng(seed)
    blocks = np.empty(n_blocks, Q8_DTYPE)
    blocks["qs"] = rng.integers(-127, 128, size=(n_blocks, QK), dtype=np.int8)
    blocks["d"] = (np.abs(rng.standard_normal(n_blocks)) * scale).astype(np.float16)
    return blocks


def lfm2_tensors(seed, cfg, conv_type=TYPE_F32, tied=True, bias="uniform", pool=None):
    """Seeded tensors of an LFM2-MoE model, named as Lfm2Engine binds them
    (src/lfm2-engine.js:78-144): [(name, shape, type, bytes)].  Dense and
    attention matrices are Q8_0; norms, router and expert bias F32; the conv
    kernel [l_cache, H] F32, F16 or Q8_0 (one block per column).  With a
    q8_0_pool, every Q8_0 matrix is a seeded slice of the pool."""
    rng = np.random.default_rng(seed)
    H, L, hd = cfg["H"], cfg["l_cache"], cfg["head_dim"]
    nq, nkv = cfg["n_heads"] * hd, cfg["n_head_kv"] * hd
    t = []

    def q8(name, i, o, n=1, scale=0.005):
        shape = [i, o] + ([n] if n > 1 else [])
        if pool is not None:
            nblk = n * o * ((i + QK - 1) // QK)
            assert i % QK == 0 and nblk <= len(pool)
            off = int(rng.integers(0, len(pool) - nblk + 1))
            t.append((name, shape, TYPE_Q8_0, pool[off:off + nblk].view(np.uint8)))
            return
        t.append((name, shape, TYPE_Q8_0, q8_0_tensor(rng, i, o, n, scale)))

    def f32(name, shape, v):
        t.append((name, list(shape), TYPE_F32, np.asarray(v, np.float32)))

    q8("token_embd.weight", H, cfg["vocab"], scale=0.01)
    f32("token_embd_norm.weight", [H], rng.uniform(0.5, 1.5, H))
    if not tied:
        q8("output.weight", H, cfg["vocab"], scale=0.01)
    for i in range(cfg["n_layers"]):
        p = "blk.%d." % i
        f32(p + "attn_norm.weight", [H], rng.uniform(0.5, 1.5, H))
        f32(p + "ffn_norm.weight", [H], rng.uniform(0.5, 1.5, H))
        if i in cfg["attn_layers"]:
            q8(p + "attn_q.weight", H, nq)
            q8(p + "attn_k.weight", H, nkv)
            q8(p + "attn_v.weight", H, nkv)
            q8(p + "attn_output.weight", nq, H)
            f32(p + "attn_q_norm.weight", [hd], rng.uniform(0.5, 1.5, hd))
            f32(p + "attn_k_norm.weight", [hd], rng.uniform(0.5, 1.5, hd))
        else:
            kern = (rng.standard_normal(L * H) * 0.5).astype(np.float32)   # index d * L + k
            if conv_type == TYPE_F32:
                t.append((p + "shortconv.conv.weight", [L, H], TYPE_F32, kern))
            elif conv_type == TYPE_F16:
                t.append((p + "shortconv.conv.weight", [L, H], TYPE_F16, kern.astype(np.float16)))
            else:
                t.append((p + "shortconv.conv.weight", [L, H], TYPE_Q8_0, q8_0_tensor(rng, L, H, 1, 0.01)))
            q8(p + "shortconv.in_proj.weight", H, 3 * H)
            q8(p + "shortconv.out_proj.weight", H, H)
        if i < cfg["n_dense"]:
            q8(p + "ffn_gate.weight", H, cfg["n_ff"])
            q8(p + "ffn_up.weight", H, cfg["n_ff"])
            q8(p + "ffn_down.weight", cfg["n_ff"], H)
        else:
            E, F = cfg["E"], cfg["F"]
            f32(p + "ffn_gate_inp.weight", [H, E], rng.standard_normal(E * H) * 0.05)
            if bias is not None:
                f32(p + "exp_probs_b.bias", [E], rng.uniform(-0.01, 0.01, E))
            q8(p + "ffn_gate_exps.weight", H, F, E)
            q8(p + "ffn_up_exps.weight", H, F, E)
            q8(p + "ffn_down_exps.weight", F, H, E)
    return t


def lfm2_gguf(seed, cfg, arch="lfm2moe", path=None, **kw):
    """GGUF bytes of lfm2_tensors(seed, cfg) with the keys Lfm2Engine reads
    (src/lfm2-engine.js:15-47; per-layer head_count_kv, 0 for short-conv
    blocks).  Returns (bytes, {name: offset}, [(name, shape, type, bytes)]);
    with `path`, the file is written there and bytes is None."""
    p = arch + "."
    kvs = [("general.architecture", GGUF_STRING, arch),
           (p + "block_count", 4, cfg["n_layers"]),
           (p + "embedding_length", 4, cfg["H"]),
           (p + "attention.head_count", 4, cfg["n_heads"]),
           (p + "attention.head_count_kv", GGUF_ARRAY,
            (5, [cfg["n_head_kv"] if i in cfg["attn_layers"] else 0 for i in range(cfg["n_layers"])])),
           (p + "attention.layer_norm_rms_epsilon", 6, cfg["eps"]),
           (p + "expert_count", 4, cfg["E"]),
           (p + "expert_used_count", 4, cfg["K"]),
           (p + "expert_feed_forward_length", 4, cfg["F"]),
           (p + "leading_dense_block_count", 4, cfg["n_dense"]),
           (p + "shortconv.l_cache", 4, cfg["l_cache"]),
           (p + "context_length", 4, cfg["ctx"]),
           (p + "rope.freq_base", 6, cfg["rope_base"])]
    tensors = lfm2_tensors(seed, cfg, **kw)
    if path is not None:
        return None, gguf_write(path, kvs, tensors), tensors
    data, offs = gguf_file(kvs, tensors)
    return data, offs, tensors
