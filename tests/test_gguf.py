"""GGUF reader on the CPU: the oracle's restatement of GGUFReader
(oracle/gguf_ref.py, src/gguf.js) pinned by a hand-assembled file and by
round trips of oracle/synth.py's writer, and the library's native reader
(csrc/gguf.cpp, include/qq_gguf.h) checked against the oracle."""
import math
import struct

import numpy as np
import pytest

import gguf_ref
import qq_hip
import synth


def _kat_file():
    """One string KV, one i32-array KV and one F32 [3, 5] tensor; every offset
    spelled out (GGUF v3 layout, little-endian)."""
    b = b"GGUF" + struct.pack("<IQQ", 3, 1, 2)                          # 0..24
    b += struct.pack("<Q", 20) + b"general.architecture"                # 24..52
    b += struct.pack("<I", 8) + struct.pack("<Q", 7) + b"lfm2moe"       # 52..71
    b += struct.pack("<Q", 3) + b"a.x"                                  # 71..82
    b += struct.pack("<I", 9) + struct.pack("<IQ", 5, 2) + struct.pack("<ii", -1, 7)   # 82..106
    b += struct.pack("<Q", 1) + b"t" + struct.pack("<I", 2)             # 106..119
    b += struct.pack("<QQ", 3, 5) + struct.pack("<IQ", 0, 0)            # 119..147
    assert len(b) == 147
    b += bytes(160 - 147)                                               # data at 160 (32-aligned)
    b += np.arange(15, dtype="<f4").tobytes()
    return b


def _native_view(g):
    """Everything the native reader reports, in the oracle's terms."""
    kvs = {}
    for i in range(g.header()["kv_count"]):
        k, t, v = g.kv(i)
        kvs.setdefault(k, (t, v))
    return g.header(), g.tensors(), kvs


def _oracle_view(r):
    kvs = {}
    for i, (k, t, _) in enumerate(r.kvs):
        v = r.kv_value(i)
        if t == 9:
            et = struct.unpack_from("<I", r.buf, r.kvs[i][2])[0]
            v = (et, len(v), None if et in (8, 9) else [float(x) for x in v])
        elif t != 8:
            v = float(v)
        kvs.setdefault(k, (t, v))
    ts = [dict(name=t["name"], shape=list(t["shape"]), type=t["type"], offset=t["offset"],
               nbytes=t["nbytes"]) for t in r.tensors]
    return ts, kvs


def _same(data):
    r = gguf_ref.Reader(data)
    g = qq_hip.Gguf(data=data)
    hd, ts, kvs = _native_view(g)
    ots, okvs = _oracle_view(r)
    assert hd["version"] == r.version and hd["file_size"] == len(data)
    assert hd["alignment"] == r.alignment and hd["data_offset"] == r.data_offset
    assert ts == ots
    assert kvs.keys() == okvs.keys()
    for k in kvs:
        a, b = kvs[k], okvs[k]
        assert a[0] == b[0], k
        if isinstance(a[1], float) and math.isnan(a[1]):
            assert math.isnan(b[1])
        else:
            assert a[1] == b[1], k
    return r, g


# ---------------------------------------------------------------- the oracle, pinned

def test_known_answer_file():
    r = gguf_ref.Reader(_kat_file())
    assert r.version == 3 and r.header()["tensor_count"] == 1 and r.header()["kv_count"] == 2
    assert r.key_value("general.architecture") == "lfm2moe"
    assert r.key_value("a.x") == [-1, 7]
    assert r.key_value("missing", "dflt") == "dflt"
    assert r.alignment == 32 and r.data_offset == 160
    m = r.tensor_meta("t")
    assert m == dict(offset=160, nbytes=256, shape=[3, 5], type=0)
    assert r.tensor_meta("u") is None
    np.testing.assert_array_equal(r.tensor_bytes("t", 60).view("<f4"), np.arange(15, dtype=np.float32))


ALL_KVS = [
    ("k.u8", 0, 250), ("k.i8", 1, -5), ("k.u16", 2, 65000), ("k.i16", 3, -30000),
    ("k.u32", 4, 4000000000), ("k.i32", 5, -2000000000), ("k.f32", 6, 1.5), ("k.bool", 7, True),
    ("k.str", 8, "héllo"), ("k.empty", 8, ""), ("k.u64", 10, 2 ** 53 + 2), ("k.i64", 11, -(2 ** 40)),
    ("k.f64", 12, math.pi),
    ("k.arr_i32", 9, (5, [1, -2, 3])), ("k.arr_str", 9, (8, ["a", "bc", ""])),
    ("k.arr_nested", 9, (9, [(4, [1, 2]), (8, ["x"])])), ("k.arr_empty", 9, (12, [])),
]


@pytest.mark.parametrize("alignment", [None, 64, 1, 4096])
def test_writer_round_trip(alignment):
    rng = np.random.default_rng(5)
    tensors = [("a", [7], 0, rng.standard_normal(7).astype(np.float32)),
               ("b.weight", [64, 3], 8, synth.q8_0_tensor(rng, 64, 3)),
               ("c", [2, 3, 4], 1, np.zeros(24, np.float16)),
               ("d", [100], 99, np.zeros(400, np.uint8))]          # unknown type: taken as F32
    data, offs = synth.gguf_file(ALL_KVS, tensors, alignment=alignment)
    r = gguf_ref.Reader(data)
    assert r.alignment == (alignment or 32)
    for k, t, v in ALL_KVS:
        got = r.key_value(k)
        if t == 9 and v[0] == 9:
            assert got == [list(x[1]) for x in v[1]]
        elif t == 9:
            assert got == list(v[1])
        elif t == 6:
            assert got == np.float32(v)
        else:
            assert got == v, k
    for name, shape, typ, arr in tensors:
        m = r.tensor_meta(name)
        assert m["offset"] == offs[name] and m["shape"] == shape and m["type"] == typ
        assert m["nbytes"] % 256 == 0 and m["nbytes"] >= arr.nbytes
        np.testing.assert_array_equal(r.tensor_bytes(name, arr.nbytes), arr.view(np.uint8).ravel())
    assert r.tensor_meta("d")["nbytes"] == 512           # 100 elements * 4, rounded to 256
    assert r.tensor_meta("b.weight")["nbytes"] == 256    # 6 blocks * 34 = 204


def test_oracle_moe_layer_reads_back_the_tensors():
    L = synth.moe_layer(3, H=64, F=96, E=8, K=2)
    data, _ = synth.moe_gguf([L, L], K=2)
    r = gguf_ref.Reader(data)
    R = gguf_ref.moe_layer(r, 1)
    for k in ("H", "F", "E", "K", "router_type", "gating"):
        assert R[k] == L[k], k
    for k in ("router", "gate", "up", "down"):
        np.testing.assert_array_equal(R[k], np.asarray(L[k]).view(np.uint8).ravel())
    np.testing.assert_array_equal(R["bias"], L["bias"])


def test_read_weight_f32_q8_0_bias():
    rng = np.random.default_rng(9)
    raw = synth.q8_0_tensor(rng, 40, 1)
    dense = synth.q8_0_dequant(raw, 40, 1)[0, 0]
    np.testing.assert_array_equal(gguf_ref.read_weight_f32(8, raw, 40), dense.astype(np.float32))


def test_oracle_errors_match_the_reference_messages():
    with pytest.raises(gguf_ref.GGUFError, match="Invalid signature: GGUX"):
        gguf_ref.Reader(b"GGUX" + bytes(40))
    bad = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    with pytest.raises(gguf_ref.GGUFError, match="Unknown KV type: 13"):
        gguf_ref.Reader(bad + bytes(16))
    r = gguf_ref.Reader(synth.gguf_file([], [], version=2)[0])
    assert r.version == 2 and r.warnings


# ---------------------------------------------------------------- native reader vs oracle

def test_native_known_answer_file():
    r, g = _same(_kat_file())
    assert g.find_tensor("t") == 0 and g.find_tensor("u") == -1
    assert g.find_key("a.x") == 1 and g.find_key("nope") == -1
    assert g.tensors()[0]["offset"] == 160


@pytest.mark.parametrize("alignment", [None, 64, 1])
def test_native_matches_oracle(alignment):
    rng = np.random.default_rng(6)
    tensors = [("x%d" % i, [32 * (i + 1), 2], 8, synth.q8_0_tensor(rng, 32 * (i + 1), 2)) for i in range(5)]
    tensors += [("dup", [4], 0, np.ones(4, np.float32)), ("dup", [8], 0, np.zeros(8, np.float32)),
                ("q4k", [512, 2], 12, np.zeros(576, np.uint8)), ("odd", [100], 99, np.zeros(400, np.uint8))]
    data, _ = synth.gguf_file(ALL_KVS + [("k.u32", 4, 1)], tensors, alignment=alignment)
    r, g = _same(data)
    assert g.find_tensor("dup") == 5               # first of equal names, as getTensorMetaByName
    assert g.kv(g.find_key("k.u32"))[2] == 4000000000.0   # first of equal keys, as findKey
    assert g.kv(g.find_key("k.u64"))[2] == float(2 ** 53 + 2)   # Number() rounding


def test_native_from_file(tmp_path):
    L = synth.moe_layer(4, H=64, F=64, E=8, K=2)
    data, _ = synth.moe_gguf([L], K=2, alignment=64)
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    g1, g2 = qq_hip.Gguf(path=str(p)), qq_hip.Gguf(data=data)
    assert g1.tensors() == g2.tensors() and g1.header() == g2.header()


def test_native_version_other_than_3_is_read():
    data, _ = synth.gguf_file([("general.architecture", 8, "lfm2moe")], [], version=2)
    assert qq_hip.Gguf(data=data).header()["version"] == 2


@pytest.mark.parametrize("data,msg", [
    (b"GGUX" + bytes(40), "Invalid signature: GGUX"),
    (b"", "Invalid signature"),
    (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13) + bytes(16),
     "Unknown KV type: 13"),
    (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", 9, 77, 1)
     + bytes(16), "Unknown KV type: 77"),
    (b"GGUF" + struct.pack("<I", 3), "truncated"),
    (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1000) + b"key", "truncated"),
    (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", 9, 4, 2 ** 60),
     "truncated"),
    (b"GGUF" + struct.pack("<IQQ", 3, 3, 0) + struct.pack("<Q", 1) + b"t", "truncated"),
])
def test_native_errors(data, msg):
    with pytest.raises(qq_hip.QQError, match=msg):
        qq_hip.Gguf(data=data)


def test_native_truncated_everywhere():
    """Every prefix of a valid file is either read whole or refused; never a crash."""
    L = synth.moe_layer(8, H=32, F=32, E=4, K=2)
    data, _ = synth.moe_gguf([L], K=2)
    r = gguf_ref.Reader(data)
    for n in range(0, r.data_offset + 1, 3):
        try:
            g = qq_hip.Gguf(data=data[:n])
        except qq_hip.QQError:
            continue
        assert len(g.tensors()) == len(r.tensors)


@pytest.mark.parametrize("arch,K,kv_k,exp_K,exp_gating", [
    ("lfm2moe", None, 0, 4, 0),      # no expert_used_count: LFM2 default
    ("lfm2moe", 3, 0, 3, 0),
    ("lfm2", 2, 0, 2, 0),
    ("qwen3moe", None, 0, 8, 1),     # Qwen3 default
    ("qwen3moe", 6, 0, 6, 1),
    ("lfm2moe", 3, 2, 2, 0),         # an explicit K wins
])
def test_native_moe_params(arch, K, kv_k, exp_K, exp_gating):
    L = synth.moe_layer(10, H=64, F=32, E=16, K=4)
    if arch == "qwen3moe":
        L["bias"] = None
    data, _ = synth.moe_gguf([L, L], arch=arch, K=K)
    g, r = qq_hip.Gguf(data=data), gguf_ref.Reader(data)
    p = g.moe_params(1, K=kv_k)
    assert (p["H"], p["F"], p["E"], p["K"], p["gating"]) == (64, 32, 16, exp_K, exp_gating)
    H, F, E, K2, gating, rtype, has_bias = gguf_ref.moe_params(r, 1, K=kv_k)
    assert (H, F, E, K2, gating, rtype, has_bias) == (p["H"], p["F"], p["E"], p["K"], p["gating"],
                                                      p["router_type"], p["has_bias"])
    assert p["has_bias"] == (1 if arch.startswith("lfm2") else 0)
    # an explicit gating overrides the architecture; softmax never uses the bias
    assert g.moe_params(1, gating=1)["has_bias"] == 0


def test_native_moe_params_errors():
    L = synth.moe_layer(12, H=64, F=32, E=8, K=2)
    data, _ = synth.moe_gguf([L], K=2)
    g = qq_hip.Gguf(data=data)
    with pytest.raises(qq_hip.QQError, match="no MoE router"):
        g.moe_params(1)
    with pytest.raises(qq_hip.QQError, match="unknown gating"):
        g.moe_params(0, gating=5)
    rng = np.random.default_rng(1)
    t = [("blk.0.ffn_gate_inp.weight", [64, 8], 0, np.zeros(512, np.float32)),
         ("blk.0.ffn_gate_exps.weight", [64, 32, 8], 8, synth.q8_0_tensor(rng, 64, 32, 8)),
         ("blk.0.ffn_up_exps.weight", [64, 32, 8], 8, synth.q8_0_tensor(rng, 64, 32, 8)),
         ("blk.0.ffn_down_exps.weight", [32, 48, 8], 8, synth.q8_0_tensor(rng, 32, 48, 8))]
    with pytest.raises(qq_hip.QQError, match="shapes do not match"):
        qq_hip.Gguf(data=synth.gguf_file([], t)[0]).moe_params(0)
    t[3] = ("blk.0.ffn_down_exps.weight", [32, 64, 8], 0, np.zeros(32 * 64 * 8, np.float32))
    with pytest.raises(qq_hip.QQError, match="must be Q8_0"):
        qq_hip.Gguf(data=synth.gguf_file([], t)[0]).moe_params(0)
