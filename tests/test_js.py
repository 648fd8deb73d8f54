"""The Node restatement (oracle/moe_ref.js, the timed CPU baseline) against the
C oracle, bit for bit, on the same raw inputs.

V8's Math.exp is its own port of fdlibm and libm's exp may differ from it in a
last binary64 digit; after the fp32 roundings of the path that only shows at a
rounding-boundary straddle, so equality here is the statistical pin of the
oracle's exp() (see oracle/qq_oracle.c).
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
import synth
from _util import ROOT

NODE = shutil.which("node")
REF_JS = os.path.join(ROOT, "oracle", "moe_ref.js")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def _save(d, name, arr):
    p = os.path.join(d, name)
    np.ascontiguousarray(arr).tofile(p)
    return p


def run_js_moe(tmp_path, L, x, hid, mask=None):
    d = str(tmp_path)
    T = x.shape[0]
    job = {
        "kind": "moe", "H": L["H"], "F": L["F"], "E": L["E"], "K": L["K"], "T": T,
        "router": _save(d, "router.bin", L["router"]), "router_type": L["router_type"],
        "bias": _save(d, "bias.bin", L["bias"]) if L.get("bias") is not None else None,
        "gate": _save(d, "gate.bin", L["gate"]), "up": _save(d, "up.bin", L["up"]),
        "down": _save(d, "down.bin", L["down"]),
        "x": _save(d, "x.bin", x), "hidden": _save(d, "hidden.bin", hid),
        "mask": sorted(mask) if mask else None,
        "gating": L.get("gating", "sigmoid"),
        "out_hidden": os.path.join(d, "o_hidden.bin"), "out_idx": os.path.join(d, "o_idx.bin"),
        "out_w": os.path.join(d, "o_w.bin"), "out_probs": os.path.join(d, "o_probs.bin"),
    }
    jp = os.path.join(d, "job.json")
    with open(jp, "w") as f:
        json.dump(job, f)
    subprocess.run([NODE, REF_JS, "run", jp], check=True, timeout=300)
    out = np.fromfile(job["out_hidden"], np.float32).reshape(T, L["H"])
    idx = np.fromfile(job["out_idx"], np.int32).reshape(T, L["K"])
    w = np.fromfile(job["out_w"], np.float64).reshape(T, L["K"])
    probs = np.fromfile(job["out_probs"], np.float32).reshape(T, L["E"])
    return out, idx, w, probs


@pytest.mark.parametrize("case", [
    dict(seed=1, H=64, F=64, E=8, K=2, T=6),
    dict(seed=2, H=96, F=160, E=6, K=3, T=4, bias=None),
    dict(seed=3, H=128, F=64, E=16, K=4, T=5, router_type=synth.TYPE_Q8_0),
    dict(seed=4, H=100, F=50, E=5, K=5, T=3),
    dict(seed=5, H=2048, F=1792, E=32, K=4, T=2),
    dict(seed=7, H=128, F=96, E=64, K=8, T=5, bias=None, gating="softmax", router_std=0.2),
    dict(seed=8, H=2048, F=768, E=128, K=8, T=2, bias=None, gating="softmax"),
    dict(seed=9, H=96, F=64, E=16, K=4, T=4, bias=None, gating="softmax",
         router_type=synth.TYPE_Q8_0),
])
def test_js_restatement_matches_c_oracle(tmp_path, case):
    case = dict(case)
    seed, T = case.pop("seed"), case.pop("T")
    L = synth.moe_layer(seed, **case)
    x, hid = synth.activations(seed + 100, T, L["H"])
    j = run_js_moe(tmp_path, L, x, hid)
    c = oracle.moe_ffn(L, x, hid)
    for a, b in zip(j, c):
        np.testing.assert_array_equal(a, b)


def test_js_restatement_mask(tmp_path):
    L = synth.moe_layer(6, H=64, F=64, E=8, K=3)
    x, hid = synth.activations(106, 5, 64)
    idx, _, _ = oracle.moe_route(L, x)
    mask = {int(idx[0, 0]), int(idx[2, 2])}
    j = run_js_moe(tmp_path, L, x, hid, mask=mask)
    c = oracle.moe_ffn(L, x, hid, mask=mask)
    np.testing.assert_array_equal(j[0], c[0])


def test_js_matvec_matches_c_oracle(tmp_path):
    rng = np.random.default_rng(7)
    d = str(tmp_path)
    for in_dim, out_dim, typ in ((1024, 3072, 8), (70, 9, 8), (200, 11, 0)):
        if typ == 8:
            w = synth.q8_0_tensor(rng, in_dim, out_dim)
        else:
            w = rng.standard_normal((out_dim, in_dim)).astype(np.float32)
        x = rng.standard_normal(in_dim).astype(np.float32)
        job = {"kind": "matvec", "in_dim": in_dim, "out_dim": out_dim, "type": typ,
               "weight": _save(d, "w.bin", w), "x": _save(d, "x.bin", x),
               "y": os.path.join(d, "y.bin")}
        with open(os.path.join(d, "job.json"), "w") as f:
            json.dump(job, f)
        subprocess.run([NODE, REF_JS, "run", os.path.join(d, "job.json")], check=True, timeout=120)
        y = np.fromfile(job["y"], np.float32)
        np.testing.assert_array_equal(y, oracle.matmul_generic(typ, w, in_dim, out_dim, x))


ADDON_EXPORTS = ["init", "lastError", "uploadQ80", "matvec", "moeCreate", "moeSetGating", "moeForward",
                 "ggufOpen", "ggufTensors", "ggufMoeParams", "ggufMoeLayer", "lfm2Create", "lfm2Info",
                 "lfm2Forward", "lfm2Reset", "bufAlloc", "bufWrite", "bufRead", "synchronize", "setWaitLimit",
                 "moeForwardDev", "matvecDev", "rmsnormDev", "release"]


def test_addon_exports():
    code = "const a=require(%r); console.log(JSON.stringify(Object.keys(a)))" % os.path.join(
        ROOT, "qwenqwen3.js_amd", "qq_napi.node")
    p = subprocess.run([NODE, "-e", code], capture_output=True, text=True, timeout=60, check=True)
    assert sorted(json.loads(p.stdout)) == sorted(ADDON_EXPORTS)


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-device error path")
def test_install_fails_loudly_without_device():
    code = ("const qq=require(%r); const scope={matmulGeneric: function(){return 'cpu'}};"
            "try { qq.install(scope, {device: 0}); console.log('installed'); }"
            "catch (e) { console.log('threw: ' + e.message + ' | ' + scope.matmulGeneric()); }"
            % os.path.join(ROOT, "qwenqwen3.js_amd", "js"))
    p = subprocess.run([NODE, "-e", code], capture_output=True, text=True, timeout=60, check=True)
    out = p.stdout.strip()
    assert out.startswith("threw: qq_init failed"), out
    assert out.endswith("| cpu")   # nothing was rebound


def test_addon_gguf_reader_matches_oracle(tmp_path):
    """ggufOpen / ggufTensors / ggufMoeParams need no device: the addon's view of
    a synthetic two-block file equals the oracle's GGUFReader restatement."""
    import gguf_ref
    L = synth.moe_layer(13, H=64, F=32, E=8, K=2)
    data, _ = synth.moe_gguf([L, L], K=3, alignment=64)
    path = tmp_path / "m.gguf"
    path.write_bytes(data)
    code = ("const a=require(%r); const g=a.ggufOpen(%r);"
            "console.log(JSON.stringify({t:a.ggufTensors(g), p:a.ggufMoeParams(g,1,0,-1)}));"
            "a.release(g); let e=''; try { a.ggufOpen(%r); } catch (x) { e=String(x); }"
            "console.log(JSON.stringify(e));") % (
        os.path.join(ROOT, "qwenqwen3.js_amd", "qq_napi.node"), str(path), str(path) + ".missing")
    p = subprocess.run([NODE, "-e", code], capture_output=True, text=True, timeout=60, check=True)
    lines = p.stdout.strip().splitlines()
    got = json.loads(lines[0])
    r = gguf_ref.Reader(data)
    assert got["t"] == [dict(name=t["name"], shape=t["shape"], type=t["type"], offset=t["offset"],
                             nbytes=t["nbytes"]) for t in r.tensors]
    H, F, E, K, gating, rtype, has_bias = gguf_ref.moe_params(r, 1)
    assert got["p"] == dict(H=H, F=F, E=E, K=K, gating=gating, routerType=rtype, hasBias=has_bias)
    assert K == 3 and "cannot open" in json.loads(lines[1])
