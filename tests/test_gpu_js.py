"""GPU: the JavaScript drop-in (Node-API addon over the C ABI) against the
Node restatement of the reference, through the reference's own call surface."""
import json
import os
import shutil
import subprocess

import pytest

from _util import ROOT

NODE = shutil.which("node")
CHECK = os.path.join(ROOT, "tests", "js", "dropin_check.js")

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(NODE is None, reason="node is not installed")]


@pytest.mark.parametrize("shape", [(256, 96, 16, 4, 6), (2048, 1792, 32, 4, 3), (100, 50, 5, 5, 4),
                                   (256, 96, 16, 4, 6, "softmax"),       # Qwen3Engine._moEFFN
                                   (2048, 768, 128, 8, 2, "softmax")])   # Qwen3-30B-A3B layer shape
def test_js_dropin(shape):
    print("js drop-in", shape, flush=True)
    p = subprocess.run([NODE, CHECK] + [str(v) for v in shape], capture_output=True, text=True, timeout=240)
    assert p.stdout.strip(), p.stderr
    res = json.loads(p.stdout.strip().splitlines()[-1])
    bad = [c for c in res["checks"] if not c["ok"]]
    assert res["ok"] and not bad, (bad, p.stderr[-2000:])
    assert res["max_rel_l2"] < 1e-4


@pytest.mark.parametrize("arch", ["lfm2moe", "qwen3moe"])
def test_js_attach_gguf(tmp_path, arch):
    """MoEDevice.attachGGUF: _moEFFN with the layers bound from a GGUF file."""
    import synth
    print("js gguf", arch, flush=True)
    kw = dict(bias=None, gating="softmax", router_std=0.05) if arch == "qwen3moe" else {}
    layers = [synth.moe_layer(60 + b, H=256, F=96, E=16, K=4, **kw) for b in range(2)]
    data, _ = synth.moe_gguf(layers, arch=arch, K=4)
    path = tmp_path / "m.gguf"
    path.write_bytes(data)
    p = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "gguf_check.js"), str(path),
                        "softmax" if arch == "qwen3moe" else "sigmoid", "3"],
                       capture_output=True, text=True, timeout=240)
    assert p.stdout.strip(), p.stderr
    res = json.loads(p.stdout.strip().splitlines()[-1])
    bad = [c for c in res["checks"] if not c["ok"]]
    assert res["ok"] and not bad, (bad, p.stderr[-2000:])
    assert res["max_rel_l2"] < 1e-4


@pytest.mark.parametrize("gating", ["sigmoid", "softmax"])
def test_js_gpu_engine(gating):
    """Lfm2GPUEngine / Qwen3GPUEngine._moEFFNGPU and _readbackRoutingData rebound by
    install() for an engine whose buffers are the device's (src/webgpu.js:1882-1945,
    :878-990), against the CPU engine's restatement."""
    print("js gpu engine", gating, flush=True)
    p = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "gpu_engine_check.js"),
                        "256", "96", "16", "4", "3", gating], capture_output=True, text=True, timeout=240)
    assert p.stdout.strip(), p.stderr
    res = json.loads(p.stdout.strip().splitlines()[-1])
    bad = [c for c in res["checks"] if not c["ok"]]
    assert res["ok"] and not bad, (bad, p.stderr[-2000:])
    assert res["max_rel_l2"] < 1e-4


def test_js_lfm2_forward(tmp_path):
    """MoEDevice.attachLfm2Forward: Lfm2Engine.forward / resetKVCache run the whole
    token on the device from the attached file, against oracle/lfm2_ref.js."""
    import synth
    import _lfm2
    print("js lfm2 forward", flush=True)
    cfg = synth.LFM2_TINY
    path, offs, tensors = _lfm2.write_model(tmp_path, 9, cfg)
    job = {"gguf": path, "kv": _lfm2.kv_dict(cfg), "tokens": [3, 77, 250, 1, 9, 120],
           "tensors": {n: {"offset": offs[n], "shape": s, "type": t} for n, s, t, _ in tensors}}
    jp = tmp_path / "job.json"
    jp.write_text(json.dumps(job))
    p = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "lfm2_check.js"), str(jp)],
                       capture_output=True, text=True, timeout=240)
    assert p.stdout.strip(), p.stderr
    res = json.loads(p.stdout.strip().splitlines()[-1])
    bad = [c for c in res["checks"] if not c["ok"]]
    assert res["ok"] and not bad, (bad, p.stderr[-2000:])
    assert res["max_rel_l2"] < 1e-4
