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
