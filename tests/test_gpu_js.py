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
