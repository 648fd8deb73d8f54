"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the C oracle and the Node restatement, which agree bit for bit on them).

CPU: the C oracle still reproduces every fixture exactly.
GPU: the HIP path through the C ABI against the fixtures: routing outputs
bit-exact, the MoE contribution within 1e-4 relative L2 (all fixtures are
token batches below the MFMA threshold or single tokens, i.e. fp32 paths).
"""
import glob
import os

import numpy as np
import pytest

import oracle
from _util import ROOT, gpu_context, moe_delta, rel_l2, upload_layer

GOLDEN = sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "*.npz")))
MOE = [p for p in GOLDEN if os.path.basename(p).startswith("moe_")]
MATVEC = [p for p in GOLDEN if os.path.basename(p).startswith("matvec_")]


def _layer(z):
    return {"H": int(z["H"]), "F": int(z["F"]), "E": int(z["E"]), "K": int(z["K"]),
            "router_type": int(z["router_type"]), "router": z["router"],
            "bias_type": 0, "bias": z["bias"] if bool(z["has_bias"]) else None,
            "gate": z["gate"], "up": z["up"], "down": z["down"]}


def _mask(z):
    m = z["mask"]
    return {int(e) for e in np.flatnonzero(m)} or None


def test_fixtures_present():
    assert len(MOE) >= 4 and len(MATVEC) >= 2


@pytest.mark.parametrize("path", MOE, ids=os.path.basename)
def test_oracle_reproduces_moe_fixture(path):
    z = np.load(path)
    out, idx, w, probs = oracle.moe_ffn(_layer(z), z["x"], z["hidden"], mask=_mask(z))
    np.testing.assert_array_equal(out, z["out_hidden"])
    np.testing.assert_array_equal(idx, z["out_idx"])
    np.testing.assert_array_equal(w, z["out_w"])
    np.testing.assert_array_equal(probs, z["out_probs"])


@pytest.mark.parametrize("path", MATVEC, ids=os.path.basename)
def test_oracle_reproduces_matvec_fixture(path):
    z = np.load(path)
    y = oracle.matmul_q8_0(z["weight"], int(z["in_dim"]), int(z["out_dim"]), z["x"])
    np.testing.assert_array_equal(y, z["y"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", MOE, ids=os.path.basename)
@pytest.mark.parametrize("tokens", ["batch", "one_by_one"])
def test_gpu_moe_fixture(path, tokens):
    z = np.load(path)
    print("golden", os.path.basename(path), tokens, flush=True)
    ctx = gpu_context()
    m = upload_layer(ctx, _layer(z))
    mask = _mask(z)
    try:
        x, hid = z["x"], z["hidden"]
        if tokens == "batch":
            out, idx, w, probs = m.forward(x, hid, mask=mask)
        else:
            parts = [m.forward(x[t:t + 1], hid[t:t + 1], mask=mask) for t in range(x.shape[0])]
            out, idx, w, probs = (np.concatenate([p[i] for p in parts]) for i in range(4))
    finally:
        for t in m._keep:
            t.release()
        m.release()
    np.testing.assert_array_equal(idx, z["out_idx"])
    np.testing.assert_array_equal(w, z["out_w"])
    np.testing.assert_array_equal(probs, z["out_probs"])
    assert rel_l2(moe_delta(out, hid), moe_delta(z["out_hidden"], hid)) < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("path", MATVEC, ids=os.path.basename)
def test_gpu_matvec_fixture(path):
    z = np.load(path)
    ctx = gpu_context()
    t = ctx.upload_q8_0(z["weight"], int(z["in_dim"]), int(z["out_dim"]))
    try:
        y = t.matvec(z["x"])[0]
    finally:
        t.release()
    assert rel_l2(y, z["y"]) < 1e-4
