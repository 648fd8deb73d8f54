#!/usr/bin/env python3
"""Write the golden fixtures of this directory.

The reference ships no tests, golden vectors or fixtures for its MoE path, so
these vectors come from the two independent CPU restatements of it in
oracle/: the C oracle (qq_oracle.c) and the Node-12 restatement (moe_ref.js,
the reference's own language and number semantics).  Every case is computed
by both and written only if they agree bit for bit.  Inputs are the seeded
synthetic tensors of oracle/synth.py (GGUF Q8_0 bytes, fp32 router, bias).

    python3 tests/golden/make_golden.py      # rewrites tests/golden/*.npz
"""
import json
import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle  # noqa: E402
import synth  # noqa: E402

NODE = shutil.which("node")
REF_JS = os.path.join(ROOT, "oracle", "moe_ref.js")

MOE_CASES = {
    # name: (layer kwargs, seed, T, mask)
    "moe_small": (dict(H=64, F=64, E=8, K=2), 1, 4, None),
    "moe_q8router_nobias": (dict(H=64, F=64, E=16, K=4, bias=None, router_type=synth.TYPE_Q8_0), 2, 3, None),
    "moe_masked": (dict(H=64, F=96, E=8, K=3), 3, 3, "first_two_ranks_of_token0"),
    "moe_zipf_skew": (dict(H=96, F=64, E=12, K=4, bias="zipf"), 4, 6, None),
}
MATVEC_CASES = {
    "matvec_q8_0": (256, 96, 5),
    "matvec_q8_0_ragged": (1000, 7, 6),      # in_dim not a multiple of 32
}


def _js(job, d):
    p = os.path.join(d, "job.json")
    with open(p, "w") as f:
        json.dump(job, f)
    subprocess.run([NODE, REF_JS, "run", p], check=True, timeout=300)


def _save_bin(d, name, arr):
    p = os.path.join(d, name)
    np.ascontiguousarray(arr).tofile(p)
    return p


def moe_case(name, kw, seed, T, mask_rule, d):
    L = synth.moe_layer(seed, **kw)
    x, hid = synth.activations(seed + 100, T, L["H"])
    mask = None
    if mask_rule == "first_two_ranks_of_token0":
        idx, _, _ = oracle.moe_route(L, x)
        mask = {int(idx[0, 0]), int(idx[0, 1])}
    out, idx, w, probs = oracle.moe_ffn(L, x, hid, mask=mask)
    if NODE:
        job = {"kind": "moe", "H": L["H"], "F": L["F"], "E": L["E"], "K": L["K"], "T": T,
               "router": _save_bin(d, "router.bin", L["router"]), "router_type": L["router_type"],
               "bias": _save_bin(d, "bias.bin", L["bias"]) if L["bias"] is not None else None,
               "gate": _save_bin(d, "gate.bin", L["gate"]), "up": _save_bin(d, "up.bin", L["up"]),
               "down": _save_bin(d, "down.bin", L["down"]),
               "x": _save_bin(d, "x.bin", x), "hidden": _save_bin(d, "hidden.bin", hid),
               "mask": sorted(mask) if mask else None,
               "out_hidden": os.path.join(d, "oh.bin"), "out_idx": os.path.join(d, "oi.bin"),
               "out_w": os.path.join(d, "ow.bin"), "out_probs": os.path.join(d, "op.bin")}
        _js(job, d)
        np.testing.assert_array_equal(np.fromfile(job["out_hidden"], np.float32).reshape(T, -1), out)
        np.testing.assert_array_equal(np.fromfile(job["out_idx"], np.int32).reshape(T, -1), idx)
        np.testing.assert_array_equal(np.fromfile(job["out_w"], np.float64).reshape(T, -1), w)
        np.testing.assert_array_equal(np.fromfile(job["out_probs"], np.float32).reshape(T, -1), probs)
    mask_arr = np.zeros(L["E"], np.uint8)
    if mask:
        mask_arr[sorted(mask)] = 1
    np.savez_compressed(
        os.path.join(HERE, name + ".npz"),
        H=L["H"], F=L["F"], E=L["E"], K=L["K"], router_type=L["router_type"],
        router=L["router"], has_bias=L["bias"] is not None,
        bias=L["bias"] if L["bias"] is not None else np.zeros(L["E"], np.float32),
        gate=L["gate"], up=L["up"], down=L["down"], x=x, hidden=hid, mask=mask_arr,
        out_hidden=out, out_idx=idx, out_w=w, out_probs=probs)


def matvec_case(name, in_dim, out_dim, seed, d):
    w, x = synth.matvec_case(seed, in_dim, out_dim)
    y = oracle.matmul_q8_0(w, in_dim, out_dim, x)
    if NODE:
        job = {"kind": "matvec", "in_dim": in_dim, "out_dim": out_dim, "type": 8,
               "weight": _save_bin(d, "w.bin", w), "x": _save_bin(d, "x.bin", x),
               "y": os.path.join(d, "y.bin")}
        _js(job, d)
        np.testing.assert_array_equal(np.fromfile(job["y"], np.float32), y)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), in_dim=in_dim, out_dim=out_dim,
                        weight=w, x=x, y=y)


def main():
    if not NODE:
        print("warning: node not found; fixtures checked against the C oracle only", file=sys.stderr)
    with tempfile.TemporaryDirectory() as d:
        for name, (kw, seed, T, mask) in MOE_CASES.items():
            moe_case(name, kw, seed, T, mask, d)
            print("wrote", name)
        for name, (i, o, seed) in MATVEC_CASES.items():
            matvec_case(name, i, o, seed, d)
            print("wrote", name)


if __name__ == "__main__":
    main()
