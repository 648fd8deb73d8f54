"""GPU: MoE layers loaded straight from GGUF files (qq_gguf_moe_layer) against
the oracle run on the same tensors read back by the oracle's GGUF reader."""
import sys

import numpy as np
import pytest

import gguf_ref
import oracle
import qq_hip
import synth
from _util import gpu_context, moe_delta, rel_l2

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _check(layer, L_ref, x, hid, tol=1e-4):
    out, idx, w, probs = layer.forward(x, hid)
    r_out, r_idx, r_w, r_probs = oracle.moe_ffn(L_ref, x, hid)
    np.testing.assert_array_equal(idx, r_idx)
    np.testing.assert_array_equal(w, r_w)
    np.testing.assert_array_equal(probs, r_probs)
    err = rel_l2(moe_delta(out, hid), moe_delta(r_out, hid))
    _say("gguf layer rel_l2", err)
    assert err < tol


@pytest.mark.parametrize("arch,T", [("lfm2moe", 1), ("lfm2moe", 7), ("qwen3moe", 1), ("qwen3moe", 5)])
def test_gguf_small_blocks(tmp_path, arch, T):
    _say("gguf small", arch, T)
    kw = dict(bias=None, gating="softmax", router_std=0.05) if arch == "qwen3moe" else {}
    layers = [synth.moe_layer(80 + b, H=256, F=96, E=16, K=4, **kw) for b in range(3)]
    data, _ = synth.moe_gguf(layers, arch=arch, K=4, alignment=64)
    path = tmp_path / "m.gguf"
    path.write_bytes(data)
    g = qq_hip.Gguf(path=str(path))
    r = gguf_ref.Reader(data)
    ctx = gpu_context()
    x, hid = synth.activations(90, T, 256)
    for b in (2, 0):
        m = g.moe_layer(ctx, b)
        try:
            L_ref = gguf_ref.moe_layer(r, b)
            assert L_ref["gating"] == layers[b]["gating"]
            _check(m, L_ref, x, hid)
        finally:
            m.release()
    g.close()


def test_gguf_q8_router_and_q8_bias(tmp_path):
    """A Q8_0 router and a Q8_0 expert-bias vector (read as _readWeightF32 does)."""
    rng = np.random.default_rng(91)
    L = synth.moe_layer(92, H=128, F=64, E=8, K=2, router_type=synth.TYPE_Q8_0)
    bias_q8 = synth.q8_0_tensor(rng, 8, 1, scale=0.01 / 64)
    tensors = [("blk.0.ffn_gate_inp.weight", [128, 8], 8, L["router"]),
               ("blk.0.exp_probs_b.bias", [8], 8, bias_q8),
               ("blk.0.ffn_gate_exps.weight", [128, 64, 8], 8, L["gate"]),
               ("blk.0.ffn_up_exps.weight", [128, 64, 8], 8, L["up"]),
               ("blk.0.ffn_down_exps.weight", [64, 128, 8], 8, L["down"])]
    data, _ = synth.gguf_file([("general.architecture", 8, "lfm2moe"), ("lfm2moe.expert_used_count", 4, 2)],
                              tensors)
    path = tmp_path / "q.gguf"
    path.write_bytes(data)
    L_ref = gguf_ref.moe_layer(gguf_ref.Reader(data), 0)
    assert L_ref["bias"] is not None and np.abs(L_ref["bias"]).max() > 0
    m = qq_hip.Gguf(path=str(path)).moe_layer(gpu_context(), 0)
    try:
        x, hid = synth.activations(93, 6, 128)
        _check(m, L_ref, x, hid)
    finally:
        m.release()


def test_gguf_full_lfm2_layer(tmp_path):
    """One LFM2-8B-A1B-shaped block (374 MB of Q8_0 experts) from a file: batch-1
    decode and a 64-token batch against the oracle."""
    L = synth.moe_layer(1)
    data, offs = synth.moe_gguf([L], K=4)
    path = tmp_path / "full.gguf"
    path.write_bytes(data)
    del data
    g = qq_hip.Gguf(path=str(path))
    assert g.moe_params(0) == dict(H=2048, F=1792, E=32, K=4, gating=0, router_type=0, has_bias=1)
    m = g.moe_layer(gpu_context(), 0)
    g.close()                    # the layer holds device copies; the mapping can go
    try:
        x, hid = synth.activations(94, 64, 2048)
        _check(m, L, x[:1], hid[:1])
        _check(m, L, x, hid)
    finally:
        m.release()


def test_gguf_layer_errors(tmp_path):
    L = synth.moe_layer(95, H=64, F=64, E=8, K=2)
    data, _ = synth.moe_gguf([L], K=2)
    g = qq_hip.Gguf(data=data)
    with pytest.raises(qq_hip.QQError, match="no MoE router"):
        g.moe_layer(gpu_context(), 3)
    # the declared tensor runs past the end of the file
    with pytest.raises(qq_hip.QQError, match="past the end"):
        qq_hip.Gguf(data=data[:len(data) - 100]).moe_layer(gpu_context(), 0)
