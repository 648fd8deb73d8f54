"""The 22-layer LFM2-8B-A1B-shaped Q8_0 MoE stack and full-size prefill chunks
on the GPU (src/lfm2-engine.js:232-258: per MoE block `x = rmsnorm(hidden)`,
then `hidden += _moEFFN(x)`; a prompt is T sequential calls, :550-555).

* Decode: 22 independently seeded full-shape layers resident in HBM, two
  tokens each run through all 22 layers back to back on the device
  (qq_moe_forward_norm_dev), against the oracle's chain
  (oracle.rmsnorm_unit + oracle.moe_ffn per layer): top-4 indices bit-exact
  at every layer, the stack's total contribution within 1e-4 relative L2.
* Prefill: one full-shape layer at T = 4096 (the largest chunk) and T = 4100
  (a 4096-row chunk on the fp16 MFMA path and a 4-row chunk on the fp32
  path): routing bit-exact on every row against the oracle, every row's
  output against the float64 dense restatement (tests/_util.py), within
  1e-2 on the MFMA rows and 1e-4 on the fp32 rows.
"""
import sys

import numpy as np
import pytest

import oracle
import synth
from _util import dense_moe_f64, full_layer, gpu_context, rel_l2, upload_layer

pytestmark = pytest.mark.gpu

N_LAYERS = 22
EPS = 1e-5


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _release(m):
    for t in m._keep:
        t.release()
    m.release()


def test_stack22_decode():
    import torch
    ctx = gpu_context()
    n_tok = 2
    _, hid = synth.activations(501, n_tok, 2048)
    h_ref = hid.copy()
    idx_ref = np.empty((n_tok, N_LAYERS, 4), np.int32)
    layers = []
    try:
        for l in range(N_LAYERS):
            L = synth.moe_layer(5000 + l)
            layers.append(upload_layer(ctx, L))
            for t in range(n_tok):
                x = oracle.rmsnorm_unit(h_ref[t], EPS)
                out, idx, _, _ = oracle.moe_ffn(L, x[None], h_ref[t:t + 1])
                h_ref[t] = out[0]
                idx_ref[t, l] = idx[0]
            del L
            _say("layer", l, "bound")
        HID = torch.from_numpy(hid.copy()).cuda()
        IDX = torch.full((n_tok, N_LAYERS, 4), -1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        for t in range(n_tok):
            for l, m in enumerate(layers):
                m.forward_norm_dev(HID[t].data_ptr(), 1, eps=EPS, idx_ptr=IDX[t, l].data_ptr())
        ctx.synchronize()
        got_idx, got = IDX.cpu().numpy(), HID.cpu().numpy()
    finally:
        for m in layers:
            _release(m)
    np.testing.assert_array_equal(got_idx, idx_ref)
    for t in range(n_tok):
        err = rel_l2(got[t].astype(np.float64) - hid[t], h_ref[t].astype(np.float64) - hid[t])
        _say("token", t, "stack rel_l2", err)
        assert err < 1e-4, (t, err)


@pytest.mark.parametrize("T", [4096, 4100])
def test_layer_prefill_full_chunks(T):
    import torch
    _say("prefill chunk", T)
    ctx = gpu_context()
    L = full_layer(1)
    _, hid = synth.activations(600 + T, T, 2048)
    x = np.stack([oracle.rmsnorm_unit(r, EPS) for r in hid])
    r_idx, r_w, r_probs = oracle.moe_route(L, x)
    m = upload_layer(ctx, L)
    try:
        HID = torch.from_numpy(hid.copy()).cuda()
        IDX = torch.empty((T, 4), dtype=torch.int32, device="cuda")
        W = torch.empty((T, 4), dtype=torch.float64, device="cuda")
        P = torch.empty((T, 32), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        m.forward_norm_dev(HID.data_ptr(), T, eps=EPS, idx_ptr=IDX.data_ptr(), w_ptr=W.data_ptr(),
                           probs_ptr=P.data_ptr())
        ctx.synchronize()
        got = HID.cpu().numpy()
        np.testing.assert_array_equal(IDX.cpu().numpy(), r_idx)
        np.testing.assert_array_equal(W.cpu().numpy(), r_w)
        np.testing.assert_array_equal(P.cpu().numpy(), r_probs)
    finally:
        _release(m)
    dense = dense_moe_f64(L, x, hid, r_idx, r_w)
    n_mfma = min(T, 4096)
    err = rel_l2(got[:n_mfma].astype(np.float64) - hid[:n_mfma], dense[:n_mfma] - hid[:n_mfma])
    _say("mfma rows rel_l2", err)
    assert err < 1e-2, err
    # no single row far off (a skipped fragment or tile would show here)
    rows = [rel_l2(got[t].astype(np.float64) - hid[t], dense[t] - hid[t]) for t in range(T)]
    _say("worst row", int(np.argmax(rows)), max(rows))
    assert max(rows[:n_mfma]) < 2e-2
    if T > 4096:
        err1 = rel_l2(got[4096:].astype(np.float64) - hid[4096:], dense[4096:] - hid[4096:])
        _say("fp32 rows rel_l2", err1)
        assert err1 < 1e-4, err1
