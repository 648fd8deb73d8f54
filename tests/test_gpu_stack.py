"""The 22-layer LFM2-8B-A1B-shaped Q8_0 MoE stack and full-size prefill chunks
on the GPU (src/lfm2-engine.js:232-258: per MoE block `x = rmsnorm(hidden)`,
then `hidden += _moEFFN(x)`; a prompt is T sequential calls, :550-555).

* Decode: 22 independently seeded full-shape layers resident in HBM, two
  tokens each run through all 22 layers back to back on the device
  (qq_moe_forward_norm_dev), against the oracle's chain
  (oracle.rmsnorm_unit + oracle.moe_ffn per layer): top-4 indices bit-exact
  at every layer, the stack's total contribution within 1e-4 relative L2.
  The same tokens through the one-launch stack (qq_moe_stack_forward_dev):
  bit-equal to the layer-by-layer chain, routing and residual.
* Prefill: the same 22 layers chained over one 4096-token chunk (the fp16
  MFMA path, layer after layer through the stack entry point's batch path):
  every row's routing at every layer bit-exact against the oracle's router fed
  with the GPU's own input residual for that layer, and 16 sampled rows per
  layer against oracle.moe_ffn on that same input within 1e-2.
* Stacks of small layers (ffn_norm weights, expert masks, softmax gating,
  token batches): the one-launch stack bit-equal to the chain of
  qq_moe_forward_norm_dev calls, routing against the oracle.
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


@pytest.fixture(scope="module")
def stack22():
    """22 independently seeded full-shape layers: the oracle's dicts and the
    device layers (8.2 GB resident), shared by the tests of this module."""
    ctx = gpu_context()
    Ls, layers = [], []
    try:
        for l in range(N_LAYERS):
            Ls.append(synth.moe_layer(5000 + l))
            layers.append(upload_layer(ctx, Ls[-1]))
        _say("22 layers bound")
        yield Ls, layers
    finally:
        for m in layers:
            _release(m)


def test_stack22_decode(stack22):
    import torch
    ctx = gpu_context()
    Ls, layers = stack22
    n_tok = 2
    _, hid = synth.activations(501, n_tok, 2048)
    h_ref = hid.copy()
    idx_ref = np.empty((n_tok, N_LAYERS, 4), np.int32)
    for l, L in enumerate(Ls):
        for t in range(n_tok):
            x = oracle.rmsnorm_unit(h_ref[t], EPS)
            out, idx, _, _ = oracle.moe_ffn(L, x[None], h_ref[t:t + 1])
            h_ref[t] = out[0]
            idx_ref[t, l] = idx[0]
    HID = torch.from_numpy(hid.copy()).cuda()
    IDX = torch.full((n_tok, N_LAYERS, 4), -1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    for t in range(n_tok):
        for l, m in enumerate(layers):
            m.forward_norm_dev(HID[t].data_ptr(), 1, eps=EPS, idx_ptr=IDX[t, l].data_ptr())
    ctx.synchronize()
    got_idx, got = IDX.cpu().numpy(), HID.cpu().numpy()
    _say("one-launch stack")
    stack = ctx.moe_stack(layers)
    try:
        HID2 = torch.from_numpy(hid.copy()).cuda()
        IDX2 = torch.full((n_tok, N_LAYERS, 4), -1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        for t in range(n_tok):
            stack.forward_dev(HID2[t].data_ptr(), 1, eps=EPS, idx_ptr=IDX2[t].data_ptr())
        ctx.synchronize()
        got2_idx, got2 = IDX2.cpu().numpy(), HID2.cpu().numpy()
    finally:
        stack.release()
    np.testing.assert_array_equal(got_idx, idx_ref)
    np.testing.assert_array_equal(got2_idx, idx_ref)
    assert np.array_equal(got2.view(np.uint32), got.view(np.uint32))
    for t in range(n_tok):
        err = rel_l2(got[t].astype(np.float64) - hid[t], h_ref[t].astype(np.float64) - hid[t])
        _say("token", t, "stack rel_l2", err)
        assert err < 1e-4, (t, err)


def test_stack22_prefill_chain(stack22):
    """The 22 layers over one 4096-token chunk (qq_moe_stack_forward_dev,
    T = 4096: the fp16 MFMA path layer after layer).  The GPU's input residual
    of each layer is read back and fed to the oracle: routing of all 4096 rows
    bit-exact (idx, w, probs), and 16 sampled rows per layer within 1e-2 of
    oracle.moe_ffn on the same input."""
    import torch
    ctx = gpu_context()
    Ls, layers = stack22
    T = 4096
    _, hid = synth.activations(610, T, 2048)
    rows = np.sort(np.random.default_rng(611).choice(T, 16, replace=False))
    HID = torch.from_numpy(hid.copy()).cuda()
    IDX = torch.empty((T, 4), dtype=torch.int32, device="cuda")
    W = torch.empty((T, 4), dtype=torch.float64, device="cuda")
    P = torch.empty((T, 32), dtype=torch.float32, device="cuda")
    worst = 0.0
    for l, (L, m) in enumerate(zip(Ls, layers)):
        torch.cuda.synchronize()
        h_in = HID.cpu().numpy()
        stack = ctx.moe_stack([m])      # one layer: the same calls the 22-layer chunk makes
        try:
            stack.forward_dev(HID.data_ptr(), T, eps=EPS, idx_ptr=IDX.data_ptr(), w_ptr=W.data_ptr(),
                              probs_ptr=P.data_ptr())
            ctx.synchronize()
        finally:
            stack.release()
        h_out = HID.cpu().numpy()
        x = np.stack([oracle.rmsnorm_unit(r, EPS) for r in h_in])
        r_idx, r_w, r_p = oracle.moe_route(L, x)
        np.testing.assert_array_equal(IDX.cpu().numpy(), r_idx)
        np.testing.assert_array_equal(W.cpu().numpy(), r_w)
        np.testing.assert_array_equal(P.cpu().numpy(), r_p)
        ref, _, _, _ = oracle.moe_ffn(L, x[rows], h_in[rows])
        err = rel_l2(h_out[rows].astype(np.float64) - h_in[rows], ref.astype(np.float64) - h_in[rows])
        worst = max(worst, err)
        _say("layer", l, "sampled rows rel_l2", err)
        assert err < 1e-2, (l, err)
    _say("worst layer", worst)


@pytest.mark.parametrize("shape,n,T,masked,weighted", [
    (dict(H=256, F=192, E=16, K=4), 5, 1, False, True),
    (dict(H=256, F=192, E=16, K=4), 5, 1, True, True),
    (dict(H=2048, F=768, E=128, K=8, bias=None, gating="softmax"), 3, 1, False, False),
    (dict(H=512, F=256, E=32, K=4), 4, 3, True, True),
    (dict(H=2048, F=1792, E=32, K=4), 3, 2, False, True),
])
def test_stack_matches_layer_chain(shape, n, T, masked, weighted):
    """qq_moe_stack_forward_dev equals qq_moe_forward_norm_dev layer after
    layer, bit for bit (T = 1: the one-launch stack; T > 1: the batch path per
    layer); without weights and masks the routing equals the oracle's chain."""
    import torch
    _say("stack", shape, n, T, masked, weighted)
    ctx = gpu_context()
    H, E, K = shape["H"], shape["E"], shape["K"]
    Ls = [synth.moe_layer(7000 + 13 * l, **shape) for l in range(n)]
    layers = [upload_layer(ctx, L) for L in Ls]
    rng = np.random.default_rng(n * 100 + T)
    nw = [torch.from_numpy(rng.uniform(0.5, 1.5, H).astype(np.float32)).cuda() for _ in range(n)] \
        if weighted else [None] * n
    mask = [1, 5] if masked else None
    _, hid = synth.activations(77 + n, T, H)
    stack = ctx.moe_stack(layers, [None if w is None else w.data_ptr() for w in nw])
    try:
        A = torch.from_numpy(hid.copy()).cuda()
        B = torch.from_numpy(hid.copy()).cuda()
        IA = torch.full((n, T, K), -1, dtype=torch.int32, device="cuda")
        IB = torch.full((n, T, K), -1, dtype=torch.int32, device="cuda")
        WB = torch.zeros((n, T, K), dtype=torch.float64, device="cuda")
        PB = torch.zeros((n, T, E), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        for l, m in enumerate(layers):
            m.forward_norm_dev(A.data_ptr(), T, norm_w_ptr=None if nw[l] is None else nw[l].data_ptr(),
                               eps=EPS, mask=mask, idx_ptr=IA[l].data_ptr())
        stack.forward_dev(B.data_ptr(), T, eps=EPS, mask=mask, idx_ptr=IB.data_ptr(), w_ptr=WB.data_ptr(),
                          probs_ptr=PB.data_ptr())
        ctx.synchronize()
        a, b = A.cpu().numpy(), B.cpu().numpy()
        ia, ib = IA.cpu().numpy(), IB.cpu().numpy()
    finally:
        stack.release()
        for m in layers:
            _release(m)
    np.testing.assert_array_equal(ib, ia)
    assert np.array_equal(b.view(np.uint32), a.view(np.uint32))
    if not weighted and not masked:
        h = hid.copy()
        for l, L in enumerate(Ls):
            x = np.stack([oracle.rmsnorm_unit(r, EPS) for r in h])
            r_idx, r_w, r_p = oracle.moe_route(L, x)
            np.testing.assert_array_equal(ib[l], r_idx)
            if l == 0:
                np.testing.assert_array_equal(WB[l].cpu().numpy(), r_w)
                np.testing.assert_array_equal(PB[l].cpu().numpy(), r_p)
            else:
                # later layers see the GPU's residual, which differs from the
                # oracle chain's by ~1e-7 relative: the weights and
                # probabilities follow it at fp32 level
                np.testing.assert_allclose(WB[l].cpu().numpy(), r_w, rtol=1e-5)
                np.testing.assert_allclose(PB[l].cpu().numpy(), r_p, rtol=1e-5, atol=1e-9)
            h, _, _, _ = oracle.moe_ffn(L, x, h)
        err = rel_l2(b.astype(np.float64) - hid, h.astype(np.float64) - hid)
        _say("stack rel_l2 vs oracle", err)
        assert err < 1e-4, err


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
