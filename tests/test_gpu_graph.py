"""Graph capture and replay (qq_capture_begin / qq_capture_end / qq_graph_launch).

A recorded sequence of device-pointer calls, replayed several times with the
program's own eager work and synchronisations between the replays, must give
what the same calls give eagerly, bit for bit (same kernels, same inputs;
every decode call draws a fresh router epoch on the device).  The eager result
itself is checked against the oracle by the parity tests; here the decode
result is also checked against the oracle so a replay that merely repeats a
stale eager result cannot pass.
"""
import sys

import numpy as np
import pytest

import oracle
import qq_hip
import synth
from _util import gpu_context, upload_layer

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("T,mfma,shape", [(1, 0, "small"), (64, 0, "small"), (96, 64, "small"),
                                          (64, 0, "lfm2")])
def test_graph_replay_matches_eager(T, mfma, shape):
    """shape "lfm2": the LFM2-8B-A1B layer, whose 64-token batch routes and
    dispatches in one launch (8 H slices) and streams 112-feature gate/up
    items; "small": H=256, F=192, E=8, K=2 (4 H slices at 64 tokens)."""
    import torch
    _say("graph replay T=%d mfma_min_tokens=%d shape=%s" % (T, mfma, shape))
    ctx = gpu_context()
    ctx.set_mfma_min_tokens(mfma)
    dims = dict(H=256, F=192, E=8, K=2) if shape == "small" else {}
    L1 = synth.moe_layer(31, **dims)
    L2 = synth.moe_layer(32, **dims)
    H, K = L1["H"], L1["K"]
    m1, m2 = upload_layer(ctx, L1), upload_layer(ctx, L2)
    try:
        x, h0 = synth.activations(33, T, H)
        dx, dh0 = _dev(torch, x), _dev(torch, h0)
        xn = torch.empty_like(dx)
        idx = torch.empty((2, T, K), dtype=torch.int32, device="cuda")

        def calls(dh):
            # two layers of a stack: x = rmsnorm(hidden), hidden += MoE(x)
            m1.forward_dev(dx.data_ptr(), dh.data_ptr(), T, idx_ptr=idx[0].data_ptr())
            ctx.rmsnorm_dev(dh.data_ptr(), None, xn.data_ptr(), T, H, 1e-5)
            m2.forward_dev(xn.data_ptr(), dh.data_ptr(), T, idx_ptr=idx[1].data_ptr())

        eager_h = dh0.clone()
        torch.cuda.synchronize()
        calls(eager_h)                       # also sizes the scratch before capture
        ctx.synchronize()
        want_h = eager_h.cpu().numpy()
        want_idx = idx.cpu().numpy()

        dh = dh0.clone()
        torch.cuda.synchronize()
        ctx.capture_begin()
        with pytest.raises(qq_hip.QQError):
            ctx.synchronize()                # refused while recording
        calls(dh)
        g = ctx.capture_end()
        try:
            for rep in range(3):
                dh.copy_(dh0)
                idx.zero_()
                torch.cuda.synchronize()
                g.launch()
                ctx.synchronize()
                got_h = dh.cpu().numpy()
                assert np.array_equal(got_h, want_h), ("replay", rep)
                assert np.array_equal(idx.cpu().numpy(), want_idx), ("replay idx", rep)
                # eager work of the program between replays
                tmp = dh0.clone()
                torch.cuda.synchronize()
                m2.forward_dev(dx.data_ptr(), tmp.data_ptr(), T)
                ctx.synchronize()
        finally:
            g.release()

        # the first layer's routing against the oracle (exact on every path)
        _, ref_idx, _, _ = oracle.moe_ffn(L1, x, h0)
        assert np.array_equal(want_idx[0], ref_idx)
    finally:
        ctx.set_mfma_min_tokens(512)
        for m in (m1, m2):
            for t in m._keep:
                t.release()
            m.release()


def test_graph_refuses_host_calls_and_double_begin():
    ctx = gpu_context()
    ctx.capture_begin()
    try:
        with pytest.raises(qq_hip.QQError):
            ctx.capture_begin()
        with pytest.raises(qq_hip.QQError):
            ctx.profile_enable(4)
    finally:
        g = ctx.capture_end()
    g.launch()                               # an empty graph replays as a no-op
    ctx.synchronize()
    g.release()
