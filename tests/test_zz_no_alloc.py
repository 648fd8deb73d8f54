"""The allocation-free forward (qq_moe_forward_noalloc_dev) against the arena
forward (qq_moe_forward_dev), both through the C ABI on the same device
buffers: top-K indices and weights bit for bit, the MoE contribution within
1e-6 relative L2 (the same kernels on the same inputs), on two calls in a row
per case -- the second with fewer rows, so it runs over what the first left in
the shared fixed array.  The last row of each call is also checked against the
oracle (1e-4 on the fp32 paths, 1e-2 on the fp16 MFMA path), so agreement
with a broken arena forward cannot pass.  A T whose scratch exceeds the fixed
array is rejected before anything is enqueued.
"""
import sys

import numpy as np
import pytest

import oracle
import qq_hip
import synth
from _util import full_layer, gpu_context, moe_delta, rel_l2, upload_layer

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _release(m):
    for t in m._keep:
        t.release()
    m.release()


@pytest.mark.parametrize("name,Ts,mfma", [
    ("lfm2", (64, 9), 0),      # LFM2-8B-A1B shape, fp32 token path
    ("lfm2", (96, 70), 64),    # fp16 MFMA path for both calls
    ("lfm2", (1, 1), 0),       # batch-1 decode (needs no scratch)
    ("small", (200, 3), 0),    # H=256, F=192, E=8, K=2
])
def test_noalloc_matches_forward_dev(name, Ts, mfma):
    import torch
    ctx = gpu_context()
    ctx.set_mfma_min_tokens(mfma)
    L = full_layer(7) if name == "lfm2" else synth.moe_layer(41, H=256, F=192, E=8, K=2)
    H, E, K = L["H"], L["E"], L["K"]
    m = upload_layer(ctx, L)
    try:
        for T in Ts:
            _say("noalloc", name, "T=%d mfma_min_tokens=%d" % (T, mfma))
            x, h0 = synth.activations(1000 + T, T, H)
            dx = _dev(torch, x)
            dh = [_dev(torch, h0), _dev(torch, h0)]
            idx = torch.zeros((2, T, K), dtype=torch.int32, device="cuda")
            w = torch.zeros((2, T, K), dtype=torch.float64, device="cuda")
            torch.cuda.synchronize()
            m.forward_dev(dx.data_ptr(), dh[0].data_ptr(), T, idx_ptr=idx[0].data_ptr(), w_ptr=w[0].data_ptr())
            m.forward_noalloc_dev(dx.data_ptr(), dh[1].data_ptr(), T, idx_ptr=idx[1].data_ptr(),
                                  w_ptr=w[1].data_ptr())
            ctx.synchronize()
            out = [d.cpu().numpy() for d in dh]
            ii, ww = idx.cpu().numpy(), w.cpu().numpy()
            np.testing.assert_array_equal(ii[1], ii[0])
            np.testing.assert_array_equal(ww[1], ww[0])
            err = rel_l2(moe_delta(out[1], h0), moe_delta(out[0], h0))
            _say("  noalloc vs forward_dev rel_l2", err, "bit-equal", bool((out[1] == out[0]).all()))
            assert err < 1e-6, err
            r_out, r_idx, r_w, _ = oracle.moe_ffn(L, x[T - 1:], h0[T - 1:])
            np.testing.assert_array_equal(ii[1][T - 1:], r_idx)
            np.testing.assert_array_equal(ww[1][T - 1:], r_w)
            e_or = rel_l2(moe_delta(out[1][T - 1:], h0[T - 1:]), moe_delta(r_out, h0[T - 1:]))
            _say("  last row vs oracle rel_l2", e_or)
            assert e_or < (1e-2 if mfma and T >= mfma else 1e-4), e_or
    finally:
        ctx.set_mfma_min_tokens(512)
        _release(m)


def test_noalloc_rejects_oversize():
    import torch
    ctx = gpu_context()
    ctx.set_mfma_min_tokens(0)
    L = full_layer(7)
    m = upload_layer(ctx, L)
    try:
        T = 4096   # ~250 MB of scratch at this shape, over the 32 MiB array
        dx = torch.zeros((T, L["H"]), dtype=torch.float32, device="cuda")
        dh = torch.zeros_like(dx)
        torch.cuda.synchronize()
        with pytest.raises(qq_hip.QQError, match="fixed array"):
            m.forward_noalloc_dev(dx.data_ptr(), dh.data_ptr(), T)
        # the context still works afterwards
        m.forward_noalloc_dev(dx[:4].data_ptr(), dh[:4].data_ptr(), 4)
        ctx.synchronize()
        assert not torch.isnan(dh[:4]).any()
    finally:
        ctx.set_mfma_min_tokens(512)
        _release(m)
