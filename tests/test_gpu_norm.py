"""GPU rmsnorm (qq_rmsnorm_dev) against the oracle's restatement of
src/tensor.js:103-114 (unit weight) and, for a weighted norm, against the
unit-weight oracle output scaled by the weight in binary64.

The GPU's sum of squares is a binary64 tree, the reference's a sequential
binary64 loop; both round an exact-product sum, so outputs agree to within
one fp32 ulp (a straddle of a rounding boundary) and almost always exactly.
"""
import numpy as np
import pytest

import oracle
from _util import gpu_context

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,H", [(1, 2048), (3, 2048), (5, 100), (2, 4096)])
def test_rmsnorm_matches_oracle(T, H):
    import torch
    print("rmsnorm", T, H, flush=True)
    rng = np.random.default_rng(T * 1000 + H)
    x = (rng.standard_normal((T, H)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, H).astype(np.float32)
    ctx = gpu_context()
    dx = torch.from_numpy(x).cuda()
    dw = torch.from_numpy(w).cuda()
    out_u = torch.empty_like(dx)
    out_w = torch.empty_like(dx)
    torch.cuda.synchronize()
    ctx.rmsnorm_dev(dx.data_ptr(), None, out_u.data_ptr(), T, H, 1e-5)
    ctx.rmsnorm_dev(dx.data_ptr(), dw.data_ptr(), out_w.data_ptr(), T, H, 1e-5)
    ctx.synchronize()
    gu, gw = out_u.cpu().numpy(), out_w.cpu().numpy()
    ref = np.stack([oracle.rmsnorm_unit(x[t], 1e-5) for t in range(T)])
    ulp = np.abs(gu.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1, ulp.max()
    assert (ulp == 0).mean() > 0.99
    refw = (ref.astype(np.float64) * w.astype(np.float64))
    assert np.max(np.abs(gw - refw) / np.maximum(np.abs(refw), 1e-30)) < 3e-7


@pytest.mark.parametrize("T,mfma,weighted,gating,H", [(1, 0, False, "sigmoid", 512),
                                                      (1, 0, True, "sigmoid", 512),
                                                      (64, 0, True, "sigmoid", 512),
                                                      (96, 64, False, "sigmoid", 512),
                                                      (1, 0, True, "softmax", 512),
                                                      # MFMA chunks: the router forms the norm
                                                      (97, 64, True, "sigmoid", 800),
                                                      (600, 64, True, "sigmoid", 2048),
                                                      (600, 64, False, "softmax", 512),
                                                      # a 4096-token MFMA chunk, then a 4-token
                                                      # stream chunk normalised by its own launch
                                                      (4100, 64, True, "sigmoid", 512),
                                                      # MFMA chunks normalised by their own launch:
                                                      # a Q8_0 router, norm weights 4 bytes off a
                                                      # 16-byte boundary
                                                      (600, 64, True, "q8router", 512),
                                                      (600, 64, True, "offset_w", 512)])
def test_fused_norm_moe_matches_two_calls(T, mfma, weighted, gating, H):
    """qq_moe_forward_norm_dev == qq_rmsnorm_dev then qq_moe_forward_dev, bit for bit
    (a single row is normalised inside the decode kernel, the rows of an MFMA
    chunk inside its router launch)."""
    import torch
    import synth
    from _util import upload_layer
    print("fused norm+moe", T, mfma, weighted, gating, H, flush=True)
    ctx = gpu_context()
    ctx.set_mfma_min_tokens(mfma)
    if gating == "softmax":
        L = synth.moe_layer(41, H=H, F=256, E=128, K=4, bias=None, gating="softmax")
    elif gating == "q8router":
        L = synth.moe_layer(41, H=H, F=256, E=16, K=4, router_type=synth.TYPE_Q8_0)
    else:
        L = synth.moe_layer(41, H=H, F=256, E=16, K=4)
    m = upload_layer(ctx, L)
    try:
        rng = np.random.default_rng(T + 7)
        h0 = (rng.standard_normal((T, H)) * 2).astype(np.float32)
        w = rng.uniform(0.5, 1.5, H).astype(np.float32) if weighted else None
        dh0 = torch.from_numpy(h0).cuda()
        if gating == "offset_w":
            dwb = torch.zeros(H + 1, dtype=torch.float32, device="cuda")
            dwb[1:] = torch.from_numpy(w).cuda()
            dw = dwb[1:]
        else:
            dw = torch.from_numpy(w).cuda() if weighted else None
        wp = dw.data_ptr() if weighted else None
        idx_a = torch.empty((T, 4), dtype=torch.int32, device="cuda")
        idx_b = torch.empty_like(idx_a)
        ha, hb = dh0.clone(), dh0.clone()
        xn = torch.empty_like(dh0)
        torch.cuda.synchronize()
        m.forward_norm_dev(ha.data_ptr(), T, norm_w_ptr=wp, eps=1e-5, idx_ptr=idx_a.data_ptr())
        ctx.rmsnorm_dev(hb.data_ptr(), wp, xn.data_ptr(), T, H, 1e-5)
        m.forward_dev(xn.data_ptr(), hb.data_ptr(), T, idx_ptr=idx_b.data_ptr())
        ctx.synchronize()
        assert np.array_equal(idx_a.cpu().numpy(), idx_b.cpu().numpy())
        assert np.array_equal(ha.cpu().numpy(), hb.cpu().numpy())
    finally:
        ctx.set_mfma_min_tokens(512)
        m.release()


def test_fused_norm_moe_decode_against_oracle():
    """One token through ffn_norm (unit weight) + the MoE block at the LFM2-8B-A1B shape."""
    import torch
    import synth
    from _util import full_layer, upload_layer, rel_l2, moe_delta
    print("fused norm+moe oracle", flush=True)
    ctx = gpu_context()
    L = full_layer(7)
    m = upload_layer(ctx, L)
    try:
        _, h0 = synth.activations(17, 1, 2048)
        x = oracle.rmsnorm_unit(h0[0], 1e-5)[None, :]
        ref_h, ref_idx, ref_w, _ = oracle.moe_ffn(L, x, h0)
        dh = torch.from_numpy(h0).cuda()
        idx = torch.empty((1, 4), dtype=torch.int32, device="cuda")
        wts = torch.empty((1, 4), dtype=torch.float64, device="cuda")
        torch.cuda.synchronize()
        m.forward_norm_dev(dh.data_ptr(), 1, eps=1e-5, idx_ptr=idx.data_ptr(), w_ptr=wts.data_ptr())
        ctx.synchronize()
        assert np.array_equal(idx.cpu().numpy(), ref_idx)
        assert np.array_equal(wts.cpu().numpy(), ref_w)
        got = dh.cpu().numpy()
        assert rel_l2(moe_delta(got, h0), moe_delta(ref_h, h0)) < 1e-4
    finally:
        m.release()
