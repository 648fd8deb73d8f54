"""The WebGPU engines' device-resident MoE block through the C ABI:
qq_moe_forward_record_dev (Lfm2GPUEngine._moEFFNGPU / Qwen3GPUEngine._moEFFNGPU,
src/webgpu.js:1882-1917, :878-915) and the device buffers standing for
GPUDevice.createBuffer / writeBuffer / readF32 (src/webgpu.js:369-430).

The routing record (src/webgpu.js:1236-1240) holds, per row, the K selected
experts, their weights and the E probabilities as floats.  Its values are the
CPU engine's routing (the oracle): selected experts equal, weights equal to the
oracle's binary64 w rounded to fp32, probabilities equal bit for bit.  The
hidden update is the one qq_moe_forward_dev makes, bit for bit (same kernels)."""
import numpy as np
import pytest

import oracle
from _util import gpu_context, rel_l2, moe_delta, full_layer, upload_layer

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _record(L, idx, w, probs):
    K, E = L["K"], L["E"]
    T = idx.shape[0]
    rec = np.zeros((T, 2 * K + E), np.float32)
    rec[:, :K] = idx
    rec[:, K:2 * K] = np.asarray(w, np.float64).astype(np.float32)
    rec[:, 2 * K:] = probs
    return rec


@pytest.mark.parametrize("T,gating,mask", [
    (1, "sigmoid", None),          # the decode kernel writes the record itself
    (1, "sigmoid", (2, 9)),
    (1, "softmax", None),
    (7, "sigmoid", None),          # router kernels, then the record kernel
    (7, "softmax", (0,)),
])
def test_record_matches_oracle(T, gating, mask):
    import torch
    import synth
    _say("record", T, gating, mask)
    ctx = gpu_context()
    if gating == "softmax":
        L = synth.moe_layer(41, bias=None, gating="softmax", router_std=0.05)
    else:
        L = full_layer(11)
    m = upload_layer(ctx, L)
    try:
        x, h0 = synth.activations(23 + T, T, L["H"])
        ref_h, ref_idx, ref_w, ref_p = oracle.moe_ffn(L, x, h0, mask=set(mask) if mask else None)
        dx = torch.from_numpy(x).cuda()
        dh = torch.from_numpy(h0).cuda()
        dh2 = torch.from_numpy(h0).cuda()
        rec = torch.full((T, 2 * L["K"] + L["E"]), -7.0, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        m.forward_record_dev(dx.data_ptr(), dh.data_ptr(), T, mask=mask, record_ptr=rec.data_ptr())
        m.forward_dev(dx.data_ptr(), dh2.data_ptr(), T, mask=mask)
        ctx.synchronize()
        want = _record(L, ref_idx, ref_w, ref_p)
        got = rec.cpu().numpy()
        np.testing.assert_array_equal(got, want)
        assert np.array_equal(dh.cpu().numpy(), dh2.cpu().numpy())
        assert rel_l2(moe_delta(dh.cpu().numpy(), h0), moe_delta(ref_h, h0)) < 1e-4
    finally:
        m.release()


def test_record_null_is_the_plain_forward():
    import torch
    import synth
    ctx = gpu_context()
    L = full_layer(11)
    m = upload_layer(ctx, L)
    try:
        x, h0 = synth.activations(5, 3, L["H"])
        dx = torch.from_numpy(x).cuda()
        da, db = torch.from_numpy(h0).cuda(), torch.from_numpy(h0).cuda()
        torch.cuda.synchronize()
        m.forward_record_dev(dx.data_ptr(), da.data_ptr(), 3)
        m.forward_dev(dx.data_ptr(), db.data_ptr(), 3)
        ctx.synchronize()
        assert np.array_equal(da.cpu().numpy(), db.cpu().numpy())
    finally:
        m.release()


def test_buffers_zeroed_write_read_free():
    ctx = gpu_context()
    n = 3 * 1000 + 4
    p = ctx.buffer_alloc(n * 4)
    try:
        z = ctx.buffer_read(p, np.full(n, 5.0, np.float32))
        assert not z.any()
        v = np.arange(n, dtype=np.float32) * 0.25 - 100.0
        ctx.buffer_write(p, v)
        assert np.array_equal(ctx.buffer_read(p, np.empty(n, np.float32)), v)
        # a byte range in the middle
        ctx.buffer_write(p + 400, np.array([1.5, -2.5], np.float32))
        got = ctx.buffer_read(p + 396, np.empty(4, np.float32))
        assert got.tolist() == [v[99], 1.5, -2.5, v[102]]
    finally:
        ctx.buffer_free(p)
