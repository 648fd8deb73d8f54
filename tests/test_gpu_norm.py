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
