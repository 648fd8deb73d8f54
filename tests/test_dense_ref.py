"""The float64 dense restatement of the expert products (tests/_util.py
dense_moe_f64), used to check every row of the large GPU cases, against the
C oracle: within 1e-6 relative L2 of the MoE contribution (they differ only by
the reference's fp32 roundings), with a mask; a planted transposition of the
down matrix and a dropped SiLU are far outside it."""
import numpy as np

import oracle
import synth
from _util import dense_moe_f64, moe_delta, rel_l2


def test_dense_matches_oracle():
    L = synth.moe_layer(3, H=256, F=192, E=8, K=3)
    x, hid = synth.activations(4, 6, 256)
    for mask in (None, {1, 5}):
        r_out, r_idx, r_w, _ = oracle.moe_ffn(L, x, hid, mask=mask)
        d = dense_moe_f64(L, x, hid, r_idx, r_w, mask=mask)
        assert rel_l2(d - hid, moe_delta(r_out, hid)) < 1e-6


def test_dense_planted_mistakes_fail():
    L = synth.moe_layer(5, H=128, F=128, E=4, K=2)
    x, hid = synth.activations(6, 4, 128)
    r_out, r_idx, r_w, _ = oracle.moe_ffn(L, x, hid)
    ref = moe_delta(r_out, hid)
    # down matrix transposed (square shapes make it type-check)
    nb = 128 // 32
    bl = np.frombuffer(L["down"].tobytes(), synth.Q8_DTYPE).reshape(4, 128, nb)
    dq = bl["qs"].reshape(4, 128, 128).transpose(0, 2, 1).reshape(4, 128, nb, 32)
    dd = bl["d"]
    bad = np.empty_like(bl)
    bad["qs"] = dq
    bad["d"] = dd
    L2 = dict(L, down=bad.view(np.uint8).ravel())
    assert rel_l2(dense_moe_f64(L2, x, hid, r_idx, r_w) - hid, ref) > 1e-2
    # the routing weights dropped (every expert weighted 1)
    assert rel_l2(dense_moe_f64(L, x, hid, r_idx, np.ones_like(r_w)) - hid, ref) > 1e-2
