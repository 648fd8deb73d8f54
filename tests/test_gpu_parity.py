"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Tolerances: top-K indices, sigmoid probabilities and normalised weights
bit-exact on every path; the MoE contribution within 1e-4 relative L2 of the
oracle's on the fp32 paths and within 1e-2 on the fp16 MFMA path (prefill
chunks of at least qq_set_mfma_min_tokens rows).
"""
import contextlib
import sys

import numpy as np
import pytest

import oracle
import synth
from _util import dense_moe_f64, full_layer, gpu_context, moe_delta, rel_l2, upload_layer

pytestmark = pytest.mark.gpu

TOL_GEMV = 1e-4
TOL_MFMA = 1e-2


@contextlib.contextmanager
def mfma_min_tokens(n):
    """Route token batches of >= n rows to the MFMA path for the block's duration."""
    ctx = gpu_context()
    ctx.set_mfma_min_tokens(n)
    try:
        yield
    finally:
        ctx.set_mfma_min_tokens(512)


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# ---------------------------------------------------------------- Q8_0 matvec

@pytest.mark.parametrize("in_dim,out_dim,rows", [
    (1024, 3072, 1),     # Qwen3-0.6B FFN up-proj (qwen3-engine.js:205)
    (1024, 3072, 3),
    (2048, 1792, 1),     # expert gate/up shape
    (1792, 2048, 2),     # expert down shape
    (1000, 77, 1),       # in_dim not a multiple of 32: partial last block
    (2080, 130, 2),      # three 1 KiB chunks
    (5000, 40, 1),       # long-row kernel
    (32, 1, 1),          # single block, single column
    (7168, 2048, 1),     # LFM2 dense ffn_down: 224 block columns, two rounds of loads
    (500, 33, 1),        # 16 block columns, partial last block
    (12800, 48, 1),      # 400 block columns: more activations than the one-vector kernel stages
])
def test_q8_0_matvec(in_dim, out_dim, rows):
    _say("matvec", in_dim, out_dim, rows)
    ctx = gpu_context()
    rng = np.random.default_rng(in_dim * 7 + out_dim)
    w = synth.q8_0_tensor(rng, in_dim, out_dim)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    t = ctx.upload_q8_0(w, in_dim, out_dim)
    try:
        y = t.matvec(x)
    finally:
        t.release()
    for r in range(rows):
        ref = oracle.matmul_q8_0(w, in_dim, out_dim, x[r])
        assert rel_l2(y[r], ref) < TOL_GEMV, (r, rel_l2(y[r], ref))


def test_q8_0_matvec_expert_slices():
    """Matrix `mat` of a 3-D tensor is expert `mat` (_expertSlice, lfm2-engine.js:489-505)."""
    ctx = gpu_context()
    rng = np.random.default_rng(5)
    H, F, E = 256, 96, 5
    w = synth.q8_0_tensor(rng, H, F, E)
    x = rng.standard_normal(H).astype(np.float32)
    t = ctx.upload_q8_0(w, H, F, E)
    try:
        for e in range(E):
            off = e * F * (H // 32) * 34
            ref = oracle.matmul_q8_0(w, H, F, x, offset=off)
            assert rel_l2(t.matvec(x, mat=e)[0], ref) < TOL_GEMV
    finally:
        t.release()


def test_q8_0_special_values():
    """Zero scales give exact zeros; a one-hot weight returns x[i]*q*d."""
    ctx = gpu_context()
    in_dim, out_dim = 64, 4
    blocks = np.zeros(out_dim * 2, synth.Q8_DTYPE)
    blocks["d"] = np.float16(0.0)
    blocks["d"][2] = np.float16(0.5)          # column 1, block 0
    blocks["qs"][2, 7] = -3                   # element 7
    w = blocks.view(np.uint8)
    x = np.arange(in_dim, dtype=np.float32) - 10.0
    t = ctx.upload_q8_0(w, in_dim, out_dim)
    try:
        y = t.matvec(x)[0]
    finally:
        t.release()
    assert y[0] == 0.0 and y[2] == 0.0 and y[3] == 0.0
    assert y[1] == np.float32(x[7] * -3 * 0.5)


# ---------------------------------------------------------------- MoE layer

def _check_moe(L, x, hid, mask=None, tol=TOL_GEMV, rows=None):
    ctx = gpu_context()
    m = upload_layer(ctx, L)
    try:
        out, idx, w, probs = m.forward(x, hid, mask=mask)
    finally:
        for t in m._keep:
            t.release()
        m.release()
    sel = np.arange(x.shape[0]) if rows is None else np.asarray(rows)
    r_out, r_idx, r_w, r_probs = oracle.moe_ffn(L, x[sel], hid[sel], mask=mask)
    np.testing.assert_array_equal(idx[sel], r_idx)
    np.testing.assert_array_equal(probs[sel], r_probs)
    np.testing.assert_array_equal(w[sel], r_w)
    err = rel_l2(moe_delta(out[sel], hid[sel]), moe_delta(r_out, hid[sel]))
    _say("moe rel_l2", err)
    assert err < tol, err
    return out, idx, w, probs


@pytest.mark.parametrize("case", [
    dict(H=64, F=64, E=8, K=2, T=1),
    dict(H=100, F=50, E=5, K=5, T=1),        # ragged dims on the batch-1 path
    dict(H=2048, F=1792, E=64, K=8, T=1),    # 64 experts, 8 used
    dict(H=4096, F=96, E=16, K=2, T=1),      # widest hidden size
    dict(H=64, F=64, E=8, K=2, T=5),
    dict(H=96, F=160, E=6, K=3, T=4),
    dict(H=2048, F=64, E=32, K=4, T=3),
    dict(H=64, F=1792, E=32, K=4, T=2),
    dict(H=100, F=50, E=5, K=5, T=3),        # K == E, ragged dims
    dict(H=128, F=96, E=4, K=2, T=100),      # 32-slot tiles, several per expert
    dict(H=256, F=320, E=8, K=3, T=200),
])
def test_moe_small(case):
    _say("moe small", case)
    T = case.pop("T")
    L = synth.moe_layer(11, **case)
    x, hid = synth.activations(12, T, case["H"])
    _check_moe(L, x, hid)


@pytest.mark.parametrize("case", [
    dict(H=512, F=96, E=65, K=3),            # two experts a lane, the second lane ragged
    dict(H=2048, F=768, E=128, K=8),         # two experts a lane, all full
    dict(H=256, F=64, E=200, K=6),           # four experts a lane, ragged
    dict(H=256, F=64, E=256, K=8),           # the largest expert count
])
def test_moe_decode_many_experts(case):
    """Batch-1 decode (sigmoid + bias gating) with more experts than lanes in a wave."""
    _say("moe decode many experts", case)
    L = synth.moe_layer(13, **case)
    x, hid = synth.activations(14, 1, case["H"])
    _check_moe(L, x, hid)


def test_moe_decode_q8_router_many_experts():
    """Batch-1 decode with a Q8_0 router and 128 experts (the scalar router loop)."""
    L = synth.moe_layer(15, H=256, F=64, E=128, K=8, router_type=synth.TYPE_Q8_0)
    x, hid = synth.activations(16, 1, 256)
    _check_moe(L, x, hid)


def test_moe_no_bias_and_q8_router():
    L = synth.moe_layer(21, H=128, F=64, E=16, K=4, bias=None, router_type=synth.TYPE_Q8_0)
    x, hid = synth.activations(22, 7, 128)
    _check_moe(L, x, hid)


def test_moe_mask():
    """expertMask skips experts without renormalising (lfm2-engine.js:464)."""
    L = synth.moe_layer(31, H=128, F=96, E=8, K=3)
    x, hid = synth.activations(32, 6, 128)
    r_idx, _, _ = oracle.moe_route(L, x)
    masked = {int(r_idx[0, 0]), int(r_idx[1, 1])}
    _check_moe(L, x, hid, mask=masked)
    # masking every expert leaves hidden untouched
    out, _, _, _ = _check_moe(L, x, hid, mask=set(range(8)))
    np.testing.assert_array_equal(out, hid)


@pytest.mark.parametrize("E,tied,T", [(8, [1, 4, 6], 3), (8, [1, 4, 6], 1), (100, [5, 70, 71], 1)])
def test_moe_ties_lower_index(E, tied, T):
    """Equal selection scores rank the lower expert first (stable sort)."""
    L = synth.moe_layer(41, H=64, F=64, E=E, K=3)
    router = np.zeros((E, 64), np.float32)
    router[tied] = 0.01
    L["router"] = router.view(np.uint8).ravel()
    L["bias"] = np.zeros(E, np.float32)
    x, hid = synth.activations(42, T, 64)
    x[:] = np.abs(x)
    _, idx, _, _ = _check_moe(L, x, hid)
    assert (idx == tied).all()


def test_moe_decode_batch1_full():
    """One LFM2-8B-A1B MoE layer at batch-1 decode (H=2048, F=1792, E=32, K=4),
    several calls in a row on one layer handle (the router flags are reused)."""
    L = full_layer(1)
    x, hid = synth.activations(101, 6, 2048)
    ctx = gpu_context()
    m = upload_layer(ctx, L)
    try:
        for t in range(6):
            mask = {int(oracle.moe_route(L, x[t:t + 1])[0][0, 1])} if t == 5 else None
            out, idx, w, probs = m.forward(x[t:t + 1], hid[t:t + 1], mask=mask)
            r_out, r_idx, r_w, r_probs = oracle.moe_ffn(L, x[t:t + 1], hid[t:t + 1], mask=mask)
            np.testing.assert_array_equal(idx, r_idx)
            np.testing.assert_array_equal(w, r_w)
            np.testing.assert_array_equal(probs, r_probs)
            err = rel_l2(moe_delta(out, hid[t:t + 1]), moe_delta(r_out, hid[t:t + 1]))
            _say("decode token", t, "rel_l2", err)
            assert err < TOL_GEMV
        ctx.synchronize()
    finally:
        for t in m._keep:
            t.release()
        m.release()


def test_moe_decode_batch64_full():
    """64-token decode batch, ~uniform routing: every token against the oracle."""
    L = full_layer(1)
    x, hid = synth.activations(202, 64, 2048)
    _, idx, _, _ = _check_moe(L, x, hid)
    assert len(np.unique(idx)) >= 28


@pytest.mark.parametrize("path", ["mfma", "fp32"])
def test_moe_prefill_2048_skewed(path):
    """2048-token chunk with Zipf-skewed routing: all top-K bit-exact; sampled rows against
    the oracle and every row against the float64 dense restatement (MFMA path at 1e-2,
    fp32 path at 1e-4), so cold experts (< 10 rows) and the partial last fragments of hot
    groups are all compared."""
    _say("prefill 2048", path)
    L = full_layer(2, bias="zipf")
    x, hid = synth.activations(303, 2048, 2048)
    rows = np.random.default_rng(0).choice(2048, 24, replace=False)
    tol = TOL_MFMA if path == "mfma" else TOL_GEMV
    with mfma_min_tokens(512 if path == "mfma" else 0):
        out, idx, w, probs = _check_moe(L, x, hid, rows=rows, tol=tol)
    r_idx, r_w, r_probs = oracle.moe_route(L, x)
    np.testing.assert_array_equal(idx, r_idx)
    np.testing.assert_array_equal(w, r_w)
    np.testing.assert_array_equal(probs, r_probs)
    counts = np.bincount(idx.ravel(), minlength=32)
    assert counts.max() >= 300 and counts.min() < 10, counts
    dense = dense_moe_f64(L, x, hid, r_idx, r_w)
    err = rel_l2(moe_delta(out, hid), dense - hid)
    per_row = [rel_l2(moe_delta(out[t], hid[t]), dense[t] - hid[t]) for t in range(2048)]
    _say("all rows rel_l2", err, "worst row", int(np.argmax(per_row)), max(per_row))
    assert err < tol, err
    assert max(per_row) < 2 * tol
    # the coldest expert's rows on their own
    cold = int(np.argmin(np.where(counts > 0, counts, 1 << 30)))
    ct = np.nonzero((idx == cold).any(axis=1))[0]
    assert rel_l2(moe_delta(out[ct], hid[ct]), dense[ct] - hid[ct]) < tol


@pytest.mark.parametrize("case", [
    dict(H=64, F=64, E=8, K=2, T=40),
    dict(H=256, F=96, E=4, K=2, T=300),      # several row tiles per expert, ragged column tile
    dict(H=128, F=160, E=16, K=4, T=33),     # many groups smaller than one fragment
    dict(H=2048, F=1792, E=64, K=8, T=64),
    dict(H=4096, F=96, E=16, K=2, T=20),
])
def test_moe_mfma_small(case):
    """The MFMA GEMMs on small shapes (threshold lowered to 2 rows), every row checked."""
    _say("moe mfma", case)
    T = case.pop("T")
    L = synth.moe_layer(51, **case)
    x, hid = synth.activations(52, T, case["H"])
    with mfma_min_tokens(2):
        _check_moe(L, x, hid, tol=TOL_MFMA)


def test_moe_mfma_mask_and_unsupported_shape():
    """Mask on the MFMA path; a hidden size that is not a multiple of 32 stays on the
    fp32 path (1e-4) even when the threshold asks for MFMA."""
    L = synth.moe_layer(61, H=128, F=96, E=8, K=3)
    x, hid = synth.activations(62, 24, 128)
    r_idx, _, _ = oracle.moe_route(L, x)
    with mfma_min_tokens(2):
        _check_moe(L, x, hid, mask={int(r_idx[0, 0]), int(r_idx[3, 2])}, tol=TOL_MFMA)
        L2 = synth.moe_layer(63, H=100, F=64, E=8, K=2)
        x2, hid2 = synth.activations(64, 24, 100)
        _check_moe(L2, x2, hid2, tol=TOL_GEMV)


@pytest.mark.parametrize("case", [
    dict(T=37, mask=2),                                              # ragged token tiles, masked experts
    dict(T=256),                                                     # T K = 1024 pairs, the largest batch
    dict(H=512, F=96, E=65, K=3, T=20),                              # two experts a lane, ragged
    dict(H=1024, F=64, E=16, K=2, T=16, bias=None),
    dict(H=2048, F=768, E=128, K=8, T=128, gating="softmax"),        # 256 workgroups
    dict(H=2048, F=768, E=128, K=8, T=64, gating="softmax", mask=3),
])
def test_moe_batch_one_launch_routing(case):
    """Small batches whose router, top-K and dispatch run as one launch
    (workgroups exchange partial logits and expert ids as tagged words):
    routing bit-exact, the layer within the batch tolerance."""
    _say("moe one-launch routing", case)
    case = dict(case)
    T = case.pop("T")
    nmask = case.pop("mask", 0)
    if "H" in case:
        kw = dict(case)
        if kw.get("gating") == "softmax":
            kw.update(bias=None, router_std=0.05)
        L = synth.moe_layer(91, **kw)
    else:
        L = full_layer(2)
    x, hid = synth.activations(92, T, L["H"])
    mask = None
    if nmask:
        r_idx, _, _ = oracle.moe_route(L, x)
        mask = {int(e) for e in r_idx[:nmask, 0]}
    _check_moe(L, x, hid, mask=mask)


@pytest.mark.parametrize("shape,T,hot,tiles", [
    ("lfm2", 64, -1, 33),    # one expert at 18 rows: 16 items past 512 (8 gate/up, 7 down segments)
    ("lfm2", 64, 1, 35),     # 48 items past: 5 segments each
    ("lfm2", 64, 2, 37),     # 80 past: 3 segments
    ("lfm2", 112, 0, 38),    # 96 past: 2 segments
    ("lfm2", 128, 0, 45),    # 208 past: a second round of whole items
    ("lfm2", 200, 0, None),  # 32-row tiles (gate/up items of 64 features)
    ("lfm2", 256, 2, None),
    ("qwen3", 19, 0, 89),    # 16-row tiles, 64-feature gate/up items: 48 past, 5 segments
    ("qwen3", 23, 0, 101),   # down rows of 24 blocks: 80 past, 3 segments
])
def test_moe_batch_remainder_items(shape, T, hot, tiles):
    """Decode batches whose items (row tiles x column groups) overflow the 512
    resident workgroups of a 256-CU MI355X by a remainder: the remainder items
    are split along the reduction dimension, each segment's fp32 partial sums
    added in segment order by the segment that finishes last.  Every row
    within the batch tolerance; a second input in between and the first input
    again bit for bit (the segment counters return to zero after each launch).
    hot: experts 0 .. hot-1 get bias +1 (picked by every token); -1: expert 5
    gets +0.1 (18 of the 64 tokens).  qwen3: the Qwen3-30B-A3B-shaped layer
    (E=128, K=8, F=768, softmax gating)."""
    _say("moe remainder items", shape, T, hot, tiles)
    if shape == "qwen3":
        L = synth.moe_layer(91, H=2048, F=768, E=128, K=8, bias=None, gating="softmax", router_std=0.05)
        x, hid = synth.activations(92, T, 2048)
    else:
        L = dict(full_layer(1))
        L["bias"] = L["bias"].copy()
        if hot > 0:
            L["bias"][:hot] += 1.0
        elif hot < 0:
            L["bias"][5] += 0.1
        x, hid = synth.activations(202, T, 2048)
    x2, hid2 = synth.activations(203, T, 2048)
    r_idx, _, _ = oracle.moe_route(L, x)
    E, K = L["E"], L["K"]
    bm = 16 if T * K <= 16 * E else 32
    c = np.bincount(r_idx.ravel(), minlength=E)
    if tiles is not None:
        assert int(np.sum((c + bm - 1) // bm)) == tiles, c
    ctx = gpu_context()
    m = upload_layer(ctx, L)
    try:
        outs = [m.forward(xx, hh) for xx, hh in ((x, hid), (x2, hid2), (x, hid))]
    finally:
        for t in m._keep:
            t.release()
        m.release()
    for (out, idx, w, probs), xx, hh in zip(outs[:2], (x, x2), (hid, hid2)):
        r_out, r_idx, r_w, r_probs = oracle.moe_ffn(L, xx, hh)
        np.testing.assert_array_equal(idx, r_idx)
        np.testing.assert_array_equal(probs, r_probs)
        np.testing.assert_array_equal(w, r_w)
        err = rel_l2(moe_delta(out, hh), moe_delta(r_out, hh))
        _say("moe rel_l2", err)
        assert err < TOL_GEMV, err
    np.testing.assert_array_equal(outs[2][0], outs[0][0])


# ---------------------------------------------------------------- Qwen3-MoE softmax gating

@pytest.mark.parametrize("case", [
    dict(H=64, F=64, E=8, K=2, T=1),
    dict(H=100, F=50, E=5, K=5, T=1),        # K == E
    dict(H=96, F=160, E=6, K=3, T=4),
    dict(H=2048, F=768, E=128, K=8, T=1),    # Qwen3-30B-A3B decode (E = 128: two experts a lane)
    dict(H=2048, F=768, E=128, K=8, T=9),
    dict(H=512, F=96, E=65, K=3, T=1),       # second lane ragged
    dict(H=256, F=64, E=200, K=4, T=1),      # four experts a lane, ragged
    dict(H=256, F=64, E=256, K=8, T=1),      # the largest expert count
    dict(H=256, F=320, E=8, K=3, T=200),
])
def test_moe_softmax_gating(case):
    """Qwen3Engine._moEFFN (qwen3-engine.js:304-363): softmax probabilities, selection by
    probability, weights p / sum p; top-K, probabilities and weights bit-exact."""
    _say("moe softmax", case)
    T = case.pop("T")
    L = synth.moe_layer(71, bias=None, gating="softmax", router_std=0.05, **case)
    x, hid = synth.activations(72, T, case["H"])
    _check_moe(L, x, hid)


def test_moe_softmax_q8_router_mask_and_mfma():
    """Q8_0 router, expert mask, and the MFMA path under softmax gating."""
    L = synth.moe_layer(73, H=256, F=96, E=16, K=4, bias=None, gating="softmax",
                        router_type=synth.TYPE_Q8_0)
    x, hid = synth.activations(74, 40, 256)
    r_idx, _, _ = oracle.moe_route(L, x)
    _check_moe(L, x, hid, mask={int(r_idx[0, 0])})
    with mfma_min_tokens(2):
        _check_moe(L, x, hid, tol=TOL_MFMA)


def test_moe_softmax_decode_calls_in_a_row():
    """Qwen3-30B-A3B-shaped layer (H=2048, F=768, E=128, K=8) at batch-1 decode: several
    calls on one handle (each draws a fresh epoch), the last one with an expert mask."""
    L = synth.moe_layer(77, H=2048, F=768, E=128, K=8, bias=None, gating="softmax",
                        router_std=0.05)
    x, hid = synth.activations(78, 5, 2048)
    ctx = gpu_context()
    m = upload_layer(ctx, L)
    try:
        for t in range(5):
            mask = {int(oracle.moe_route(L, x[t:t + 1])[0][0, 2])} if t == 4 else None
            out, idx, w, probs = m.forward(x[t:t + 1], hid[t:t + 1], mask=mask)
            r_out, r_idx, r_w, r_probs = oracle.moe_ffn(L, x[t:t + 1], hid[t:t + 1], mask=mask)
            np.testing.assert_array_equal(idx, r_idx)
            np.testing.assert_array_equal(w, r_w)
            np.testing.assert_array_equal(probs, r_probs)
            err = rel_l2(moe_delta(out, hid[t:t + 1]), moe_delta(r_out, hid[t:t + 1]))
            _say("softmax decode token", t, "rel_l2", err)
            assert err < TOL_GEMV
    finally:
        for t in m._keep:
            t.release()
        m.release()


def test_moe_softmax_decode_q8_router_and_ties():
    """Batch-1 softmax decode with a Q8_0 router, and equal probabilities ranked by index."""
    L = synth.moe_layer(79, H=256, F=64, E=128, K=8, bias=None, gating="softmax",
                        router_type=synth.TYPE_Q8_0)
    x, hid = synth.activations(80, 1, 256)
    _check_moe(L, x, hid)
    E, tied = 96, [3, 5, 70, 71]
    L = synth.moe_layer(81, H=64, F=64, E=E, K=4, bias=None, gating="softmax")
    router = np.zeros((E, 64), np.float32)
    router[tied + [90]] = 0.01
    L["router"] = router.view(np.uint8).ravel()
    x, hid = synth.activations(82, 1, 64)
    x[:] = np.abs(x)
    _, idx, _, _ = _check_moe(L, x, hid)
    assert (idx == tied).all()


@pytest.mark.parametrize("T", [1, 5])
def test_moe_softmax_wide_logits(T):
    """Router logits tens apart: exponentials below 2^-22 take the in-order sum, and a
    dominant logit underflows the others to zero (probability 1, weight 1)."""
    _say("moe softmax wide logits", T)
    L = synth.moe_layer(83, H=256, F=64, E=128, K=8, bias=None, gating="softmax",
                        router_std=1.0)
    x, hid = synth.activations(84, T, 256)
    _check_moe(L, x, hid)
    E = 96
    L = synth.moe_layer(85, H=64, F=64, E=E, K=2, bias=None, gating="softmax")
    router = np.zeros((E, 64), np.float32)
    router[77, 0] = 200.0
    L["router"] = router.view(np.uint8).ravel()
    x, hid = synth.activations(86, T, 64)
    x[:, 0] = 1.0
    _, idx, w, probs = _check_moe(L, x, hid)
    assert (idx[:, 0] == 77).all() and (w[:, 0] == 1.0).all() and (probs[:, 77] == 1.0).all()


def test_moe_softmax_set_gating_rejects_unknown():
    ctx = gpu_context()
    L = synth.moe_layer(75, H=64, F=64, E=8, K=2, bias=None)
    m = upload_layer(ctx, L)
    try:
        with pytest.raises(RuntimeError, match="gating"):
            m.set_gating(7)
    finally:
        for t in m._keep:
            t.release()
        m.release()
