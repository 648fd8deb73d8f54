"""Pins of the CPU oracle (oracle/qq_oracle.c) to the mathematics of the
reference path, independent of the HIP code.

The reference ships no tests or golden vectors, so each oracle function is
checked against something that fixes it from outside: numpy's IEEE binary16,
exact rational arithmetic, closed forms, numpy's stable argsort, a float64
dense re-derivation, and invariants whose violation a plausible mistake
(transposed layout, dropped sign extension, wrong scale offset, rounding at
the wrong step) would cause.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
import synth


# ------------------------------------------------------------------ fp16

def test_f16_decode_exhaustive():
    """All 65,536 patterns against numpy's binary16 and the closed form."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float64)
    got = np.array([oracle.f16_to_f64(int(b)) for b in bits])
    nan = np.isnan(ref)
    assert (np.isnan(got) == nan).all()
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    # closed form on normals: (-1)^s 2^(e-15) (1 + m/1024)
    for b in (0x3c00, 0x0400, 0x7bff, 0xc000, 0x0001, 0x03ff, 0x8001):
        s, e, m = b >> 15, (b >> 10) & 31, b & 1023
        cf = (-1) ** s * (2.0 ** (e - 15) * (1 + m / 1024) if e else 2.0 ** -14 * (m / 1024))
        assert oracle.f16_to_f64(b) == cf


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.002),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e4),
        np.array([0.0, -0.0, 65504.0, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 1e-9, np.inf, -np.inf], np.float32),
    ])
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(got, ref)


# ------------------------------------------------------------------ Q8_0 matvec

def _terms(w, x, in_dim, out_dim):
    """Per-column lists of exact terms x_i * q_i * d_b in the reference's order."""
    nb = (in_dim + 31) // 32
    blocks = np.frombuffer(w.tobytes(), synth.Q8_DTYPE).reshape(out_dim, nb)
    cols = []
    for c in range(out_dim):
        t = []
        for b in range(nb):
            d = float(blocks["d"][c, b])
            for i in range(32):
                k = 32 * b + i
                if k < in_dim:
                    t.append((float(x[k]), int(blocks["qs"][c, b, i]), d))
        cols.append(t)
    return cols


def test_q8_0_matvec_exact_and_sequential():
    """y[c] = fp32(sequential float64 sum); the exact rational sum is within the
    sequential-sum error bound of it."""
    rng = np.random.default_rng(1)
    in_dim, out_dim = 96, 7
    w = synth.q8_0_tensor(rng, in_dim, out_dim)
    x = rng.standard_normal(in_dim).astype(np.float32)
    y = oracle.matmul_q8_0(w, in_dim, out_dim, x)
    for c, terms in enumerate(_terms(w, x, in_dim, out_dim)):
        prods = np.array([xv * q * d for xv, q, d in terms])            # exact in float64
        seq = np.cumsum(prods)[-1]                                      # sequential order
        assert y[c] == np.float32(seq)
        exact = sum(Fraction(xv) * q * Fraction(d) for xv, q, d in terms)
        bound = len(terms) * 2.0 ** -53 * float(np.abs(prods).sum())
        assert abs(float(exact) - seq) <= bound
        # every term is exact in binary64 (24 + 8 + 11 significant bits)
        for xv, q, d in terms[:5]:
            assert Fraction(xv * q * d) == Fraction(xv) * q * Fraction(d)


def test_q8_0_one_hot_layout():
    """A single nonzero weight lands where the column-major layout puts it,
    with int8 sign extension and the block's own fp16 scale at +0."""
    in_dim, out_dim = 64, 3
    blocks = np.zeros(out_dim * 2, synth.Q8_DTYPE)
    blocks["d"][:] = np.float16(1.0)
    blocks["d"][2 * 1 + 1] = np.float16(0.25)      # column 1, block 1
    blocks["qs"][2 * 1 + 1, 5] = -7                # element 32 + 5 of column 1
    w = blocks.view(np.uint8)
    x = np.arange(in_dim, dtype=np.float32) + 1.0
    y = oracle.matmul_q8_0(w, in_dim, out_dim, x)
    np.testing.assert_array_equal(y, np.array([0.0, x[37] * -7 * 0.25, 0.0], np.float32))
    # the same bytes read as if rows were k (a transposed layout) give another answer
    yt = oracle.matmul_q8_0(w[: 2 * 34], 32, 2, x[:32])
    assert not np.array_equal(yt, y[:2])


def test_q8_0_closed_forms():
    rng = np.random.default_rng(2)
    in_dim, out_dim = 128, 9
    w = synth.q8_0_tensor(rng, in_dim, out_dim)
    # zero scales -> exact zeros
    z = np.frombuffer(w.tobytes(), synth.Q8_DTYPE).copy()
    z["d"] = 0
    assert (oracle.matmul_q8_0(z.view(np.uint8), in_dim, out_dim, rng.standard_normal(in_dim)) == 0).all()
    # all-ones x -> column sums of the dequantised weights
    dense = synth.q8_0_dequant(w, in_dim, out_dim)[0]
    np.testing.assert_allclose(oracle.matmul_q8_0(w, in_dim, out_dim, np.ones(in_dim, np.float32)),
                               dense.sum(axis=1), rtol=1e-6)
    # scaling x by a power of two scales every term exactly
    x = rng.standard_normal(in_dim).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_q8_0(w, in_dim, out_dim, x * 8),
                                  oracle.matmul_q8_0(w, in_dim, out_dim, x) * 8)


def test_q8_0_partial_last_block():
    """in_dim not a multiple of 32: the tail of the last block is never read."""
    rng = np.random.default_rng(3)
    in_dim, out_dim = 70, 4
    w = synth.q8_0_tensor(rng, in_dim, out_dim)
    x = rng.standard_normal(in_dim).astype(np.float32)
    y = oracle.matmul_q8_0(w, in_dim, out_dim, x)
    # garbage in the unread tail changes nothing
    b = np.frombuffer(w.tobytes(), synth.Q8_DTYPE).copy().reshape(out_dim, 3)
    b["qs"][:, 2, in_dim - 64:] = 99
    np.testing.assert_array_equal(oracle.matmul_q8_0(b.view(np.uint8).ravel(), in_dim, out_dim, x), y)
    dense = synth.q8_0_dequant(w, in_dim, out_dim)[0]
    np.testing.assert_allclose(y, dense @ x.astype(np.float64), rtol=1e-6, atol=1e-7)


def test_f32_matvec_and_generic():
    rng = np.random.default_rng(4)
    in_dim, out_dim = 200, 6
    W = rng.standard_normal((out_dim, in_dim)).astype(np.float32)
    x = rng.standard_normal(in_dim).astype(np.float32)
    y = oracle.matmul_f32(W, in_dim, out_dim, x)
    for c in range(out_dim):
        prods = W[c].astype(np.float64) * x.astype(np.float64)
        assert y[c] == np.float32(np.cumsum(prods)[-1])
    np.testing.assert_array_equal(oracle.matmul_generic(0, W, in_dim, out_dim, x), y)
    with pytest.raises(ValueError, match="Unsupported tensor type"):
        oracle.matmul_generic(12, W, in_dim, out_dim, x)


def test_silu_rounding():
    """arr[i] *= 1/(1+exp(-arr[i])): binary64 math, one fp32 rounding."""
    v = np.array([0.0, -0.0, 1.0, -1.0, 3.5, -20.0, 20.0, 1e-8, -88.0, 0.693147], np.float32)
    got = oracle.silu(v)
    for a, g in zip(v, got):
        a = float(a)
        assert g == np.float32(a * (1.0 / (1.0 + math.exp(-a))))
    assert got[0] == 0.0
    pos = np.linspace(0, 30, 1000).astype(np.float32)
    sp = oracle.silu(pos)
    assert (np.diff(sp) >= 0).all() and (sp <= pos).all()


def test_rmsnorm_unit():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(2048).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
    np.testing.assert_allclose(oracle.rmsnorm_unit(x), ref, rtol=2e-7)


# ------------------------------------------------------------------ routing

def _small_layer(seed, **kw):
    kw.setdefault("H", 64)
    kw.setdefault("F", 64)
    kw.setdefault("E", 8)
    kw.setdefault("K", 2)
    return synth.moe_layer(seed, **kw)


def test_route_matches_stable_argsort():
    L = _small_layer(10, H=256, E=32, K=4)
    x, _ = synth.activations(11, 200, 256)
    idx, w, probs = oracle.moe_route(L, x)
    # selection scores recomputed from the oracle's probabilities
    sel = (probs + L["bias"][None, :]).astype(np.float32)
    ref = np.argsort(-sel.astype(np.float64), axis=1, kind="stable")[:, :4]
    np.testing.assert_array_equal(idx, ref)
    # every selected score >= every unselected one
    for t in range(len(x)):
        chosen = sel[t, idx[t]]
        rest = np.delete(sel[t], idx[t])
        assert chosen.min() >= rest.max()
    # sum of weights = S / (S + 1e-6), S the sum of selected probabilities
    S = np.take_along_axis(probs.astype(np.float64), idx, axis=1).sum(axis=1)
    np.testing.assert_allclose(w.sum(axis=1), S / (S + 1e-6), rtol=1e-12)
    # probabilities are sigmoid of the F32 router logits
    W = L["router"].view(np.float32).reshape(32, 256).astype(np.float64)
    logits = (x.astype(np.float64) @ W.T).astype(np.float32)
    np.testing.assert_allclose(probs, 1 / (1 + np.exp(-logits.astype(np.float64))), rtol=1e-6)


def test_route_ties_go_to_lower_index():
    L = _small_layer(12, E=8, K=3)
    router = np.zeros((8, 64), np.float32)
    router[[6, 2, 4]] = 0.5
    L["router"] = router.view(np.uint8).ravel()
    L["bias"] = np.zeros(8, np.float32)
    x = np.abs(synth.activations(13, 4, 64)[0])
    idx, _, _ = oracle.moe_route(L, x)
    assert (idx == [2, 4, 6]).all()
    # a bias that breaks the tie in favour of the higher index wins
    L["bias"][6] = 1e-3
    idx, _, _ = oracle.moe_route(L, x)
    assert (idx == [6, 2, 4]).all()


def test_route_q8_router_and_no_bias():
    L = _small_layer(14, H=128, E=16, K=4, bias=None, router_type=synth.TYPE_Q8_0)
    x, _ = synth.activations(15, 30, 128)
    idx, w, probs = oracle.moe_route(L, x)
    dense = synth.q8_0_dequant(L["router"], 128, 16)[0]
    logits = (x.astype(np.float64) @ dense.T).astype(np.float32)
    p = (1 / (1 + np.exp(-logits.astype(np.float64)))).astype(np.float32)
    np.testing.assert_array_equal(idx, np.argsort(-p.astype(np.float64), axis=1, kind="stable")[:, :4])


# ------------------------------------------------------- softmax gating (Qwen3)

def _onehot_logit_layer(logits, K):
    """A softmax-gated layer whose router logits for x = e_0 are exactly
    `logits` (one product per logit: x_0 * W[e][0] = 1 * logit)."""
    E = len(logits)
    L = _small_layer(20, H=32, F=32, E=E, K=K, bias=None, gating="softmax")
    router = np.zeros((E, 32), np.float32)
    router[:, 0] = logits
    L["router"] = router.view(np.uint8).ravel()
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 1.0
    return L, x


def test_softmax_route_closed_forms():
    # equal logits: every probability 1/E exactly, the first K experts (ties go
    # to the lower index), every weight 1/K exactly (E, K powers of two)
    L, x = _onehot_logit_layer(np.full(16, 0.75, np.float32), 4)
    idx, w, probs = oracle.moe_route(L, x)
    assert (probs == np.float32(1 / 16)).all()
    assert (idx[0] == [0, 1, 2, 3]).all()
    assert (w[0] == 0.25).all()
    # one dominant logit: probability 1, weight 1 (the others underflow)
    lg = np.zeros(8, np.float32)
    lg[5] = 200.0
    L, x = _onehot_logit_layer(lg, 1)
    idx, w, probs = oracle.moe_route(L, x)
    assert idx[0, 0] == 5 and w[0, 0] == 1.0 and probs[0, 5] == 1.0
    # a tie at the K boundary goes to the lower index
    L, x = _onehot_logit_layer(np.array([0, 3, 1, 3, 2, 0], np.float32), 2)
    idx, _, _ = oracle.moe_route(L, x)
    assert (idx[0] == [1, 3]).all()


def test_softmax_route_against_float64_softmax():
    L = _small_layer(21, H=256, E=64, K=8, bias=None, gating="softmax", router_std=0.2)
    x, _ = synth.activations(22, 100, 256)
    idx, w, probs = oracle.moe_route(L, x)
    W = L["router"].view(np.float32).reshape(64, 256).astype(np.float64)
    logits = (x.astype(np.float64) @ W.T).astype(np.float32).astype(np.float64)
    ref = np.exp(logits - logits.max(axis=1, keepdims=True))
    ref /= ref.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(probs, ref, rtol=2e-7, atol=1e-30)
    np.testing.assert_array_equal(
        idx, np.argsort(-probs.astype(np.float64), axis=1, kind="stable")[:, :8])
    for t in range(len(x)):
        assert probs[t, idx[t]].min() >= np.delete(probs[t], idx[t]).max()
    # renormalised from 0: the weights sum to 1 (to rounding)
    np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-12)
    S = np.take_along_axis(probs.astype(np.float64), idx, axis=1)
    np.testing.assert_allclose(w, S / S.sum(axis=1, keepdims=True), rtol=1e-15)


def test_softmax_layer_invariants():
    # identical experts: the block adds sum_k w_k * expert(x) = expert(x) (sum w = 1)
    L = _small_layer(23, H=64, F=64, E=16, K=4, bias=None, gating="softmax", router_std=0.2)
    for name in ("gate", "up", "down"):
        per = L[name].size // 16
        L[name] = np.tile(L[name][:per], 16)
    x, hid = synth.activations(24, 6, 64)
    out, idx, w, _ = oracle.moe_ffn(L, x, hid)
    L1 = dict(L, E=1, K=1, router=np.zeros(64, np.float32).view(np.uint8))
    for name in ("gate", "up", "down"):
        L1[name] = L[name][:L[name].size // 16]
    one, _, _, _ = oracle.moe_ffn(L1, x, hid)
    np.testing.assert_allclose(out - hid, one - hid, rtol=1e-5, atol=1e-7)
    # masking every selected expert leaves hidden unchanged
    for t in range(len(x)):
        o, _, _, _ = oracle.moe_ffn(L, x[t:t + 1], hid[t:t + 1], mask=set(idx[t].tolist()))
        np.testing.assert_array_equal(o, hid[t:t + 1])


# ------------------------------------------------------------------ whole block

def test_moe_dense_rederivation():
    """The block against a float64 numpy derivation from dense dequantised weights."""
    L = _small_layer(20, H=96, F=64, E=6, K=3)
    x, hid = synth.activations(21, 5, 96)
    out, idx, w, probs = oracle.moe_ffn(L, x, hid)
    G = synth.q8_0_dequant(L["gate"], 96, 64, 6)
    U = synth.q8_0_dequant(L["up"], 96, 64, 6)
    D = synth.q8_0_dequant(L["down"], 64, 96, 6)
    for t in range(5):
        xv = x[t].astype(np.float64)
        acc = np.zeros(96)
        for k in range(3):
            e = idx[t, k]
            g = G[e] @ xv
            u = U[e] @ xv
            acc += w[t, k] * (D[e] @ (g / (1 + np.exp(-g)) * u))
        np.testing.assert_allclose(out[t].astype(np.float64) - hid[t], acc, rtol=2e-5, atol=1e-6)


def test_moe_mask_equals_zeroed_expert():
    """Masking expert e (lfm2-engine.js:464) equals zeroing its down scales, bit
    for bit: its term is then w*0 added to the fp32 accumulator."""
    L = _small_layer(22, E=8, K=3)
    x, hid = synth.activations(23, 6, 64)
    idx, _, _ = oracle.moe_route(L, x)
    e = int(idx[0, 1])
    masked, _, _, _ = oracle.moe_ffn(L, x, hid, mask={e})
    Z = dict(L)
    d = np.frombuffer(L["down"].tobytes(), synth.Q8_DTYPE).copy().reshape(8, 64, 2)
    d["d"][e] = 0
    Z["down"] = d.view(np.uint8).ravel()
    zeroed, _, _, _ = oracle.moe_ffn(Z, x, hid)
    np.testing.assert_array_equal(masked, zeroed)
    all_masked, _, _, _ = oracle.moe_ffn(L, x, hid, mask=set(range(8)))
    np.testing.assert_array_equal(all_masked, hid)


def test_moe_identical_experts():
    """With every expert identical the block is (S/(S+1e-6)) * expert(x)."""
    L = _small_layer(24, E=4, K=4)
    one = lambda t, rows: np.tile(np.frombuffer(t.tobytes(), np.uint8).reshape(4, -1)[0], 4)
    for name in ("gate", "up", "down"):
        L[name] = one(L[name], None)
    x, hid = synth.activations(25, 3, 64)
    out, idx, w, probs = oracle.moe_ffn(L, x, hid)
    single = dict(L, E=1, K=1, bias=None)
    single["router"] = L["router"][: 64 * 4]
    for t in range(3):
        y1, _, w1, _ = oracle.moe_ffn(single, x[t:t + 1], np.zeros((1, 64), np.float32))
        expert = y1[0].astype(np.float64) / w1[0, 0]
        np.testing.assert_allclose(out[t].astype(np.float64) - hid[t], w[t].sum() * expert,
                                   rtol=1e-5, atol=1e-7)


def test_moe_batch_equals_per_token():
    L = _small_layer(26, H=64, F=96, E=8, K=2)
    x, hid = synth.activations(27, 7, 64)
    out, idx, w, probs = oracle.moe_ffn(L, x, hid)
    for t in range(7):
        o1, i1, w1, p1 = oracle.moe_ffn(L, x[t:t + 1], hid[t:t + 1])
        np.testing.assert_array_equal(o1[0], out[t])
        np.testing.assert_array_equal(i1[0], idx[t])
        np.testing.assert_array_equal(w1[0], w[t])


def test_moe_rejects_bad_types():
    L = _small_layer(28)
    L["router_type"] = 12
    with pytest.raises(ValueError):
        oracle.moe_ffn(L, *synth.activations(29, 1, 64))
