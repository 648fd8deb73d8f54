"""Shared helpers of the parity tests."""
import functools
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def rel_l2(a, b):
    """||a - b|| / ||b|| in float64."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (nb if nb > 0 else 1.0))


def moe_delta(hidden_out, hidden_in):
    """The MoE block's own contribution, hidden_out - hidden_in, in float64."""
    return np.asarray(hidden_out, np.float64) - np.asarray(hidden_in, np.float64)


@functools.lru_cache(maxsize=4)
def full_layer(seed, bias="uniform", router_type=0):
    import synth
    return synth.moe_layer(seed, bias=bias, router_type=router_type)


@functools.lru_cache(maxsize=1)
def gpu_context():
    import qq_hip
    return qq_hip.Context(0)


def upload_layer(ctx, L):
    """Upload an oracle-format layer dict through the C ABI."""
    H, F, E, K = L["H"], L["F"], L["E"], L["K"]
    gate = ctx.upload_q8_0(L["gate"], H, F, E)
    up = ctx.upload_q8_0(L["up"], H, F, E)
    down = ctx.upload_q8_0(L["down"], F, H, E)
    m = ctx.moe_create(L["router"], L["router_type"], L.get("bias"), gate, up, down, H, F, E, K)
    if L.get("gating") == "softmax":
        import qq_hip
        m.set_gating(qq_hip.GATING_SOFTMAX)
    return m


def dense_moe_f64(L, x, hidden, idx, w, mask=None):
    """The expert products of an MoE layer in float64 over the dequantised
    weights, written independently of the C oracle's loops (dense matrices,
    BLAS products, no fp32 rounding anywhere):

        out[t] = hidden[t] + sum_k w[t,k] * down_e (silu(gate_e x_t) * up_e x_t),  e = idx[t,k]

    with the routing (idx, w) taken as given -- the tests check it bit for
    bit against the oracle first.  Experts in `mask` are skipped (their
    weights are not renormalised, src/lfm2-engine.js:464).  It differs from
    the reference only by the reference's fp32 roundings (~1e-7 relative)."""
    import synth
    H, F, E = L["H"], L["F"], L["E"]
    x64 = np.asarray(x, np.float64).reshape(-1, H)
    out = np.array(hidden, np.float64).reshape(-1, H)
    idx = np.asarray(idx).reshape(x64.shape[0], -1)
    w = np.asarray(w, np.float64).reshape(idx.shape)
    nbH, nbF = (H + 31) // 32, (F + 31) // 32
    gsz, dsz = F * nbH * 34, H * nbF * 34
    for e in range(E):
        if mask is not None and e in mask:
            continue
        t, k = np.nonzero(idx == e)
        if t.size == 0:
            continue
        wg = synth.q8_0_dequant(L["gate"][e * gsz:(e + 1) * gsz], H, F)[0]   # [F, H]
        wu = synth.q8_0_dequant(L["up"][e * gsz:(e + 1) * gsz], H, F)[0]
        wd = synth.q8_0_dequant(L["down"][e * dsz:(e + 1) * dsz], F, H)[0]   # [H, F]
        xs = x64[t]
        g = xs @ wg.T
        u = xs @ wu.T
        h = g / (1.0 + np.exp(-g)) * u
        y = h @ wd.T
        np.add.at(out, t, w[t, k][:, None] * y)
    return out
