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
