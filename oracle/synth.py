"""Seeded synthetic inputs in the reference's GGUF byte layout.

TEST INFRASTRUCTURE: used by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg to build identical inputs for the HIP path and the oracle.

Layouts follow the reference:
  * Q8_0 block = {fp16 d (little-endian) @+0, int8 qs[32] @+2}, 34 bytes
    (src/tensor.js:1-2, src/gguf.js:307-309).
  * A 2-D GGUF tensor [in_dim, out_dim] is column-major: column c holds
    ceil(in_dim/32) blocks (src/tensor.js:4-5, 36).
  * A 3-D expert tensor [in_dim, out_dim, E] is E such matrices back to back
    (src/lfm2-engine.js:489-505).
  * The F32 router [H, E] is expert-major: column e is H floats
    (src/tensor.js:469-482).

Value distributions are the benchmark workloads': qs ~ U{-127..127},
d = fp16_RNE(|N(0,1)| * 0.002), router ~ N(0, 0.02), activations ~ N(0, 1).
"""
import numpy as np

QK = 32
BLK = 34
Q8_DTYPE = np.dtype([("d", "<f2"), ("qs", "i1", (QK,))])
assert Q8_DTYPE.itemsize == BLK

TYPE_F32 = 0
TYPE_Q8_0 = 8

# Zipf(s=1.1) expert bias for the skewed prefill workload:
# bias_e = ZIPF_ALPHA * ln(pmf(rank_e)) over a seeded expert permutation.
# With this alpha the hottest experts receive 300+ of the 2048 tokens and the
# coldest fewer than 10 (tests/test_synth.py checks this on the oracle's routing).
ZIPF_S = 1.1
ZIPF_ALPHA = 0.17


def q8_0_tensor(rng, in_dim, out_dim, n_mats=1, scale=0.002):
    """GGUF-layout Q8_0 bytes of n_mats matrices [in_dim, out_dim]."""
    nb = (in_dim + QK - 1) // QK
    n = n_mats * out_dim * nb
    blocks = np.empty(n, Q8_DTYPE)
    blocks["qs"] = rng.integers(-127, 128, size=(n, QK), dtype=np.int8)
    if in_dim % QK:
        # the reference never reads past in_dim (src/tensor.js:44); zero the tail
        blocks["qs"].reshape(n_mats, out_dim, nb, QK)[:, :, -1, in_dim % QK:] = 0
    blocks["d"] = (np.abs(rng.standard_normal(n)) * scale).astype(np.float16)
    return blocks.view(np.uint8)


def q8_0_dequant(buf, in_dim, out_dim, n_mats=1):
    """float64 [n_mats, out_dim, in_dim] dense view of GGUF Q8_0 bytes."""
    nb = (in_dim + QK - 1) // QK
    blocks = np.frombuffer(np.ascontiguousarray(buf).tobytes(), Q8_DTYPE).reshape(n_mats, out_dim, nb)
    w = blocks["qs"].astype(np.float64) * blocks["d"].astype(np.float64)[..., None]
    return w.reshape(n_mats, out_dim, nb * QK)[:, :, :in_dim]


def zipf_bias(rng, E, s=ZIPF_S, alpha=ZIPF_ALPHA):
    k = np.arange(1, E + 1, dtype=np.float64)
    pmf = k ** (-s)
    pmf /= pmf.sum()
    perm = rng.permutation(E)
    return (alpha * np.log(pmf[perm])).astype(np.float32)


def moe_layer(seed, H=2048, F=1792, E=32, K=4, bias="uniform", router_type=TYPE_F32,
              router_std=0.02, gating="sigmoid"):
    """One LFM2-MoE MoE layer's tensors, as Lfm2Engine binds them
    (src/lfm2-engine.js:129-137), or with gating="softmax" a Qwen3-MoE layer
    (src/qwen3-engine.js:48-73: no bias tensor; pass bias=None).

    bias: "uniform" -> U(-0.01, 0.01) F32; "zipf" -> Zipf(1.1) skew; None -> absent.
    router_type: TYPE_F32 (float32 [H, E]) or TYPE_Q8_0.
    """
    rng = np.random.default_rng(seed)
    if router_type == TYPE_F32:
        router = (rng.standard_normal((E, H)) * router_std).astype(np.float32).view(np.uint8).ravel()
    elif router_type == TYPE_Q8_0:
        router = q8_0_tensor(rng, H, E, 1, scale=router_std / 64.0)
    else:
        raise ValueError(router_type)
    if bias is None:
        b = None
    elif bias == "uniform":
        b = rng.uniform(-0.01, 0.01, E).astype(np.float32)
    elif bias == "zipf":
        b = zipf_bias(rng, E)
    else:
        raise ValueError(bias)
    return {
        "H": H, "F": F, "E": E, "K": K,
        "router_type": router_type, "router": router,
        "bias_type": TYPE_F32, "bias": b,
        "gate": q8_0_tensor(rng, H, F, E),
        "up": q8_0_tensor(rng, H, F, E),
        "down": q8_0_tensor(rng, F, H, E),
        "gating": gating,
    }


def activations(seed, T, H):
    """(x, hidden): x is the ffn_norm output fed to the MoE, hidden the residual."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    hidden = rng.standard_normal((T, H)).astype(np.float32)
    return x, hidden


def matvec_case(seed, in_dim=1024, out_dim=3072):
    """Q8_0 matvec workload: GGUF [in_dim, out_dim] weight and x ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    w = q8_0_tensor(rng, in_dim, out_dim)
    x = rng.standard_normal(in_dim).astype(np.float32)
    return w, x
