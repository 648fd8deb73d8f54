"""The seeded workload generator: byte layout of the reference's GGUF Q8_0
tensors and the routing skew of the prefill workload."""
import numpy as np

import oracle
import synth


def test_q8_0_block_layout():
    rng = np.random.default_rng(0)
    w = synth.q8_0_tensor(rng, 64, 3, n_mats=2)
    assert w.nbytes == 2 * 3 * 2 * 34
    raw = w.tobytes()
    # block (mat 1, column 2, block 1) starts at ((1*3 + 2)*2 + 1) * 34
    off = ((1 * 3 + 2) * 2 + 1) * 34
    d = np.frombuffer(raw[off:off + 2], "<f2")[0]
    qs = np.frombuffer(raw[off + 2:off + 34], np.int8)
    dense = synth.q8_0_dequant(w, 64, 3, 2)
    np.testing.assert_array_equal(dense[1, 2, 32:64], qs.astype(np.float64) * float(d))
    assert np.abs(np.frombuffer(w.tobytes(), synth.Q8_DTYPE)["qs"]).max() <= 127


def test_scales_are_fp16_of_abs_normal():
    rng = np.random.default_rng(1)
    w = synth.q8_0_tensor(rng, 32, 20000)
    d = np.frombuffer(w.tobytes(), synth.Q8_DTYPE)["d"].astype(np.float64)
    assert (d >= 0).all()
    # |N(0,1)| * 0.002 has mean 0.002 * sqrt(2/pi)
    assert abs(d.mean() - 0.002 * np.sqrt(2 / np.pi)) < 2e-5


def test_zipf_prefill_routing_is_skewed():
    """The 2048-token prefill workload's routing: hot experts take 300+ tokens,
    cold ones fewer than 10 (counted on the oracle's own routing)."""
    L = synth.moe_layer(2, bias="zipf")
    x, _ = synth.activations(303, 2048, 2048)
    idx, _, _ = oracle.moe_route(L, x)
    counts = np.bincount(idx.ravel(), minlength=32)
    assert counts.max() >= 300 and counts.min() < 10, counts
