"""Pins of the Node restatement of the LFM2 single-token forward
(oracle/lfm2_ref.js, src/lfm2-engine.js:228-487) against an independent
float64 forward (tests/_lfm2.py: numpy, no intermediate fp32 rounding): the
two agree to fp32 rounding, and a plausible mistake planted in the float64
forward (on the CPU) is far outside that agreement."""
import numpy as np
import pytest

import synth
import _lfm2

pytestmark = pytest.mark.skipif(_lfm2.node() is None, reason="node is not installed")

TOKENS = [5, 17, 250, 3, 99, 0, 42, 7]


def _run(tmp_path, seed, tokens=TOKENS, start=0, cfg=synth.LFM2_TINY, model=_lfm2.F64Model, **kw):
    path, offs, tensors = _lfm2.write_model(tmp_path, seed, cfg, **kw)
    logits, routes = _lfm2.js_forward(tmp_path, path, offs, tensors, cfg, tokens, start)
    ref = model(tensors, cfg)
    errs = [np.linalg.norm(logits[i] - r) / np.linalg.norm(r)
            for i, r in enumerate(ref.forward(t, start + i) for t, i in zip(tokens, range(len(tokens))))]
    return logits, routes, ref, errs


@pytest.mark.parametrize("seed,kw", [
    (3, {}),                                                # tied head, F32 conv kernel
    (4, dict(conv_type=synth.TYPE_F16, tied=False)),        # F16 conv kernel, own output.weight
    (5, dict(conv_type=synth.TYPE_Q8_0, bias=None)),        # Q8_0 conv kernel, no expert bias
])
def test_js_forward_matches_float64(tmp_path, seed, kw):
    logits, routes, ref, errs = _run(tmp_path, seed, **kw)
    assert max(errs) < 2e-6, errs
    assert routes == ref.routes
    assert logits.shape == (len(TOKENS), synth.LFM2_TINY["vocab"])


def test_js_forward_from_a_later_position(tmp_path):
    """Positions start..start+T-1 with an empty cache (RoPE angles of later positions)."""
    _, _, _, errs = _run(tmp_path, 6, tokens=TOKENS[:4], start=40)
    assert max(errs) < 2e-6, errs


class _InterleavedRope(_lfm2.F64Model):
    """Rotates pairs (2i, 2i+1) instead of the split halves (i, i + half)."""

    def _rope(self, x, pos):
        hd = x.shape[-1]
        half = hd // 2
        th = pos / self.c["rope_base"] ** (np.arange(half) / half)
        a, b = x[..., 0::2].copy(), x[..., 1::2].copy()
        out = np.empty_like(x)
        out[..., 0::2] = a * np.cos(th) - b * np.sin(th)
        out[..., 1::2] = a * np.sin(th) + b * np.cos(th)
        return out


class _ConvStateNotShifted(_lfm2.F64Model):
    """Keeps the oldest conv input instead of shifting the window."""

    def forward(self, token, pos):
        saved = {i: s.copy() for i, s in self.st.items()}
        out = super().forward(token, pos)
        for i in self.st:
            self.st[i][1:] = self.st[i][1:]
            self.st[i][0] = saved[i][0]
        return out


@pytest.mark.parametrize("model", [_InterleavedRope, _ConvStateNotShifted])
def test_planted_mistakes_are_far_outside(tmp_path, model):
    _, _, _, errs = _run(tmp_path, 3, model=model)
    assert max(errs[1:]) > 1e-3, errs


def test_streamed_model_file_equals_in_memory_file(tmp_path):
    """synth.gguf_write (used for the multi-GB bench model) lays a file out byte for
    byte as synth.gguf_file does, and the pool-sliced model is well formed."""
    data, offs, _ = synth.lfm2_gguf(3, synth.LFM2_TINY)
    path = tmp_path / "s.gguf"
    _, offs2, _ = synth.lfm2_gguf(3, synth.LFM2_TINY, path=str(path))
    assert path.read_bytes() == data and offs2 == offs
    pool = synth.q8_0_pool(1, 1 << 16)
    _, offs3, tensors = synth.lfm2_gguf(4, synth.LFM2_TINY, path=str(tmp_path / "p.gguf"), pool=pool)
    for name, shape, typ, arr in tensors:
        if typ == synth.TYPE_Q8_0:
            n = shape[2] if len(shape) > 2 else 1
            assert len(arr) == n * shape[1] * (shape[0] // 32) * 34, name


def test_cpu_baseline_bench_mode_runs(tmp_path):
    """oracle/lfm2_ref.js bench: per-block and head times for the CPU baseline."""
    import json
    import os
    import subprocess
    cfg = synth.LFM2_TINY
    path, offs, tensors = _lfm2.write_model(tmp_path, 3, cfg)
    job = {"gguf": path, "kv": _lfm2.kv_dict(cfg), "tokens": [0], "start": 0,
           "tensors": {n: {"offset": offs[n], "shape": s, "type": t} for n, s, t, _ in tensors}}
    jp = tmp_path / "job.json"
    jp.write_text(json.dumps(job))
    p = subprocess.run([_lfm2.node(), os.path.join(_lfm2.ROOT, "oracle", "lfm2_ref.js"), "bench", str(jp), "0.2"],
                       capture_output=True, text=True, timeout=120, check=True)
    r = json.loads(p.stdout.strip().splitlines()[-1])
    assert r["tokens"] >= 1 and r["head_ms"] > 0
    kinds = [b["kind"] for b in r["blocks"]]
    assert kinds == ["conv+dense", "conv+dense", "attn+moe", "conv+moe", "attn+moe", "conv+moe"]
