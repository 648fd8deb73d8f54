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
