"""The LFM2 single-token device forward (include/qq_lfm2.h) through the C ABI
against the Node restatement of the reference's forward (oracle/lfm2_ref.js,
pinned by tests/test_lfm2_oracle.py) on small synthetic model files: logits
within 1e-4 relative L2 per token, every MoE block's expert choice equal."""
import numpy as np
import pytest

import synth
import _lfm2
from _util import gpu_context, rel_l2

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(_lfm2.node() is None, reason="node is not installed")]

TOKENS = [5, 17, 250, 3, 99, 0, 42, 7]
TOL = 1e-4


def _say(*a):
    print(*a, flush=True)


def _model(tmp_path, seed, cfg=synth.LFM2_TINY, **kw):
    import qq_hip
    path, offs, tensors = _lfm2.write_model(tmp_path, seed, cfg, **kw)
    g = qq_hip.Gguf(path)
    try:
        m = qq_hip.Lfm2Model(gpu_context(), g)
    finally:
        g.close()
    return m, path, offs, tensors


def _check_tokens(tmp_path, seed, cfg=synth.LFM2_TINY, tokens=TOKENS, start=0, **kw):
    import torch
    m, path, offs, tensors = _model(tmp_path, seed, cfg, **kw)
    try:
        ref, routes = _lfm2.js_forward(tmp_path, path, offs, tensors, cfg, tokens, start)
        T, V, nl, K = len(tokens), m.info["n_vocab"], m.info["n_layers"], m.info["n_experts_used"]
        logits = torch.empty((T, V), dtype=torch.float32, device="cuda")
        idx = torch.full((T, nl, K), -1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        for t, tok in enumerate(tokens):
            m.forward_dev(tok, start + t, logits[t].data_ptr(), idx[t].data_ptr())
        gpu_context().synchronize()
        got, gi = logits.cpu().numpy(), idx.cpu().numpy()
        for t in range(T):
            err = rel_l2(got[t], ref[t])
            _say("token", t, "rel_l2", err)
            assert err < TOL, (t, err)
        moe = [l for l in range(nl) if l >= cfg["n_dense"]]
        assert [gi[t, l].tolist() for t in range(T) for l in moe] == routes
        return m, got
    except BaseException:
        m.release()
        raise


@pytest.mark.parametrize("seed,kw", [
    (3, {}),
    (4, dict(conv_type=synth.TYPE_F16, tied=False)),
    (5, dict(conv_type=synth.TYPE_Q8_0, bias=None)),
])
def test_forward_matches_oracle(tmp_path, seed, kw):
    _say("lfm2 forward", seed, kw)
    m, _ = _check_tokens(tmp_path, seed, **kw)
    m.release()


def test_forward_full_width(tmp_path):
    """LFM2-8B-A1B widths on three blocks: a dense FFN of 7168 (the residual
    matvec over 7168 inputs, 8 input values per thread), one attention block
    with 32 query / 8 KV heads (GQA ratio 4), one MoE block (8 experts of
    1792, top-4, through the batch-1 decode kernel) and the 65536-row output
    head."""
    _say("lfm2 full width")
    cfg = dict(synth.LFM2_8B_A1B, n_layers=3, attn_layers=(1,), n_dense=1, E=8, ctx=64)
    m, _ = _check_tokens(tmp_path, 12, cfg=cfg, tokens=TOKENS[:4])
    m.release()


def test_forward_rows_past_one_chunk(tmp_path):
    """H = 3072 (96 blocks per input row), dense FFNs only (the batch-1 MoE
    kernel takes H <= 2048): the output head, q/k/v, short-conv in_proj and
    dense gate/up matvecs cover a row's blocks in two chunks (64 or 80 blocks
    in flight per row group), and every matvec holds 8 or 9 input values per
    thread; 48 query / 12 KV heads."""
    _say("lfm2 H=3072")
    cfg = dict(synth.LFM2_TINY, H=3072, n_heads=48, n_head_kv=12, n_layers=4, attn_layers=(1,), n_dense=4,
               n_ff=1024, vocab=500)
    m, _ = _check_tokens(tmp_path, 21, cfg=cfg, tokens=TOKENS[:3])
    m.release()


def test_forward_routed_mask_and_payload(tmp_path):
    """qq_lfm2_forward_routed: with an expert mask (skipped in every MoE block,
    src/lfm2-engine.js:464) the logits follow the oracle run with the same
    mask, and every MoE block's onRouterUpdate payload (src/lfm2-engine.js:
    449-456) matches the oracle's: the selected experts equal, their weights
    and the E probabilities within 1e-5 relative (past the first block the
    hidden state differs from the oracle's in the last bits, and with it the
    later routers' logits)."""
    _say("lfm2 routed forward, mask and payload")
    cfg = synth.LFM2_TINY
    m, path, offs, tensors = _model(tmp_path, 6, cfg)
    try:
        tokens = TOKENS[:5]
        _, routes0 = _lfm2.js_forward(tmp_path, path, offs, tensors, cfg, tokens[:1], 0)
        mask = {routes0[0][0], routes0[1][1]}          # experts the unmasked run selects
        ref, _, pay = _lfm2.js_forward(tmp_path, path, offs, tensors, cfg, tokens, 0, mask=mask, payloads=True)
        nl = m.info["n_layers"]
        moe = [l for l in range(nl) if l >= cfg["n_dense"]]
        assert len(pay) == len(tokens) * len(moe)
        for t, tok in enumerate(tokens):
            logits, idx, w, probs = m.forward_routed(tok, t, mask=mask)
            err = rel_l2(logits, ref[t])
            _say("token", t, "rel_l2", err)
            assert err < TOL, (t, err)
            for j, l in enumerate(moe):
                p = pay[t * len(moe) + j]
                assert p["layer"] == l
                assert idx[l].tolist() == p["selected"]
                assert rel_l2(w[l], p["weights"]) < 1e-5, (t, l)
                assert rel_l2(probs[l], p["probs"]) < 1e-5, (t, l)
            for l in range(cfg["n_dense"]):          # dense rows are left as they are
                assert (idx[l] == -1).all() and np.isnan(w[l]).all()
    finally:
        m.release()


@pytest.mark.parametrize("start", [253, 700])
def test_forward_long_context(tmp_path, start):
    """Positions past 256 take the chunked attention (chunks of 256 positions and a
    join); the cache holds zeros below `start` on both sides."""
    _say("lfm2 long context", start)
    cfg = dict(synth.LFM2_TINY, ctx=1024)
    m, _ = _check_tokens(tmp_path, 8, cfg=cfg, tokens=TOKENS[:6], start=start)
    m.release()


@pytest.mark.parametrize("start", [1100, 3584])
def test_forward_long_context_full_width(tmp_path, start):
    """LFM2-8B-A1B attention widths (32 query / 8 KV heads of 64, H = 2048, a
    dense FFN of 7168) past one 256-position chunk: positions 1100.. (5
    chunks) and 3584.. (15 chunks of the 4096-position cache), each side's
    cache zero below `start` (src/lfm2-engine.js:329-392)."""
    _say("lfm2 full-width long context", start)
    cfg = dict(synth.LFM2_8B_A1B, n_layers=2, attn_layers=(1,), n_dense=2, vocab=512, ctx=4096)
    m, _ = _check_tokens(tmp_path, 14, cfg=cfg, tokens=TOKENS[:4], start=start)
    m.release()


def test_info_reset_and_host_entry_point(tmp_path):
    _say("lfm2 info/reset")
    cfg = synth.LFM2_TINY
    m, got = _check_tokens(tmp_path, 3, tokens=TOKENS[:3])
    try:
        assert m.info["n_layers"] == cfg["n_layers"] and m.info["n_vocab"] == cfg["vocab"]
        assert m.info["n_attn_layers"] == len(cfg["attn_layers"]) and m.info["head_dim"] == 64
        assert m.info["max_ctx"] == cfg["ctx"] and m.info["n_ff"] == cfg["n_ff"]
        # resetState: the same tokens again give the same logits, bit for bit
        m.reset()
        again = [m.forward(t, i) for i, t in enumerate(TOKENS[:3])]
        for t in range(3):
            np.testing.assert_array_equal(again[t], got[t])
        # skipLogits
        assert m.forward(TOKENS[3], 3, logits=False) is None
    finally:
        m.release()


def test_bad_token_position_and_file(tmp_path):
    import qq_hip
    _say("lfm2 errors")
    cfg = synth.LFM2_TINY
    m, _, _, _ = _model(tmp_path, 3)
    try:
        with pytest.raises(qq_hip.QQError, match="token"):
            m.forward(cfg["vocab"], 0)
        with pytest.raises(qq_hip.QQError, match="position"):
            m.forward(0, cfg["ctx"])
    finally:
        m.release()
    bad = dict(cfg, l_cache=4)
    with pytest.raises(qq_hip.QQError, match="l_cache"):
        _model(tmp_path, 7, bad)
