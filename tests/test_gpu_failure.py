"""Failure path of the device-side waits of the batch-1 decode kernel and of
the one-launch routing and dispatch of small batches, forced from the host (qq_set_wait_limit): with a zero bound every wait gives up at its
first poll that misses a word, the kernel still runs to its end, and the call
either reports the timeout or -- when every wait happened to find its words
on the first poll -- returns the correct result; never a wrong result without
an error.  A failed call leaves each element of hidden at its old or its
correct new value.  The calls after it, with the default bound, are correct:
the host moves the device epoch past every tag the failed launch can have
used, so words it left behind (planted here through a test hook) are never
accepted.  An LFM2 model refuses to run after a timeout until it is reset."""
import numpy as np
import pytest

import oracle
import qq_hip
import synth
from _util import full_layer, gpu_context, moe_delta, rel_l2, upload_layer

pytestmark = pytest.mark.gpu


def test_zero_wait_bound_fails_loudly_and_recovers():
    import torch
    import synth
    print("decode wait bound 0, then default", flush=True)
    ctx = gpu_context()
    L = full_layer(11)
    m = upload_layer(ctx, L)
    try:
        x, h0 = synth.activations(31, 4, L["H"])
        ref_h, ref_idx, _, _ = oracle.moe_ffn(L, x, h0)
        dx = torch.from_numpy(x).cuda()
        dh = torch.from_numpy(h0).cuda()
        idx = torch.full((4, L["K"]), -1, dtype=torch.int32, device="cuda")
        # the new rows as the default bound computes them (the kernel's sums
        # run in a fixed order, so a repeat gives the same bits)
        new_h = dh.clone()
        for t in range(3):
            m.forward_dev(dx[t].data_ptr(), new_h[t].data_ptr(), 1)
        torch.cuda.synchronize()
        ctx.synchronize()
        new_h = new_h.cpu().numpy()
        failed = 0
        fail_e0 = None
        ctx.set_wait_limit(0)
        try:
            for t in range(3):
                e0 = ctx.debug_epoch()
                m.forward_dev(dx[t].data_ptr(), dh[t].data_ptr(), 1, idx_ptr=idx[t].data_ptr())
                try:
                    ctx.synchronize()
                except qq_hip.QQError as e:
                    assert "timed out" in str(e), e
                    failed += 1
                    fail_e0 = e0
                    # every element is its old or its correct new value
                    got = dh[t].cpu().numpy()
                    old_or_new = (got.view(np.uint32) == h0[t].view(np.uint32)) | \
                                 (got.view(np.uint32) == new_h[t].view(np.uint32))
                    assert old_or_new.all(), np.flatnonzero(~old_or_new)[:8]
                    # the epoch moved past the tags of the failed call and of
                    # a workgroup that started after workgroup 0 advanced it
                    e1 = ctx.debug_epoch()
                    assert (e1 - e0) % (1 << 32) >= 2 * 1 + 2, (e0, e1)
                    dh[t].copy_(torch.from_numpy(h0[t]))
                    continue
                assert ctx.debug_epoch() == (e0 + 1) % (1 << 32)
                # no error reported: the result must be the right one
                got = dh[t].cpu().numpy()
                assert np.array_equal(idx[t].cpu().numpy(), ref_idx[t])
                assert rel_l2(moe_delta(got, h0[t]), moe_delta(ref_h[t], h0[t])) < 1e-4
        finally:
            ctx.set_wait_limit(qq_hip.QQ_WAIT_LIMIT_US_DEFAULT)
        print("calls that timed out:", failed, "of 3", flush=True)
        # the workgroups start up to ~0.5 us apart and poll the routing table
        # right after publishing their own logits, so the first poll of some
        # workgroup misses a later member's word in every call
        # words tagged as a failed call's late workgroup would have left them
        # (the failed call's tag and the one after it) are never accepted
        assert failed >= 1
        e_fail = ctx.debug_epoch()
        for d in (1, 2):
            ctx.debug_plant_words(fail_e0 + d)
        assert ctx.debug_epoch() == e_fail
        # recovery: fresh rows through the default bound, exact routing and 1e-4
        for t in range(3, 4):
            m.forward_dev(dx[t].data_ptr(), dh[t].data_ptr(), 1, idx_ptr=idx[t].data_ptr())
        ctx.synchronize()
        assert np.array_equal(idx[3].cpu().numpy(), ref_idx[3])
        assert rel_l2(moe_delta(dh[3].cpu().numpy(), h0[3]), moe_delta(ref_h[3], h0[3])) < 1e-4
        # and the host-pointer call
        out, oidx, _, _ = m.forward(x[:1], h0[:1])
        assert np.array_equal(oidx, ref_idx[:1])
        assert rel_l2(moe_delta(out, h0[:1]), moe_delta(ref_h[:1], h0[:1])) < 1e-4
    finally:
        m.release()


def test_wait_limit_rejects_negative():
    ctx = gpu_context()
    with pytest.raises(qq_hip.QQError):
        ctx.set_wait_limit(-1)


def test_planted_words_of_the_current_tag_are_accepted():
    """The check above is not vacuous: words planted with the tag the next
    call will use do reach its result (the exchange reads them)."""
    import torch
    import synth
    print("decode with words planted at the next tag", flush=True)
    ctx = gpu_context()
    L = full_layer(12)
    m = upload_layer(ctx, L)
    try:
        x, h0 = synth.activations(32, 1, L["H"])
        ref_h, ref_idx, _, _ = oracle.moe_ffn(L, x, h0)
        dx = torch.from_numpy(x).cuda()
        dh = torch.from_numpy(h0).cuda()
        torch.cuda.synchronize()
        ctx.debug_plant_words(ctx.debug_epoch() + 1)
        m.forward_dev(dx[0].data_ptr(), dh[0].data_ptr(), 1)
        ctx.synchronize()
        bad = rel_l2(moe_delta(dh[0].cpu().numpy(), h0[0]), moe_delta(ref_h[0], h0[0]))
        assert not bad < 1e-4, bad
        # and the next call is exact again (its tag is fresh)
        dh[0].copy_(torch.from_numpy(h0[0]))
        m.forward_dev(dx[0].data_ptr(), dh[0].data_ptr(), 1)
        ctx.synchronize()
        assert rel_l2(moe_delta(dh[0].cpu().numpy(), h0[0]), moe_delta(ref_h[0], h0[0])) < 1e-4
    finally:
        m.release()


@pytest.mark.skipif(__import__("_lfm2").node() is None, reason="node is not installed")
def test_lfm2_forward_refuses_after_a_timeout(tmp_path):
    """An LFM2 model's forward fails with QQ_E_STATE after a timed-out call on
    its context until qq_lfm2_reset, then runs and matches a fresh model."""
    import _lfm2
    print("lfm2 forward after a timed-out decode wait", flush=True)
    cfg = synth.LFM2_TINY
    path, offs, tensors = _lfm2.write_model(tmp_path, 21, cfg)
    ctx = gpu_context()
    g = qq_hip.Gguf(path)
    try:
        m = qq_hip.Lfm2Model(ctx, g)
    finally:
        g.close()
    try:
        ref = m.forward(5, 0).copy()
        m.reset()
        ctx.set_wait_limit(0)
        timed_out = False
        try:
            for _ in range(4):
                try:
                    m.forward(5, 0)
                except qq_hip.QQError as e:
                    assert "timed out" in str(e), e
                    timed_out = True
                    break
                m.reset()
        finally:
            ctx.set_wait_limit(qq_hip.QQ_WAIT_LIMIT_US_DEFAULT)
        assert timed_out
        with pytest.raises(qq_hip.QQError, match="qq_lfm2_reset"):
            m.forward(5, 0)
        m.reset()
        got = m.forward(5, 0)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        m.release()


def test_stack_zero_wait_bound_fails_loudly_and_recovers():
    """The one-launch stack under a zero wait bound: the call reports the
    timeout (or is exact), each element of hidden is its old value or the
    stack's correct result, the epoch moves past every tag the launch can
    have used (2 per layer), and the next call is exact."""
    import torch
    print("stack decode wait bound 0, then default", flush=True)
    ctx = gpu_context()
    n, H = 6, 256
    Ls = [synth.moe_layer(900 + l, H=H, F=192, E=16, K=4) for l in range(n)]
    layers = [upload_layer(ctx, L) for L in Ls]
    stack = ctx.moe_stack(layers)
    try:
        _, h0 = synth.activations(33, 1, H)
        good = torch.from_numpy(h0.copy()).cuda()
        torch.cuda.synchronize()
        stack.forward_dev(good.data_ptr(), 1)
        ctx.synchronize()
        good = good.cpu().numpy()
        failed = 0
        ctx.set_wait_limit(0)
        try:
            for _ in range(3):
                dh = torch.from_numpy(h0.copy()).cuda()
                torch.cuda.synchronize()
                e0 = ctx.debug_epoch()
                stack.forward_dev(dh.data_ptr(), 1)
                try:
                    ctx.synchronize()
                except qq_hip.QQError as e:
                    assert "timed out" in str(e), e
                    failed += 1
                    got = dh.cpu().numpy()
                    ok = (got.view(np.uint32) == h0.view(np.uint32)) | (got.view(np.uint32) == good.view(np.uint32))
                    assert ok.all()
                    assert (ctx.debug_epoch() - e0) % (1 << 32) >= 2 * n + 2
                    for d in range(1, 2 * n + 1):
                        ctx.debug_plant_words(e0 + d)
                    continue
                assert np.array_equal(dh.cpu().numpy().view(np.uint32), good.view(np.uint32))
                assert ctx.debug_epoch() == (e0 + n) % (1 << 32)
        finally:
            ctx.set_wait_limit(qq_hip.QQ_WAIT_LIMIT_US_DEFAULT)
        assert failed >= 1
        dh = torch.from_numpy(h0.copy()).cuda()
        torch.cuda.synchronize()
        stack.forward_dev(dh.data_ptr(), 1)
        ctx.synchronize()
        assert np.array_equal(dh.cpu().numpy().view(np.uint32), good.view(np.uint32))
    finally:
        stack.release()
        for m in layers:
            for t in m._keep:
                t.release()
            m.release()


def test_host_call_recovers_through_the_multi_launch_path():
    """qq_moe_forward under a zero wait bound: a timed-out decode launch is
    run again through the multi-launch path (no co-residency needed), so
    every call returns the oracle's routing and a result within 1e-4."""
    print("host-pointer decode under wait bound 0", flush=True)
    ctx = gpu_context()
    L = full_layer(13)
    m = upload_layer(ctx, L)
    try:
        x, h0 = synth.activations(34, 3, L["H"])
        ref_h, ref_idx, ref_w, _ = oracle.moe_ffn(L, x, h0)
        t0 = ctx.debug_epoch()
        ctx.set_wait_limit(0)
        try:
            for t in range(3):
                out, idx, w, _ = m.forward(x[t:t + 1], h0[t:t + 1])
                assert np.array_equal(idx, ref_idx[t:t + 1])
                assert np.array_equal(w, ref_w[t:t + 1])
                assert rel_l2(moe_delta(out, h0[t:t + 1]), moe_delta(ref_h[t:t + 1], h0[t:t + 1])) < 1e-4
        finally:
            ctx.set_wait_limit(qq_hip.QQ_WAIT_LIMIT_US_DEFAULT)
        # the decode launches did time out (the epoch moved past their tags)
        assert (ctx.debug_epoch() - t0) % (1 << 32) >= qq_hip.SYNC_EPOCH_SKIP
    finally:
        m.release()


def test_batch_routing_zero_wait_bound_fails_loudly_and_recovers():
    """The one-launch router + top-K + dispatch of a 64-token batch under a
    zero wait bound: a call that reports the timeout leaves hidden exactly as
    it was (its dispatch is written empty, so the expert kernels behind it do
    nothing), one that does not is correct; words left with the failed call's
    tags are never accepted; the host-pointer call is run again through the
    multi-launch path and is correct."""
    import torch
    print("batch routing wait bound 0, then default", flush=True)
    ctx = gpu_context()
    L = full_layer(12)
    m = upload_layer(ctx, L)
    T = 64
    try:
        x, h0 = synth.activations(35, T, L["H"])
        ref_h, ref_idx, ref_w, _ = oracle.moe_ffn(L, x, h0)
        dx = torch.from_numpy(x).cuda()
        dh = torch.from_numpy(h0).cuda()
        idx = torch.full((T, L["K"]), -1, dtype=torch.int32, device="cuda")
        failed = 0
        fail_e0 = None
        ctx.set_wait_limit(0)
        try:
            for _ in range(3):
                dh.copy_(torch.from_numpy(h0))
                torch.cuda.synchronize()
                e0 = ctx.debug_epoch()
                m.forward_dev(dx.data_ptr(), dh.data_ptr(), T, idx_ptr=idx.data_ptr())
                try:
                    ctx.synchronize()
                except qq_hip.QQError as e:
                    assert "timed out" in str(e), e
                    failed += 1
                    fail_e0 = e0
                    got = dh.cpu().numpy()
                    assert np.array_equal(got.view(np.uint32), h0.view(np.uint32))
                    assert (ctx.debug_epoch() - e0) % (1 << 32) >= qq_hip.SYNC_EPOCH_SKIP
                    continue
                assert ctx.debug_epoch() == (e0 + 1) % (1 << 32)
                assert np.array_equal(idx.cpu().numpy(), ref_idx)
                assert rel_l2(moe_delta(dh.cpu().numpy(), h0), moe_delta(ref_h, h0)) < 1e-4
        finally:
            ctx.set_wait_limit(qq_hip.QQ_WAIT_LIMIT_US_DEFAULT)
        print("calls that timed out:", failed, "of 3", flush=True)
        # workgroup 0 polls its token tile's other slices right after
        # publishing its own, before the later workgroups have published
        assert failed >= 1
        for d in (1, 2):
            ctx.debug_plant_words(fail_e0 + d)
        dh.copy_(torch.from_numpy(h0))
        torch.cuda.synchronize()
        m.forward_dev(dx.data_ptr(), dh.data_ptr(), T, idx_ptr=idx.data_ptr())
        ctx.synchronize()
        assert np.array_equal(idx.cpu().numpy(), ref_idx)
        assert rel_l2(moe_delta(dh.cpu().numpy(), h0), moe_delta(ref_h, h0)) < 1e-4
        # the host-pointer call under a zero bound: retried without the fused launch
        t0 = ctx.debug_epoch()
        ctx.set_wait_limit(0)
        try:
            out, oidx, ow, _ = m.forward(x, h0)
        finally:
            ctx.set_wait_limit(qq_hip.QQ_WAIT_LIMIT_US_DEFAULT)
        assert np.array_equal(oidx, ref_idx)
        assert np.array_equal(ow, ref_w)
        assert rel_l2(moe_delta(out, h0), moe_delta(ref_h, h0)) < 1e-4
        assert (ctx.debug_epoch() - t0) % (1 << 32) >= qq_hip.SYNC_EPOCH_SKIP
    finally:
        m.release()
