#!/usr/bin/env python3
"""Benchmark of the LFM2-MoE Q8_0 MoE feed-forward path on one MI355X.

Metric: MoE-layer tokens/sec + HBM GB/s (% of peak), LFM2-8B-A1B-shape Q8_0.

A step is one pass of the MoE block (router, top-K, expert SwiGLU products,
weighted combine, residual) over one batch of synthetic tokens.  Default
workload: batch-1 decode through one MoE layer (H=2048, F=1792, E=32, K=4,
Q8_0 experts), rotating over `--layers` independently seeded layer instances
(16 x 374 MB = 6 GB resident) so that consecutive steps never find their
expert weights in L2 or the 256 MB Infinity Cache.

Other workloads (--workload): decode_b64 (64-token decode batch), prefill_2048
(2048-token chunk, Zipf-skewed routing), stack22_decode / stack22_prefill (22
independently seeded layers, rmsnorm + MoE per layer, 1 token resp. a
4096-token chunk per step), matvec (one Q8_0 matvec 1024 -> 3072, rotating
over 80 weights), qwen3_decode_b1 / qwen3_prefill_2048 (one Qwen3-30B-A3B-shaped
MoE layer, H=2048, F=768, E=128, K=8, softmax routing, no bias), lfm2_decode
(one token through a whole LFM2-8B-A1B-shaped model on the device -- 24
blocks: 18 short-conv, 6 GQA attention, 2 dense FFN, 22 MoE; vocab 65536 --
at positions 0, 1, 2, ... of one sequence; qq_lfm2_forward_dev).

Inputs are generated on the device before the timed region.  Times come from
HIP events on the stream the kernels run on.  `value` times the steps
launched call by call; `graph_ms_per_step` times the same steps replayed from
HIP graphs recorded through the library (one graph per distinct step,
qq_capture_begin/end).  The per-kernel roofline figure comes from a third
pass over the same steps in which every launch carries its own start/stop
events (hipExtLaunchKernelGGL, qq_profile_*).

Beside `value`, the batch-1 decode lines carry `host_call`: the same layer
through the host-pointer call the JS drop-in makes (x and hidden in over
PCIe, results out, a synchronise per call), timed on the host.  The default
line also carries `prefill_2048`: a shortened 2048-token prefill chunk with
the MFMA roofline of its grouped GEMMs (skip with --no-prefill-leg).

Prints one JSON line.
"""
import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwenqwen3.js_amd"))

METRIC = "MoE-layer tokens/sec + HBM GB/s (% of peak), LFM2-8B-A1B-shape Q8_0"
LFM2_METRIC = "whole-model decode tokens/sec, LFM2-8B-A1B-shape Q8_0"
HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0     # MI355X dense fp16 MFMA
H, F, E, K = 2048, 1792, 32, 4     # set per workload in main() from SHAPES
GATING = "sigmoid"
SHAPES = {
    # name: (H, F, E, K, gating)
    "lfm2": (2048, 1792, 32, 4, "sigmoid"),     # LFM2-8B-A1B MoE layer
    "qwen3": (2048, 768, 128, 8, "softmax"),    # Qwen3-30B-A3B MoE layer
}
QBLK = 34
STACK_LAYERS = 22
MV_IN, MV_OUT = 1024, 3072

WORKLOADS = {
    # name: (kind, T tokens per step, bias kind, config name)
    "decode_b1": ("layer", 1, "uniform", "moe_layer_decode_batch1"),
    "decode_b64": ("layer", 64, "uniform", "moe_layer_decode_batch64"),
    "prefill_2048": ("layer", 2048, "zipf", "moe_layer_prefill_2048_zipf"),
    "stack22_decode": ("stack", 1, "uniform", "moe_stack22_decode_batch1"),
    "stack22_prefill": ("stack", 4096, "uniform", "moe_stack22_prefill_4096"),
    "matvec": ("matvec", 1, None, "q8_0_matvec_1024x3072"),
    "qwen3_decode_b1": ("layer", 1, None, "qwen3moe_layer_decode_batch1", "qwen3"),
    "qwen3_decode_b64": ("layer", 64, None, "qwen3moe_layer_decode_batch64", "qwen3"),
    "qwen3_prefill_2048": ("layer", 2048, None, "qwen3moe_layer_prefill_2048", "qwen3"),
    "lfm2_decode": ("lfm2", 1, "uniform", "lfm2_8b_a1b_token_decode"),
}
LFM2_POS = 512        # positions cycle over 0 .. LFM2_POS - 1
LFM2_BYTES = {}       # algorithmic bytes per launch of the lfm2 kernels (set by run_lfm2)
MFMA_KERNELS = ("mfma_gateup", "mfma_down")


def expert_bytes():
    gate = F * (H // 32) * QBLK
    down = H * (F // 32) * QBLK
    return gate, down


def kernel_bytes(name, T, n_experts):
    """Algorithmic HBM bytes of one launch of `name`: every weight, router and
    activation byte the math needs, once; intermediate buffers the kernels
    exchange (partial sums, grouped rows) are not counted."""
    gate, down = expert_bytes()
    router = E * H * 4 + E * 4
    if name == "moe_decode":
        # experts, router and bias, x, hidden read and written
        return n_experts * (2 * gate + down) + router + 3 * T * H * 4
    if name == "router_logits":
        return E * H * 4 + T * H * 4
    if name in ("grouped_gateup", "stream_gateup", "mfma_gateup"):
        return n_experts * 2 * gate + T * H * 4
    if name in ("grouped_down", "stream_down", "mfma_down"):
        return n_experts * down
    if name in ("combine", "rmsnorm"):
        return 2 * T * H * 4
    if name == "q8_0_matvec":
        return MV_OUT * (MV_IN // 32) * QBLK + MV_IN * 4 + MV_OUT * 4
    return LFM2_BYTES.get(name)


def kernel_flops(name, n_pairs):
    """Algorithmic FLOPs of one launch of an expert-product kernel over n_pairs
    (token, expert) rows: 2 per multiply-add of the real rows only (padding
    rows of a tile are not counted)."""
    if name in ("mfma_gateup", "grouped_gateup", "stream_gateup"):
        return 2.0 * n_pairs * H * 2 * F
    if name in ("mfma_down", "grouped_down", "stream_down"):
        return 2.0 * n_pairs * F * H
    return None


def layer_bytes(T, n_experts):
    gate, down = expert_bytes()
    return n_experts * (2 * gate + down) + E * H * 4 + E * 4 + 2 * T * H * 4


def make_layer(torch, ctx, seed, bias_kind):
    """One layer's tensors: GGUF Q8_0 bytes made on the device, repacked by the library."""
    import qq_hip
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    tensors = []
    for in_dim, out_dim in ((H, F), (H, F), (F, H)):
        nblk = E * out_dim * (in_dim // 32)
        blocks = torch.empty((nblk, QBLK), dtype=torch.uint8, device="cuda")
        qs = torch.randint(-127, 128, (nblk, 32), generator=g, device="cuda", dtype=torch.int8)
        d = (torch.randn(nblk, generator=g, device="cuda").abs() * 0.002).to(torch.float16)
        blocks[:, 2:] = qs.view(torch.uint8)
        blocks[:, :2] = d.view(torch.uint8).view(nblk, 2)
        torch.cuda.synchronize()
        tensors.append(ctx.upload_q8_0_dev(blocks.data_ptr(), blocks.numel(), in_dim, out_dim, E))
        del blocks, qs, d
    rng = np.random.default_rng(seed)
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    if GATING == "softmax":
        layer = ctx.moe_create(router, qq_hip.TYPE_F32, None, *tensors, H, F, E, K)
        return layer.set_gating(qq_hip.GATING_SOFTMAX)
    if bias_kind == "zipf":
        k = np.arange(1, E + 1, dtype=np.float64)
        pmf = k ** -1.1
        pmf /= pmf.sum()
        bias = (0.17 * np.log(pmf[rng.permutation(E)])).astype(np.float32)
    else:
        bias = rng.uniform(-0.01, 0.01, E).astype(np.float32)
    return ctx.moe_create(router, qq_hip.TYPE_F32, bias, *tensors, H, F, E, K)


def make_matvec_weight(torch, ctx, seed):
    """One GGUF Q8_0 [1024, 3072] weight made on the device, repacked by the library."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    nblk = MV_OUT * (MV_IN // 32)
    blocks = torch.empty((nblk, QBLK), dtype=torch.uint8, device="cuda")
    blocks[:, 2:] = torch.randint(-127, 128, (nblk, 32), generator=g, device="cuda",
                                  dtype=torch.int8).view(torch.uint8)
    d = (torch.randn(nblk, generator=g, device="cuda").abs() * 0.002).to(torch.float16)
    blocks[:, :2] = d.view(torch.uint8).view(nblk, 2)
    torch.cuda.synchronize()
    return ctx.upload_q8_0_dev(blocks.data_ptr(), blocks.numel(), MV_IN, MV_OUT, 1)


CPU_RUNS = 5


def _cpu_job(kind, shape, d):
    """Raw input files for the Node baseline, from the oracle's seeded generator
    (oracle/synth.py): Q8_0 int8 uniform in [-127, 127] with fp16 scales
    |N(0,1)| * 0.002, the F32 router N(0, 0.02), the bias U(-0.01, 0.01), and
    x and hidden rows N(0,1) -- the distributions of the GPU run's inputs."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import synth

    def raw(name, arr):
        path = os.path.join(d, name)
        np.ascontiguousarray(arr).tofile(path)
        return path

    if kind == "matvec":
        w, _ = synth.matvec_case(31, MV_IN, MV_OUT)
        x = np.random.default_rng(32).standard_normal((64, MV_IN)).astype(np.float32)
        return {"kind": "matvec", "in_dim": MV_IN, "out_dim": MV_OUT, "weight": raw("w.bin", w),
                "x": raw("x.bin", x)}
    Hs, Fs, Es, Ks, gating = SHAPES[shape]
    L = synth.moe_layer(41, H=Hs, F=Fs, E=Es, K=Ks, bias=None if gating == "softmax" else "uniform",
                        gating=gating)
    x, hid = synth.activations(42, 64, Hs)
    job = {"kind": "moe", "H": Hs, "F": Fs, "E": Es, "K": Ks, "gating": gating,
           "router": raw("router.bin", L["router"]), "router_type": L["router_type"],
           "gate": raw("gate.bin", L["gate"]), "up": raw("up.bin", L["up"]), "down": raw("down.bin", L["down"]),
           "x": raw("x.bin", x), "hidden": raw("hidden.bin", hid)}
    if L.get("bias") is not None:
        job["bias"] = raw("bias.bin", L["bias"])
    return job


def _node_job(kind, shape, seconds):
    """Median rate of CPU_RUNS bounded runs of the Node baseline, or None
    without node."""
    import shutil
    import tempfile
    node = shutil.which("node")
    if not node:
        return None
    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=base) as d:
        job = _cpu_job(kind, shape, d)
        jp = os.path.join(d, "job.json")
        with open(jp, "w") as f:
            json.dump(job, f)
        per_run = max(seconds / CPU_RUNS, 0.5)
        p = subprocess.run([node, os.path.join(ROOT, "oracle", "moe_ref.js"), "bench-job", jp,
                            str(CPU_RUNS), str(per_run)],
                           capture_output=True, text=True, timeout=seconds * 4 + 300, check=True)
    return json.loads(p.stdout.strip().splitlines()[-1])


def cpu_baseline(seconds, kind, shape="lfm2"):
    """The reference's CPU path restated for Node 12 (oracle/moe_ref.js: same loop
    order and float64 arithmetic as src/tensor.js / src/lfm2-engine.js, checked bit
    for bit against the C oracle by the tests), timed on one host thread: the
    median of CPU_RUNS bounded runs of single-token calls on the oracle
    generator's inputs.  Without node, the C oracle is timed instead."""
    ncores = os.cpu_count() or 0
    if kind == "lfm2":
        return lfm2_cpu_baseline(seconds)
    r = _node_job("matvec" if kind == "matvec" else "moe", shape, seconds)
    if r and kind == "matvec":
        return {"value": round(r["median_per_s"], 3), "unit": "matvecs/s", "cores": 1, "kind": "port",
                "sample": "median of %d runs of %.1f s (%s matvecs/s) of matmulQ80xF32 (1024 -> 3072 "
                          "Q8_0, x ~ N(0,1)): the reference's JS CPU path restated for Node %s, 1 thread "
                          "of %d host cores" % (len(r["runs"]), r["seconds_per_run"],
                                                ", ".join("%.1f" % v for v in r["runs"]), r["node"], ncores)}
    per = STACK_LAYERS if kind == "stack" else 1
    if r:
        what = ("Qwen3-MoE layer calls (H=2048, F=768, E=128, K=8, softmax routing, Q8_0 experts; "
                "Qwen3Engine._moEFFN)" if shape == "qwen3" else
                "MoE-layer calls (H=2048, F=1792, E=32, K=4, Q8_0 experts; Lfm2Engine._moEFFN)")
        return {
            "value": round(r["median_per_s"] / per, 4), "unit": "tokens/s", "cores": 1,
            "kind": "port",
            "sample": "median of %d runs of %.1f s (%s tokens/s) of single-token %s on the oracle "
                      "generator's inputs (int8 uniform, fp16 scales |N(0,1)|*0.002, router N(0,0.02), "
                      "x N(0,1)): the reference's JS CPU path restated for Node %s, 1 thread of %d host "
                      "cores; tokens are independent, so tokens/s is the rate at any batch%s"
                      % (len(r["runs"]), r["seconds_per_run"], ", ".join("%.2f" % v for v in r["runs"]),
                         what, r["node"], ncores,
                         "; divided by %d layers for the stack" % per if per > 1 else ""),
        }
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import synth
    L = synth.moe_layer(7)
    x, hid = synth.activations(8, 64, H)
    oracle.moe_ffn(L, x[:1], hid[:1])
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.moe_ffn(L, x[n % 64:n % 64 + 1], hid[n % 64:n % 64 + 1])
        n += 1
    el = time.perf_counter() - t0
    return {"value": round(n / el / per, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": "%d single-token MoE-layer calls in %.1f s on the C oracle (node absent), "
                      "1 thread of %d host cores" % (n, el, ncores)}


def lfm2_model_file(seed, cfg, tag):
    """A synthetic LFM2-MoE GGUF file of shapes cfg (Q8_0 matrices sliced from
    a seeded pool of random blocks) in the temp directory."""
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import synth
    pool = synth.q8_0_pool(seed, 6 << 20)
    d = tempfile.gettempdir()
    if os.path.isdir("/dev/shm"):
        st = os.statvfs("/dev/shm")
        if st.f_bavail * st.f_frsize > (16 << 30):
            d = "/dev/shm"      # memory-backed: the 8.9 GB file is written and mapped quickly
    path = os.path.join(d, "qq_%s_%d.gguf" % (tag, os.getpid()))
    _, offs, tensors = synth.lfm2_gguf(seed, cfg, path=path, pool=pool)
    return path, offs, tensors


def lfm2_cpu_baseline(seconds):
    """oracle/lfm2_ref.js (the reference's Lfm2Engine.forward restated for Node)
    timed on a 3-block model of the full widths -- one short-conv + dense
    block, one attention + MoE block, one short-conv + MoE block, and the
    65536-word head -- and scaled to the 24 blocks of LFM2-8B-A1B (2 / 6 / 16
    of each kind).  The 24-block file (8.9 GB) does not fit Node 12's buffers."""
    import shutil
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import synth
    import _lfm2
    node = shutil.which("node")
    if not node:
        return None
    cfg = dict(synth.LFM2_8B_A1B, n_layers=3, attn_layers=(1,), n_dense=1)
    path, offs, tensors = lfm2_model_file(11, cfg, "lfm2cpu")
    try:
        job = {"gguf": path, "kv": _lfm2.kv_dict(cfg), "tokens": [0], "start": 0,
               "tensors": {n: {"offset": offs[n], "shape": sh, "type": t} for n, sh, t, _ in tensors}}
        jp = path + ".json"
        with open(jp, "w") as f:
            json.dump(job, f)
        p = subprocess.run([node, os.path.join(ROOT, "oracle", "lfm2_ref.js"), "bench", jp, str(seconds)],
                           capture_output=True, text=True, timeout=seconds * 4 + 300, check=True)
        r = json.loads(p.stdout.strip().splitlines()[-1])
    finally:
        for f in (path, path + ".json"):
            if os.path.exists(f):
                os.remove(f)
    per = {b["kind"]: b["ms"] for b in r["blocks"]}
    full = synth.LFM2_8B_A1B
    n_attn = len(full["attn_layers"])
    n_conv_dense = full["n_dense"]
    ms = (n_conv_dense * per["conv+dense"] + n_attn * per["attn+moe"] +
          (full["n_layers"] - n_attn - n_conv_dense) * per["conv+moe"] + r["head_ms"])
    ncores = os.cpu_count() or 0
    return {"value": round(1000.0 / ms, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": "%d tokens in %.1f s through a 3-block full-width LFM2 model (block ms: "
                      "conv+dense %.0f, attn+moe %.0f, conv+moe %.0f; head %.0f) with "
                      "oracle/lfm2_ref.js (the reference's Lfm2Engine.forward restated for Node %s), "
                      "scaled to 2 + 6 + 16 blocks + head = %.0f ms per token; 1 thread of %d host "
                      "cores" % (r["tokens"], r["seconds"], per["conv+dense"], per["attn+moe"],
                                 per["conv+moe"], r["head_ms"], r["node"], ms, ncores)}


def run_lfm2(args, torch, ctx, stream):
    """The whole-model decode workload.  Returns (ms_per_step, kernels,
    roofline, config, extra)."""
    import qq_hip
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import synth
    cfg = synth.LFM2_8B_A1B
    t0 = time.time()
    path, offs, tensors = lfm2_model_file(1, cfg, "lfm2gpu")
    try:
        g = qq_hip.Gguf(path)
        try:
            model = qq_hip.Lfm2Model(ctx, g)
        finally:
            g.close()
    finally:
        os.remove(path)
    setup_s = time.time() - t0
    info = model.info
    V = info["n_vocab"]
    logits = torch.empty(V, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    p0 = max(0, min(args.position0, info["max_ctx"] - LFM2_POS))

    def step(i):
        model.forward_dev((i * 7919) % V, p0 + i % LFM2_POS, logits.data_ptr())

    total_ms = _time_steps(torch, ctx, stream, step, args.steps, args.warmup)
    ms_per_step = total_ms / args.steps
    # one pass with per-launch events over the first positions of a fresh sequence
    n_prof = min(args.steps, 64)
    model.reset()
    ctx.profile_enable(n_prof * 160)
    for i in range(n_prof):
        step(i)
    prof = ctx.profile_read()
    ctx.profile_enable(0)
    ctx.synchronize()

    # algorithmic bytes per token (Q8_0: 34 bytes per 32 weights)
    Hh, V, nq = info["n_embd"], info["n_vocab"], info["n_heads"] * info["head_dim"]
    nkv = info["n_head_kv"] * info["head_dim"]
    n_attn, nl, ndense = info["n_attn_layers"], info["n_layers"], info["n_dense_lead"]
    n_conv = nl - n_attn
    q8 = QBLK / 32.0
    w_conv = (3 * Hh * Hh + Hh * Hh) * q8
    w_attn = (2 * Hh * nq + 2 * Hh * nkv) * q8
    w_dense = 3 * Hh * info["n_ff"] * q8
    w_head = Hh * V * q8
    mv_bytes = n_conv * w_conv + n_attn * w_attn + ndense * w_dense + w_head
    mv_launches = 2 * n_conv + 2 * n_attn + 2 * ndense + 1
    LFM2_BYTES["lfm2_matvec"] = mv_bytes / mv_launches
    avg_n_prof = p0 + (n_prof + 1) / 2.0
    LFM2_BYTES["lfm2_attention"] = info["n_head_kv"] * avg_n_prof * 64 * 4 * 2
    LFM2_BYTES["lfm2_embed"] = Hh * q8 + Hh * 4
    n_moe = nl - ndense
    moe_bytes = n_moe * kernel_bytes("moe_decode", 1, K)
    avg_n = p0 + (min(args.steps, LFM2_POS) + 1) / 2.0
    kv_bytes = n_attn * info["n_head_kv"] * avg_n * 64 * 4 * 2
    tok_bytes = mv_bytes + moe_bytes + kv_bytes
    kernels = kernel_table(prof, 1, K, K)
    dom, roofline = roofline_of(prof, kernels, args.workload)
    config = {"workload": "lfm2_8b_a1b_token_decode", "blocks": nl, "attention_blocks": n_attn,
              "dense_ffn_blocks": ndense, "moe_blocks": n_moe, "H": Hh, "heads": info["n_heads"],
              "kv_heads": info["n_head_kv"], "head_dim": info["head_dim"], "n_ff": info["n_ff"],
              "F": F, "E": E, "K": K, "vocab": V, "weights": "Q8_0", "activations": "f32",
              "positions": "%d..%d (step i at position %d + i %% %d, one sequence)"
                           % (p0, p0 + LFM2_POS - 1, p0, LFM2_POS),
              "timed_positions": "%d..%d" % (p0, p0 + min(args.steps, LFM2_POS) - 1)}
    extra = {"us_per_token": round(ms_per_step * 1000.0, 2),
             "hbm_bytes_per_token": int(tok_bytes),
             "hbm_gbps_token": round(tok_bytes / (ms_per_step * 1e6), 1),
             "hbm_frac_token": round(tok_bytes / (ms_per_step * 1e6) / HBM_PEAK_GBPS, 4),
             "launches_per_token": int(round(sum(c for _, c in prof.values()) / n_prof)),
             "setup_s": round(setup_s, 1)}
    model.release()
    return ms_per_step, kernels, roofline, config, extra


def copy_calibration(steps):
    """A plain copy of known size: FETCH_SIZE and WRITE_SIZE of one dispatch
    should each read 1 GiB; the ratio calibrates the traffic counters."""
    import torch
    n = 1 << 30
    a = torch.ones(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        b.copy_(a)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    print(json.dumps({"copy_bytes": n, "ms": round(ms, 4), "read_plus_write_gbps": round(2 * n / (ms * 1e6), 1)}))
    return 0


def _time_steps(torch, ctx, stream, run, steps, warmup):
    # warm-up steps are the ones just before step 0 in the rotation (-warmup .. -1),
    # so the first timed steps do not meet the instances the warm-up has touched
    for i in range(-warmup, 0):
        run(i)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(steps):
        run(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ctx.synchronize()          # raises if a device-side wait expired
    return ev0.elapsed_time(ev1)


def host_call_leg(ctx, layers, X, HID, steps, warmup):
    """The host-pointer drop-in, qq_moe_forward: the call the JS _moEFFN makes
    through the Node-API addon for every token (src/lfm2-engine.js:257).  x and
    hidden go in over PCIe, hidden and the routing come out, and the call
    synchronises.  Wall clock per call on the host, the same layer rotation as
    the device-resident steps; without and with the router payload (the
    probabilities onRouterUpdate carries)."""
    import ctypes
    L = ctx.L
    x = np.ascontiguousarray(X.cpu().numpy())
    h = np.ascontiguousarray(HID.cpu().numpy())
    S, T, H = x.shape
    K, E = layers[0].K, layers[0].E
    idx = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float64)
    probs = np.empty((T, E), np.float32)
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    px = [vp(x[s]) for s in range(S)]
    ph = [vp(h[s]) for s in range(S)]
    pi, pw, pp = vp(idx), vp(w), vp(probs)
    out = {}
    for key, want in (("us_per_call", None), ("with_router_payload_us_per_call", pp)):
        for i in range(-warmup, steps):
            if i == 0:
                t0 = time.perf_counter()
            lay = layers[i % len(layers)]
            rc = L.qq_moe_forward(ctx.h, lay.h, px[i % S], ph[i % S], T, None, pi, pw, want)
            if rc:
                raise RuntimeError("qq_moe_forward: %s" % L.qq_last_error(ctx.h).decode())
        out[key] = round((time.perf_counter() - t0) * 1e6 / steps, 2)
    out["tokens_per_s"] = round(T * 1e6 / out["us_per_call"], 1)
    out["calls"] = steps
    return out


def prefill_leg(torch, ctx, stream, steps, warmup, n_layers=4):
    """One MoE layer over a 2048-token prefill chunk with Zipf-skewed routing
    (the prefill_2048 workload, shortened): the expert products on the fp16
    MFMA grouped GEMMs, so the prefill GEMM's MFMA roofline is reported beside
    the decode line.  n_layers fresh layer instances (1.5 GB > the 256 MB
    Infinity Cache) rotated; per-launch events on the library stream.  The
    layers and inputs are those of `--workload prefill_2048` (layer seeds
    1000 + i, input seed 99), so the leg's kernel times are the ones a
    profile of that workload shows: the Zipf permutation of the experts, and
    with it the row tiles, differs from seed to seed."""
    T = 2048
    layers = [make_layer(torch, ctx, 1000 + i, "zipf") for i in range(n_layers)]
    gx = torch.Generator(device="cuda")
    gx.manual_seed(99)
    X = torch.randn((2, T, H), generator=gx, device="cuda", dtype=torch.float32)
    HID = torch.randn((2, T, H), generator=gx, device="cuda", dtype=torch.float32)
    idx = torch.empty((2, T, K), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()

    def step(i):
        layers[i % n_layers].forward_dev(X[i % 2].data_ptr(), HID[i % 2].data_ptr(), T,
                                         idx_ptr=idx[i % 2].data_ptr())

    total_ms = _time_steps(torch, ctx, stream, step, steps, warmup)
    ctx.profile_enable(steps * 10)
    for i in range(steps):
        step(i)
    prof = ctx.profile_read()
    ctx.profile_enable(0)
    ctx.synchronize()
    n_exp = float(len(np.unique(idx.cpu().numpy())))
    kernels = kernel_table(prof, T, n_exp, T * K)
    for lay in layers:
        for t in getattr(lay, "_keep", ()):
            t.release()
        lay.release()
    ms = total_ms / steps
    out = {"workload": "moe_layer_prefill_2048_zipf", "T": T, "layer_instances": n_layers, "steps": steps,
           "ms_per_step": round(ms, 4), "tokens_per_s": round(T / (ms / 1000.0), 1)}
    for name in MFMA_KERNELS:
        if name in kernels:
            k = kernels[name]
            out[name] = {"avg_us": k["avg_us"], "tflops": k["tflops"], "peak_tflops": MFMA_PEAK_TFLOPS,
                         "frac": round(k["tflops"] / MFMA_PEAK_TFLOPS, 4)}
    _, out["roofline"] = roofline_of(prof, kernels, "prefill_2048")
    ideal, target_ms = LEG_TARGETS["moe_layer_prefill_2048_zipf"]
    out["ideal"] = ideal
    out["target_ms_per_step"] = target_ms
    out["meets_target"] = ms <= target_ms
    return out


# Per workload: (ideal time at the roofline, the performance target in ms per step)
LEG_TARGETS = {
    "q8_0_matvec_1024x3072": ("0.42 us per matvec at 8 TB/s (launch bound)", None),
    "moe_layer_decode_batch64": ("47.0 us per step at 8 TB/s", 78.3e-3),
    "moe_layer_prefill_2048_zipf": ("72.2 us per step at 2.5 PFLOP/s", 180e-3),
    "moe_stack22_decode_batch1": ("129 us per token at 8 TB/s", 216e-3),
    "moe_stack22_prefill_4096": ("3.17 ms per chunk at 2.5 PFLOP/s", 7.94),
}


def leg(torch, ctx, stream, name, step, steps, warmup, tokens, launches, T, n_exp_fn, layers_per_step=1,
        value_unit="tokens/s", extra=None):
    """One configuration timed beside the headline line: `steps` steps of
    step(i) between two events on the library stream (after `warmup`), then
    the same steps again with per-launch events for the dominant kernel's
    roofline.  tokens: rows per step (matvecs for the matvec leg)."""
    total_ms = _time_steps(torch, ctx, stream, step, steps, warmup)
    ctx.profile_enable(steps * launches)
    for i in range(steps):
        step(i)
    prof = ctx.profile_read()
    ctx.profile_enable(0)
    ctx.synchronize()
    n_exp = n_exp_fn()
    kernels = kernel_table(prof, T, n_exp, T * K, decode_layers=layers_per_step if T == 1 else 1)
    _, roof = roofline_of(prof, kernels, LEG_WORKLOADS.get(name, name))
    ms = total_ms / steps
    out = {"workload": name, "steps": steps, "ms_per_step": round(ms, 5),
           "value": round(tokens / (ms / 1000.0), 1), "unit": value_unit, "roofline": roof,
           "kernels": {k: {kk: v[kk] for kk in ("avg_us", "launches", "gbps", "tflops") if kk in v}
                       for k, v in kernels.items()}}
    if layers_per_step > 1 and T == 1:
        out["us_per_token"] = round(ms * 1000.0, 2)
    ideal, target_ms = LEG_TARGETS.get(name, (None, None))
    out["ideal"] = ideal
    if target_ms is not None:
        out["target_ms_per_step"] = target_ms
        out["meets_target"] = ms <= target_ms
    if extra:
        out.update(extra)
    return out


# leg name -> the --workload whose profiles/traffic_<workload>.json holds its traffic
LEG_WORKLOADS = {"q8_0_matvec_1024x3072": "matvec", "moe_layer_decode_batch64": "decode_b64",
                 "moe_layer_prefill_2048_zipf": "prefill_2048", "moe_stack22_decode_batch1": "stack22_decode",
                 "moe_stack22_prefill_4096": "stack22_prefill"}


def config_legs(torch, ctx, stream, layers, warmup):
    """Configs 1, 3, 5a and 5b of the benchmark timed beside the batch-1 line
    (config 4 is prefill_leg): the 1024 -> 3072 matvec over 80 rotated
    weights; a 64-token decode batch over 4 of the line's layers; the 22-layer
    stack (the line's 16 layers and 6 more, 8.2 GB) for one token and for a
    4096-token chunk."""
    legs = {}
    gx = torch.Generator(device="cuda")
    gx.manual_seed(7)
    # config 1
    n_w = 80
    ws = [make_matvec_weight(torch, ctx, 500 + i) for i in range(n_w)]
    Xm = torch.randn((16, MV_IN), generator=gx, device="cuda", dtype=torch.float32)
    Ym = torch.empty((16, MV_OUT), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    legs["matvec"] = leg(torch, ctx, stream, "q8_0_matvec_1024x3072",
                         lambda i: ws[i % n_w].matvec_dev(Xm[i % 16].data_ptr(), Ym[i % 16].data_ptr(), 1),
                         400, warmup, 1, 2, 1, lambda: 0, value_unit="matvecs/s",
                         extra={"weight_instances": n_w})
    for w in ws:
        w.release()
    del Xm, Ym
    # config 3
    T = 64
    X = torch.randn((2, T, H), generator=gx, device="cuda", dtype=torch.float32)
    HID = torch.randn((2, T, H), generator=gx, device="cuda", dtype=torch.float32)
    idx = torch.empty((2, T, K), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    lay4 = layers[:4]
    legs["decode_b64"] = leg(
        torch, ctx, stream, "moe_layer_decode_batch64",
        lambda i: lay4[i % 4].forward_dev(X[i % 2].data_ptr(), HID[i % 2].data_ptr(), T, idx_ptr=idx[i % 2].data_ptr()),
        100, warmup, T, 10, T, lambda: float(np.mean([len(np.unique(idx[s].cpu().numpy())) for s in range(2)])),
        extra={"layer_instances": 4})
    del X, HID
    # configs 5a and 5b
    stack_layers = list(layers[:STACK_LAYERS])
    extra_layers = [make_layer(torch, ctx, 1000 + i, "uniform") for i in range(len(stack_layers), STACK_LAYERS)]
    stack_layers += extra_layers
    st = ctx.moe_stack(stack_layers)
    for T, steps, name in ((1, 100, "moe_stack22_decode_batch1"), (4096, 4, "moe_stack22_prefill_4096")):
        HID = torch.randn((2, T, H), generator=gx, device="cuda", dtype=torch.float32)
        idx = torch.empty((2, STACK_LAYERS, T, K), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        legs["stack22_decode" if T == 1 else "stack22_prefill"] = leg(
            torch, ctx, stream, name,
            lambda i: st.forward_dev(HID[i % 2].data_ptr(), T, eps=1e-5, idx_ptr=idx[i % 2].data_ptr()),
            steps, min(warmup, 2) if T > 1 else warmup, T, 12 * STACK_LAYERS, T,
            lambda: float(np.mean([len(np.unique(idx[s, l].cpu().numpy())) for s in range(2)
                                   for l in range(STACK_LAYERS)])),
            layers_per_step=STACK_LAYERS,
            extra={"layers": STACK_LAYERS, "per_layer": "rmsnorm(hidden) -> MoE -> hidden +=",
                   "call": "qq_moe_stack_forward_dev (%s)" % ("one launch for the 22 layers" if T == 1
                                                               else "layer after layer")})
        del HID, idx
    st.release()
    for lay in extra_layers:
        for t in getattr(lay, "_keep", ()):
            t.release()
        lay.release()
    return legs


def timed(torch, ctx, stream, step, period, steps, warmup, launches_per_step):
    """step(i) enqueues step i and depends only on i % period.

    Times `steps` steps between two events on the library stream twice: with
    every step's calls launched one by one, and with step i replayed from a
    HIP graph recorded once per residue i % period (qq_capture_begin/end).
    Then runs the steps once more, launched one by one with per-launch
    events.  Returns (eager_ms, graph_ms, {kernel: (ms_sum, count)})."""
    eager_ms = _time_steps(torch, ctx, stream, step, steps, warmup)
    graphs = []
    for r in range(period):
        ctx.capture_begin()
        step(r)
        graphs.append(ctx.capture_end())
    graph_ms = _time_steps(torch, ctx, stream, lambda i: graphs[i % period].launch(), steps, warmup)
    for g in graphs:
        g.release()
    ctx.profile_enable(steps * launches_per_step)
    for i in range(steps):
        step(i)
    prof = ctx.profile_read()
    ctx.profile_enable(0)
    ctx.synchronize()
    return eager_ms, graph_ms, prof


def kernel_table(prof, T, n_exp, n_pairs, decode_layers=1):
    """Per-kernel averages; decode_layers: layers one decode launch runs (a
    stack launch runs them all, so its algorithmic bytes are that many layers')."""
    kernels = {}
    for name, (ms, cnt) in prof.items():
        b = kernel_bytes(name, T, n_exp)
        if name == "moe_decode" and b is not None:
            b *= decode_layers
        avg_us = 1000.0 * ms / cnt
        kernels[name] = {"avg_us": round(avg_us, 3), "launches": cnt,
                         "bytes": None if b is None else int(b),
                         "gbps": None if b is None else round(b / (avg_us * 1e3), 1)}
        fl = kernel_flops(name, n_pairs)
        if fl is not None:
            kernels[name]["tflops"] = round(fl / (avg_us * 1e6), 1)
    return kernels


def roofline_of(prof, kernels, workload):
    """Roofline entry of the kernel with the largest total time."""
    dom = max(prof, key=lambda n: prof[n][0])
    k = kernels[dom]
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_%s.json" % workload)
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get(dom)
    if dom in MFMA_KERNELS:
        return dom, {"kernel": dom, "bound": "mfma", "achieved": k["tflops"],
                     "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(k["tflops"] / MFMA_PEAK_TFLOPS, 4), "traffic": traffic}
    return dom, {"kernel": dom, "bound": "hbm", "achieved": k["gbps"], "peak": HBM_PEAK_GBPS,
                 "unit": "GB/s",
                 "frac": None if k["gbps"] is None else round(k["gbps"] / HBM_PEAK_GBPS, 4),
                 "traffic": traffic}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="decode_b1")
    ap.add_argument("--layers", type=int, default=16, help="distinct layer instances rotated over")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill-leg", action="store_true",
                    help="decode_b1: skip the 2048-token prefill GEMM leg reported beside the line")
    ap.add_argument("--no-legs", action="store_true",
                    help="decode_b1: skip the legs of configs 1, 3, 5a and 5b reported beside the line")
    ap.add_argument("--position0", type=int, default=0,
                    help="lfm2_decode: first position of the timed sequence (step i runs at "
                         "position0 + i %% 512)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only time a 1 GiB device-to-device copy (reference kernel for the "
                         "rocprof FETCH_SIZE / WRITE_SIZE scale factors)")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.steps)

    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (--gpus %d refused)"
              % args.gpus, file=sys.stderr)
        return 2

    import torch
    import qq_hip

    kind, T, bias_kind, wname = WORKLOADS[args.workload][:4]
    shape = WORKLOADS[args.workload][4] if len(WORKLOADS[args.workload]) > 4 else "lfm2"
    global H, F, E, K, GATING
    H, F, E, K, GATING = SHAPES[shape]
    torch.cuda.init()
    ctx = qq_hip.Context(0)
    # the library launches on this stream; every event below is recorded on it
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)
    gx = torch.Generator(device="cuda")
    gx.manual_seed(99)
    extra = {}

    if kind == "lfm2":
        keep = []
        ms_per_step, kernels, roofline, config, extra = run_lfm2(args, torch, ctx, stream)
        value, unit, dtype, graph_ms = 1000.0 / ms_per_step, "tokens/s", "f32", None
    elif kind == "matvec":
        n_w = 80                      # 80 x 3.36 MB > the 256 MB Infinity Cache
        keep = [make_matvec_weight(torch, ctx, 500 + i) for i in range(n_w)]
        X = torch.randn((16, MV_IN), generator=gx, device="cuda", dtype=torch.float32)
        Y = torch.empty((16, MV_OUT), device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        period = n_w

        def step(i):
            keep[i % n_w].matvec_dev(X[i % 16].data_ptr(), Y[i % 16].data_ptr(), 1)

        total_ms, graph_ms, prof = timed(torch, ctx, stream, step, period, args.steps,
                                         args.warmup, 2)
        ms_per_step = total_ms / args.steps
        kernels = kernel_table(prof, 1, 0, 0)
        dom, roofline = roofline_of(prof, kernels, args.workload)
        value, unit = args.steps / (total_ms / 1000.0), "matvecs/s"
        config = {"workload": wname, "in_dim": MV_IN, "out_dim": MV_OUT, "weights": "Q8_0",
                  "weight_instances": n_w}
        dtype = "f32"
        extra["hbm_gbps"] = round(kernel_bytes("q8_0_matvec", 1, 0) / (ms_per_step * 1e6), 1)
    else:
        stack = kind == "stack"
        n_layers = STACK_LAYERS if stack else (args.layers if T == 1 else min(args.layers, 4))
        keep = [make_layer(torch, ctx, 1000 + i, bias_kind) for i in range(n_layers)]
        S = 64 if T == 1 else 2
        X = torch.randn((S, T, H), generator=gx, device="cuda", dtype=torch.float32)
        HID = torch.randn((S, T, H), generator=gx, device="cuda", dtype=torch.float32)
        idx = torch.empty((S, n_layers if stack else 1, T, K), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()

        if stack:
            moe_stack = ctx.moe_stack(keep)

            def step(i):
                # one token (or chunk) through every layer: hidden += MoE(rmsnorm(hidden))
                # (qq_moe_stack_forward_dev: one launch for a single token)
                s = i % S
                moe_stack.forward_dev(HID[s].data_ptr(), T, eps=1e-5, idx_ptr=idx[s].data_ptr())
        else:
            def step(i):
                s = i % S
                keep[i % n_layers].forward_dev(X[s].data_ptr(), HID[s].data_ptr(), T,
                                               idx_ptr=idx[s, 0].data_ptr())

        calls = n_layers if stack else 1
        period = S if stack else int(np.lcm(S, n_layers))
        total_ms, graph_ms, prof = timed(torch, ctx, stream, step, period, args.steps,
                                         args.warmup, 10 * calls)
        ms_per_step = total_ms / args.steps
        # distinct experts per layer call (weights each call must read at least once)
        used = idx.cpu().numpy()
        ns = min(S, args.steps)
        n_exp = float(np.mean([len(np.unique(used[s, l])) for s in range(ns)
                               for l in range(used.shape[1])]))
        n_pairs = T * K
        kernels = kernel_table(prof, T, n_exp, n_pairs, decode_layers=STACK_LAYERS if stack and T == 1 else 1)
        dom, roofline = roofline_of(prof, kernels, args.workload)
        value, unit = T * args.steps / (total_ms / 1000.0), "tokens/s"
        config = {"workload": wname, "H": H, "F": F, "E": E, "K": K, "T": T,
                  "weights": "Q8_0", "activations": "f32", "router": "f32 (f64 accumulate)",
                  "gating": "softmax (Qwen3-MoE)" if GATING == "softmax" else "sigmoid + bias (LFM2-MoE)",
                  "layer_instances": n_layers, "distinct_experts_per_layer_call": round(n_exp, 2)}
        if stack:
            config["per_layer"] = "rmsnorm(hidden) -> MoE -> hidden +="
            config["call"] = "qq_moe_stack_forward_dev (%s)" % (
                "one launch for the 22 layers" if T == 1 else "layer after layer")
            moe_stack.release()
        dtype = "f16" if dom in MFMA_KERNELS else "f32"
        lb = layer_bytes(T, n_exp) * calls
        extra["hbm_gbps_layer"] = round(lb / (ms_per_step * 1e6), 1)
        extra["hbm_frac_layer"] = round(lb / (ms_per_step * 1e6) / HBM_PEAK_GBPS, 4)
        extra["tflops_layer"] = round(6.0 * n_pairs * H * F * calls / (ms_per_step * 1e9), 2)
        if stack and T == 1:
            extra["us_per_token"] = round(ms_per_step * 1000.0, 2)
        if not stack and T == 1:
            # beside `value`: the same layer through the host-pointer call (PCIe included)
            extra["host_call"] = host_call_leg(ctx, keep, X, HID, min(args.steps, 400), min(args.warmup, 40))
        if args.workload == "decode_b1" and not args.no_prefill_leg:
            # beside `value`: the prefill GEMM's MFMA roofline on a 2048-token chunk
            extra["prefill_2048"] = prefill_leg(torch, ctx, stream, max(min(args.steps, 20), 5),
                                                max(min(args.warmup, 3), 1))
        if args.workload == "decode_b1" and not args.no_legs:
            # beside `value`: every other configuration of the benchmark
            extra["legs"] = config_legs(torch, ctx, stream, keep, max(min(args.warmup, 5), 1))
            if "prefill_2048" in extra:
                extra["legs"]["prefill_2048"] = extra["prefill_2048"]

    result = {
        "metric": LFM2_METRIC if kind == "lfm2" else METRIC,
        "value": round(value, 1),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": config,
    }
    result.update(extra)
    # the same steps replayed from HIP graphs
    result["graph_ms_per_step"] = None if graph_ms is None else round(graph_ms / args.steps, 5)
    result["roofline"] = roofline
    result["kernels"] = kernels
    for obj in keep:
        for t in getattr(obj, "_keep", ()):
            t.release()
        obj.release()
    ctx.close()

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds, kind, shape)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
