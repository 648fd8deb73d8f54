#!/usr/bin/env python3
"""Benchmark of the LFM2-MoE Q8_0 MoE layer on one MI355X.

Metric: MoE-layer tokens/sec + HBM GB/s (% of peak), LFM2-8B-A1B-shape Q8_0.

A step is one pass of the MoE block (router, top-K, expert SwiGLU products,
weighted combine, residual) over one batch of synthetic tokens.  Default
workload: batch-1 decode through one MoE layer (H=2048, F=1792, E=32, K=4,
Q8_0 experts), rotating over `--layers` independently seeded layer instances
(16 x 374 MB = 6 GB resident) so that consecutive steps never find their
expert weights in L2 or the 256 MB Infinity Cache.

Inputs are generated on the device before the timed region.  Times come from
HIP events on the stream the kernels run on; the per-kernel roofline figure
comes from a second pass over the same steps with every launch bracketed by
its own event pair (qq_profile_*).

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
HBM_PEAK_GBPS = 8000.0
H, F, E, K = 2048, 1792, 32, 4
QBLK = 34

WORKLOADS = {
    # name: (T tokens per step, bias kind, description)
    "decode_b1": (1, "uniform", "moe_layer_decode_batch1"),
    "decode_b64": (64, "uniform", "moe_layer_decode_batch64"),
    "prefill_2048": (2048, "zipf", "moe_layer_prefill_2048_zipf"),
}


def expert_bytes():
    gate = F * (H // 32) * QBLK
    down = H * (F // 32) * QBLK
    return gate, down


def kernel_bytes(name, T, n_experts, n_pairs):
    """Algorithmic HBM bytes of one launch of `name`: every weight, router and
    activation byte the math needs, once; intermediate buffers the kernels
    exchange (partial sums, grouped rows) are not counted."""
    gate, down = expert_bytes()
    router = E * H * 4 + E * 4
    if name == "decode_experts":
        return n_experts * (2 * gate + down) + router + T * H * 4
    if name == "decode_combine":
        return 2 * T * H * 4
    if name == "router_logits":
        return E * H * 4 + T * H * 4
    if name == "grouped_gateup":
        return n_experts * 2 * gate + T * H * 4
    if name == "grouped_down":
        return n_experts * down
    if name == "combine":
        return 2 * T * H * 4
    return None


MFMA_KERNELS = ("mfma_gateup", "mfma_down")
MFMA_PEAK_TFLOPS = 2500.0     # MI355X dense fp16 MFMA


def kernel_flops(name, n_pairs):
    """Algorithmic FLOPs of one launch of an expert-product kernel over n_pairs
    (token, expert) rows: 2 per multiply-add of the real rows only (padding
    rows of a tile are not counted)."""
    if name in ("mfma_gateup", "grouped_gateup"):
        return 2.0 * n_pairs * H * 2 * F
    if name in ("mfma_down", "grouped_down"):
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
    if bias_kind == "zipf":
        k = np.arange(1, E + 1, dtype=np.float64)
        pmf = k ** -1.1
        pmf /= pmf.sum()
        bias = (0.17 * np.log(pmf[rng.permutation(E)])).astype(np.float32)
    else:
        bias = rng.uniform(-0.01, 0.01, E).astype(np.float32)
    return ctx.moe_create(router, qq_hip.TYPE_F32, bias, *tensors, H, F, E, K)


def cpu_baseline(seconds):
    """The reference's CPU path restated for Node 12 (oracle/moe_ref.js: same loop
    order and float64 arithmetic as src/tensor.js / src/lfm2-engine.js, checked bit
    for bit against the C oracle by the tests), timed on one host thread:
    tokens/sec through one MoE layer on a bounded sample of single-token calls.
    Without node, the C oracle is timed instead."""
    import shutil
    node = shutil.which("node")
    ncores = os.cpu_count() or 0
    if node:
        p = subprocess.run([node, os.path.join(ROOT, "oracle", "moe_ref.js"), "bench", str(seconds)],
                           capture_output=True, text=True, timeout=seconds * 4 + 120, check=True)
        r = json.loads(p.stdout.strip().splitlines()[-1])
        return {
            "value": round(r["tokens_per_s"], 3), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": "%d single-token MoE-layer calls (H=2048, F=1792, E=32, K=4, Q8_0 experts) in "
                      "%.1f s: the reference's JS CPU path restated for Node %s, 1 thread of %d "
                      "host cores; tokens are independent, so tokens/s is the rate at any batch"
                      % (r["tokens"], r["seconds"], r["node"], ncores),
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
    return {"value": round(n / el, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": "%d single-token MoE-layer calls in %.1f s on the C oracle (node absent), "
                      "1 thread of %d host cores" % (n, el, ncores)}


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


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="decode_b1")
    ap.add_argument("--layers", type=int, default=16, help="distinct layer instances rotated over")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
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

    T, bias_kind, wname = WORKLOADS[args.workload]
    torch.cuda.init()
    ctx = qq_hip.Context(0)
    # the library launches on this stream; every event below is recorded on it
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)

    n_layers = args.layers if T == 1 else min(args.layers, 4)
    layers = [make_layer(torch, ctx, 1000 + i, bias_kind) for i in range(n_layers)]
    S = 64 if T == 1 else 2
    gx = torch.Generator(device="cuda")
    gx.manual_seed(99)
    X = torch.randn((S, T, H), generator=gx, device="cuda", dtype=torch.float32)
    HID = torch.randn((S, T, H), generator=gx, device="cuda", dtype=torch.float32)
    idx = torch.empty((S, T, K), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()

    def step(i):
        s = i % S
        layers[i % n_layers].forward_dev(X[s].data_ptr(), HID[s].data_ptr(), T,
                                         idx_ptr=idx[s].data_ptr())

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ctx.synchronize()          # raises if a device-side wait expired
    total_ms = ev0.elapsed_time(ev1)
    ms_per_step = total_ms / args.steps

    # distinct experts per step (weights each step must read at least once)
    used = idx.cpu().numpy()
    n_exp = float(np.mean([len(np.unique(used[s])) for s in range(min(S, args.steps))]))
    n_pairs = T * K

    # per-kernel pass: same steps, every launch bracketed by its own events
    ctx.profile_enable(args.steps * 8)
    for i in range(args.steps):
        step(i)
    prof = ctx.profile_read()
    ctx.profile_enable(0)
    ctx.synchronize()
    kernels = {}
    for name, (ms, cnt) in prof.items():
        b = kernel_bytes(name, T, n_exp, n_pairs)
        avg_us = 1000.0 * ms / cnt
        fl = kernel_flops(name, n_pairs)
        kernels[name] = {"avg_us": round(avg_us, 3), "launches": cnt,
                         "bytes": None if b is None else int(b),
                         "gbps": None if b is None else round(b / (avg_us * 1e3), 1)}
        if fl is not None:
            kernels[name]["tflops"] = round(fl / (avg_us * 1e6), 1)
    dom = max(prof, key=lambda n: prof[n][0])
    dom_k = kernels[dom]

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_%s.json" % args.workload)
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get(dom)

    if dom in MFMA_KERNELS:
        roofline = {"kernel": dom, "bound": "mfma", "achieved": dom_k["tflops"],
                    "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(dom_k["tflops"] / MFMA_PEAK_TFLOPS, 4), "traffic": traffic}
    else:
        roofline = {"kernel": dom, "bound": "hbm", "achieved": dom_k["gbps"],
                    "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": None if dom_k["gbps"] is None else round(dom_k["gbps"] / HBM_PEAK_GBPS, 4),
                    "traffic": traffic}
    layer_flops = 6.0 * n_pairs * H * F
    lb = layer_bytes(T, n_exp)
    tokens_per_s = T * args.steps / (total_ms / 1000.0)
    result = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if dom in MFMA_KERNELS else "f32",
        "data": "synthetic",
        "config": {"workload": wname, "H": H, "F": F, "E": E, "K": K, "T": T,
                   "weights": "Q8_0", "activations": "f32", "router": "f32 (f64 accumulate)",
                   "layer_instances": n_layers, "distinct_experts_per_step": round(n_exp, 2)},
        "hbm_gbps_layer": round(lb / (ms_per_step * 1e6), 1),
        "hbm_frac_layer": round(lb / (ms_per_step * 1e6) / HBM_PEAK_GBPS, 4),
        "tflops_layer": round(layer_flops / (ms_per_step * 1e9), 2),
        "roofline": roofline,
        "kernels": kernels,
    }
    for l in layers:
        for t in l._keep:
            t.release()
        l.release()
    ctx.close()

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
