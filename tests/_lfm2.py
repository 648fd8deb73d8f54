"""Helpers of the LFM2 whole-token tests: a synthetic model file, the Node
restatement of the reference's forward (oracle/lfm2_ref.js) run as a job, and
an independent float64 forward (numpy, no fp32 rounding) that pins it."""
import json
import os
import shutil
import subprocess

import numpy as np

import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def node():
    return shutil.which("node")


def kv_dict(cfg, arch="lfm2moe"):
    p = arch + "."
    return {"general.architecture": arch, p + "block_count": cfg["n_layers"],
            p + "embedding_length": cfg["H"], p + "attention.head_count": cfg["n_heads"],
            p + "attention.head_count_kv": [cfg["n_head_kv"] if i in cfg["attn_layers"] else 0
                                            for i in range(cfg["n_layers"])],
            p + "attention.layer_norm_rms_epsilon": float(np.float32(cfg["eps"])),
            p + "expert_count": cfg["E"], p + "expert_used_count": cfg["K"],
            p + "expert_feed_forward_length": cfg["F"],
            p + "leading_dense_block_count": cfg["n_dense"],
            p + "shortconv.l_cache": cfg["l_cache"], p + "context_length": cfg["ctx"],
            p + "rope.freq_base": float(np.float32(cfg["rope_base"]))}


def write_model(tmp, seed, cfg, **kw):
    """Writes the GGUF file; returns (path, offsets, tensors)."""
    data, offs, tensors = synth.lfm2_gguf(seed, cfg, **kw)
    path = os.path.join(str(tmp), "lfm2_%d.gguf" % seed)
    with open(path, "wb") as f:
        f.write(data)
    return path, offs, tensors


def js_forward(tmp, path, offs, tensors, cfg, tokens, start=0, mask=None, payloads=False):
    """Logits [T, vocab] and per-MoE-layer routes of lfm2_ref.js (with the
    experts in `mask` skipped); with payloads=True also the onRouterUpdate
    payload of every MoE block ({layer, probs, selected, weights}, T x blocks)."""
    job = {"gguf": path, "kv": kv_dict(cfg), "tokens": [int(t) for t in tokens], "start": start,
           "tensors": {n: {"offset": offs[n], "shape": s, "type": t} for n, s, t, _ in tensors},
           "out_logits": os.path.join(str(tmp), "logits.f32"),
           "out_routes": os.path.join(str(tmp), "routes.json")}
    if mask is not None:
        job["mask"] = sorted(int(e) for e in mask)
    if payloads:
        job["out_payloads"] = os.path.join(str(tmp), "payloads.json")
    jp = os.path.join(str(tmp), "lfm2_job.json")
    with open(jp, "w") as f:
        json.dump(job, f)
    subprocess.run([node(), os.path.join(ROOT, "oracle", "lfm2_ref.js"), "run", jp], check=True,
                   timeout=600)
    logits = np.fromfile(job["out_logits"], np.float32).reshape(len(tokens), -1)
    with open(job["out_routes"]) as f:
        routes = json.load(f)
    if not payloads:
        return logits, routes
    with open(job["out_payloads"]) as f:
        return logits, routes, json.load(f)


# ---------------------------------------------------------------- float64 forward

def _dense(tensors):
    """name -> float64 array: Q8_0 matrices [out, in]; F32/F16 as stored."""
    out = {}
    for name, shape, typ, data in tensors:
        if typ == synth.TYPE_Q8_0:
            n = shape[2] if len(shape) > 2 else 1
            w = synth.q8_0_dequant(data, shape[0], shape[1], n)
            out[name] = w if len(shape) > 2 else w[0]
        elif typ == synth.TYPE_F16:
            out[name] = np.asarray(data, np.float16).astype(np.float64)
        else:
            out[name] = np.asarray(data, np.float32).astype(np.float64)
    return out


class F64Model:
    """The LFM2 forward of the reference (src/lfm2-engine.js:228-487) in float64
    without intermediate fp32 rounding: the pin of lfm2_ref.js."""

    def __init__(self, tensors, cfg):
        self.W = _dense(tensors)
        self.c = cfg
        C, hd, nkv = cfg["ctx"], cfg["head_dim"], cfg["n_head_kv"]
        self.kc = {i: np.zeros((nkv, C, hd)) for i in cfg["attn_layers"]}
        self.vc = {i: np.zeros((nkv, C, hd)) for i in cfg["attn_layers"]}
        self.st = {i: np.zeros((cfg["l_cache"] - 1, cfg["H"])) for i in range(cfg["n_layers"])
                   if i not in cfg["attn_layers"]}
        self.routes = []

    def _norm(self, x, w):
        return w * x / np.sqrt(np.mean(x * x) + self.c["eps"])

    def _rope(self, x, pos):
        hd = x.shape[-1]
        half = hd // 2
        th = pos / self.c["rope_base"] ** (np.arange(half) / half)
        a, b = x[..., :half].copy(), x[..., half:].copy()
        return np.concatenate([a * np.cos(th) - b * np.sin(th), a * np.sin(th) + b * np.cos(th)], -1)

    def forward(self, token, pos):
        c, W = self.c, self.W
        H, hd, L = c["H"], c["head_dim"], c["l_cache"]
        h = W["token_embd.weight"][token].copy()
        for i in range(c["n_layers"]):
            p = "blk.%d." % i
            x = self._norm(h, W[p + "attn_norm.weight"])
            if i in c["attn_layers"]:
                q = (W[p + "attn_q.weight"] @ x).reshape(c["n_heads"], hd)
                k = (W[p + "attn_k.weight"] @ x).reshape(c["n_head_kv"], hd)
                v = (W[p + "attn_v.weight"] @ x).reshape(c["n_head_kv"], hd)
                q = np.stack([self._norm(r, W[p + "attn_q_norm.weight"]) for r in q])
                k = np.stack([self._norm(r, W[p + "attn_k_norm.weight"]) for r in k])
                q, k = self._rope(q, pos), self._rope(k, pos)
                self.kc[i][:, pos], self.vc[i][:, pos] = k, v
                grp = c["n_heads"] // c["n_head_kv"]
                o = np.zeros((c["n_heads"], hd))
                for hh in range(c["n_heads"]):
                    g = hh // grp
                    s = self.kc[i][g, :pos + 1] @ q[hh] / np.sqrt(hd)
                    e = np.exp(s - s.max())
                    o[hh] = (e / e.sum()) @ self.vc[i][g, :pos + 1]
                h = h + W[p + "attn_output.weight"] @ o.ravel()
            else:
                bcx = W[p + "shortconv.in_proj.weight"] @ x
                B, Cg, xx = bcx[:H], bcx[H:2 * H], bcx[2 * H:]
                bx = B * xx
                kern = W[p + "shortconv.conv.weight"]
                kern = (kern.reshape(H, L) if kern.ndim == 1 else kern.reshape(H, -1)[:, :L])
                win = np.vstack([self.st[i], bx])            # [L, H], oldest first
                co = (kern.T * win).sum(0)
                self.st[i] = win[1:]
                h = h + W[p + "shortconv.out_proj.weight"] @ (Cg * co)
            x = self._norm(h, W[p + "ffn_norm.weight"])
            if i < c["n_dense"]:
                g = W[p + "ffn_gate.weight"] @ x
                u = W[p + "ffn_up.weight"] @ x
                h = h + W[p + "ffn_down.weight"] @ (g / (1 + np.exp(-g)) * u)
            else:
                lg = W[p + "ffn_gate_inp.weight"].reshape(c["E"], H) @ x
                pr = 1 / (1 + np.exp(-lg))
                sc = pr + W.get(p + "exp_probs_b.bias", 0.0)
                sel = np.argsort(-sc, kind="stable")[:c["K"]]
                self.routes.append(sel.tolist())
                wts = pr[sel] / (pr[sel].sum() + 1e-6)
                for e, wk in zip(sel, wts):
                    g = W[p + "ffn_gate_exps.weight"][e] @ x
                    u = W[p + "ffn_up_exps.weight"][e] @ x
                    h = h + wk * (W[p + "ffn_down_exps.weight"][e] @ (g / (1 + np.exp(-g)) * u))
        hn = self._norm(h, W["token_embd_norm.weight"])
        out = W["output.weight"] if "output.weight" in W else W["token_embd.weight"]
        return out @ hn
