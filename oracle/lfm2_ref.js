'use strict';
// lfm2_ref.js -- Node 12 restatement of the reference's LFM2 single-token
// forward (Lfm2Engine.forward, src/lfm2-engine.js:228-280).
//
// TEST INFRASTRUCTURE ONLY: the checker of the device forward (tests/) and
// the CPU baseline of the whole-token bench leg.  Never loaded by the product.
//
// Same semantics and floating-point operation order as the reference
// (float64 arithmetic, fp32 stores wherever the reference stores into a
// Float32Array):
//   constructor / _loadWeights   src/lfm2-engine.js:15-144 (config keys, defaults,
//                                layer kinds, headDim / nKV / nFF derivation)
//   _dequantConvKernel           src/lfm2-engine.js:146-180
//   forward                      src/lfm2-engine.js:228-280
//   _shortConv                   src/lfm2-engine.js:282-327
//   _selfAttention               src/lfm2-engine.js:329-392 (GQA, KV cache)
//   _denseFfn                    src/lfm2-engine.js:394-403
//   _moEFFN                      src/lfm2-engine.js:413-487 (moe_ref.js)
//   embeddingLookupGeneric       src/tensor.js:499-523 (Q8_0 and F32 rows)
//   rmsnorm / perHeadRMSNorm     src/tensor.js:103-129
//   applyRoPE                    src/tensor.js:132-147 (split-half pairs)
//   KVCache store / getK / getV  src/kv-cache.js:1-50 ([layer][head][pos][dim])
//
// CLI: node lfm2_ref.js run <job.json>   (job written by tests/: the GGUF
//      file, its tensor table and config keys, the tokens; writes the logits
//      of every token, float32 little-endian)
//      node lfm2_ref.js bench <job.json> <seconds>

const fs = require('fs');
const M = require('./moe_ref.js');

const QK = 32;
const QBLOCK = 34;

function embedRow(meta, token) {
    const n = meta.shape[0];
    const out = new Float32Array(n);
    if (meta.type === 8) {
        const nb = Math.ceil(n / QK);
        const i8 = new Int8Array(meta.buffer), u8 = new Uint8Array(meta.buffer);
        const col = meta.offset + token * nb * QBLOCK;
        for (let b = 0; b < nb; b++) {
            const p = col + b * QBLOCK;
            const d = M.halfToNumber(u8[p] | (u8[p + 1] << 8));
            for (let i = 0; i < QK && b * QK + i < n; i++) out[b * QK + i] = i8[p + 2 + i] * d;
        }
        return out;
    }
    if (meta.type === 0) {
        const dv = new DataView(meta.buffer);
        for (let i = 0; i < n; i++) out[i] = dv.getFloat32(meta.offset + (token * n + i) * 4, true);
        return out;
    }
    throw new Error('Unsupported embedding type: ' + meta.type);
}

function rmsnormInPlace(x, wMeta, eps) {
    const n = x.length;
    let ss = 0;
    for (let i = 0; i < n; i++) ss += x[i] * x[i];
    const inv = 1.0 / Math.sqrt(ss / n + eps);
    const w = M.readWeightF32(wMeta, n);
    for (let i = 0; i < n; i++) x[i] = w[i] * x[i] * inv;
}

function headNormInPlace(x, nHeads, hd, wMeta, eps) {
    const w = M.readWeightF32(wMeta, hd);
    for (let h = 0; h < nHeads; h++) {
        let ss = 0;
        for (let d = 0; d < hd; d++) ss += x[h * hd + d] * x[h * hd + d];
        const inv = 1.0 / Math.sqrt(ss / hd + eps);
        for (let d = 0; d < hd; d++) x[h * hd + d] = w[d] * x[h * hd + d] * inv;
    }
}

function ropeInPlace(x, nHeads, hd, pos, base) {
    const half = hd >> 1;
    for (let h = 0; h < nHeads; h++) {
        for (let i = 0; i < half; i++) {
            const th = pos * (1.0 / Math.pow(base, i / half));
            const c = Math.cos(th), s = Math.sin(th);
            const a = x[h * hd + i], b = x[h * hd + i + half];
            x[h * hd + i] = a * c - b * s;
            x[h * hd + i + half] = a * s + b * c;
        }
    }
}

function convKernelF32(meta) {
    const L = meta.shape[0], D = meta.shape[1];
    if (meta.type === 0) return new Float32Array(meta.buffer, meta.offset, L * D);
    const out = new Float32Array(L * D);
    const u8 = new Uint8Array(meta.buffer);
    if (meta.type === 1) {
        for (let i = 0; i < L * D; i++) {
            const p = meta.offset + 2 * i;
            out[i] = M.halfToNumber(u8[p] | (u8[p + 1] << 8));
        }
        return out;
    }
    if (meta.type === 8) {
        const i8 = new Int8Array(meta.buffer);
        const per = Math.ceil(L / QK) * QBLOCK;
        for (let d = 0; d < D; d++) {
            const p = meta.offset + d * per;
            const sc = M.halfToNumber(u8[p] | (u8[p + 1] << 8));
            for (let k = 0; k < L; k++) out[d * L + k] = i8[p + 2 + k] * sc;
        }
        return out;
    }
    throw new Error('Unsupported conv kernel type: ' + meta.type);
}

// Config and weights as the reference's constructor derives them.
function buildModel(kv, metas) {
    const arch = kv['general.architecture'] || 'lfm2moe';
    const g = function (k) { return kv[arch + '.' + k]; };
    const m = {};
    m.nLayers = Number(g('block_count')) || 24;
    m.nEmb = Number(g('embedding_length')) || 2048;
    m.nHeads = Number(g('attention.head_count')) || 32;
    m.eps = Number(g('attention.layer_norm_rms_epsilon')) || 1e-5;
    m.nExperts = Number(g('expert_count')) || 32;
    m.nExpertsUsed = Number(g('expert_used_count')) || 4;
    m.nDenseLead = Number(g('leading_dense_block_count')) || 2;
    m.lCache = Number(g('shortconv.l_cache')) || 3;
    m.maxCtx = Math.min(Number(g('context_length')) || 4096, 4096);
    m.ropeBase = Number(g('rope.freq_base') || g('rope_freq_base')) || 5000000;
    const kvh = g('attention.head_count_kv');
    m.nHeadKV = Array.isArray(kvh) ? Math.max.apply(null, kvh.filter(function (v) { return v > 0; }))
                                   : (Number(kvh) || 8);
    const t = function (name) { return metas[name] || null; };
    m.tokEmbd = t('token_embd.weight');
    m.outputNorm = t('token_embd_norm.weight');
    m.output = t('output.weight') || m.tokEmbd;
    m.layers = [];
    let ci = 0;
    for (let i = 0; i < m.nLayers; i++) {
        const p = 'blk.' + i + '.';
        const conv = t(p + 'shortconv.conv.weight');
        const L = { rec: conv !== null, moe: i >= m.nDenseLead, attnNorm: t(p + 'attn_norm.weight'),
                    ffnNorm: t(p + 'ffn_norm.weight'), cacheIdx: -1 };
        if (L.rec) {
            L.inProj = t(p + 'shortconv.in_proj.weight');
            L.outProj = t(p + 'shortconv.out_proj.weight');
            L.kern = convKernelF32(conv);
        } else {
            L.cacheIdx = ci++;
            L.wq = t(p + 'attn_q.weight'); L.wk = t(p + 'attn_k.weight');
            L.wv = t(p + 'attn_v.weight'); L.wo = t(p + 'attn_output.weight');
            L.qNorm = t(p + 'attn_q_norm.weight'); L.kNorm = t(p + 'attn_k_norm.weight');
        }
        if (L.moe) {
            L.routerWeight = t(p + 'ffn_gate_inp.weight');
            L.ffnGateExps = t(p + 'ffn_gate_exps.weight');
            L.ffnUpExps = t(p + 'ffn_up_exps.weight');
            L.ffnDownExps = t(p + 'ffn_down_exps.weight');
            L.expProbsBias = t(p + 'exp_probs_b.bias');
        } else {
            L.gate = t(p + 'ffn_gate.weight'); L.up = t(p + 'ffn_up.weight'); L.down = t(p + 'ffn_down.weight');
        }
        m.layers.push(L);
    }
    m.nVocab = m.tokEmbd.shape[1];
    const a = m.layers.find(function (L) { return !L.rec; });
    m.headDim = a ? Math.floor(a.wq.shape[1] / m.nHeads) : 64;
    m.nKV = a ? a.wk.shape[1] : m.nHeadKV * m.headDim;
    m.nAttn = ci;
    const H = m.nEmb;
    m.hidden = new Float32Array(H);
    m.normed = new Float32Array(H);
    m.moeOut = new Float32Array(H);
    m.kCache = new Float32Array(ci * m.nHeadKV * m.maxCtx * m.headDim);
    m.vCache = new Float32Array(ci * m.nHeadKV * m.maxCtx * m.headDim);
    m.convState = m.layers.map(function (L) { return L.rec ? new Float32Array((m.lCache - 1) * H) : null; });
    m.routes = null;       // selected experts of every MoE block, when an array
    m.payloads = null;     // the whole onRouterUpdate payload of every MoE block, when an array
    m.expertMask = null;   // Set of experts skipped in every MoE block (src/lfm2-engine.js:464)
    return m;
}

function shortConv(m, li, L) {
    const H = m.nEmb, K = m.lCache;
    const bcx = M.matmulGeneric(L.inProj, m.normed);
    const bx = new Float32Array(H), y = new Float32Array(H), co = new Float32Array(H);
    for (let d = 0; d < H; d++) bx[d] = bcx[d] * bcx[2 * H + d];
    const st = m.convState[li];
    for (let d = 0; d < H; d++)
        co[d] = L.kern[d * K] * st[d] + L.kern[d * K + 1] * st[H + d] + L.kern[d * K + 2] * bx[d];
    st.copyWithin(0, H, 2 * H);
    st.set(bx, H);
    for (let d = 0; d < H; d++) y[d] = bcx[H + d] * co[d];
    return M.matmulGeneric(L.outProj, y);
}

function attention(m, L, pos) {
    const hd = m.headDim, nH = m.nHeads, nKVH = m.nHeadKV, C = m.maxCtx;
    const q = M.matmulGeneric(L.wq, m.normed);
    const k = M.matmulGeneric(L.wk, m.normed);
    const v = M.matmulGeneric(L.wv, m.normed);
    headNormInPlace(q, nH, hd, L.qNorm, m.eps);
    headNormInPlace(k, nKVH, hd, L.kNorm, m.eps);
    ropeInPlace(q, nH, hd, pos, m.ropeBase);
    ropeInPlace(k, nKVH, hd, pos, m.ropeBase);
    const lay = L.cacheIdx * nKVH * C * hd;
    for (let h = 0; h < nKVH; h++)
        for (let d = 0; d < hd; d++) {
            m.kCache[lay + (h * C + pos) * hd + d] = k[h * hd + d];
            m.vCache[lay + (h * C + pos) * hd + d] = v[h * hd + d];
        }
    const n = pos + 1;
    const scale = 1.0 / Math.sqrt(hd);
    const sc = new Float32Array(nH * n);
    const out = new Float32Array(nH * hd);
    for (let h = 0; h < nH; h++) {
        const g = (h * nKVH / nH) | 0;
        for (let p = 0; p < n; p++) {
            let dot = 0;
            for (let d = 0; d < hd; d++) dot += q[h * hd + d] * m.kCache[lay + (g * C + p) * hd + d];
            sc[h * n + p] = dot * scale;
        }
        M.softmaxF32(sc, h * n, (h + 1) * n);
        for (let p = 0; p < n; p++) {
            const w = sc[h * n + p];
            if (w === 0) continue;
            for (let d = 0; d < hd; d++) out[h * hd + d] += m.vCache[lay + (g * C + p) * hd + d] * w;
        }
    }
    return M.matmulGeneric(L.wo, out);
}

function denseFfn(m, L) {
    const g = M.matmulGeneric(L.gate, m.normed);
    M.siluInPlace(g);
    const u = M.matmulGeneric(L.up, m.normed);
    M.mulInPlace(g, u);
    M.addVec(m.hidden, M.matmulGeneric(L.down, g));
}

// tm (optional): { block(li, ms), head(ms) } receives the time of every block
// and of the output head.
function forward(m, token, pos, skipLogits, tm) {
    const now = function () { return Number(process.hrtime.bigint()) / 1e6; };
    m.hidden.set(embedRow(m.tokEmbd, token));
    for (let li = 0; li < m.nLayers; li++) {
        const ta = tm ? now() : 0;
        const L = m.layers[li];
        m.normed.set(m.hidden);
        rmsnormInPlace(m.normed, L.attnNorm, m.eps);
        M.addVec(m.hidden, L.rec ? shortConv(m, li, L) : attention(m, L, pos));
        m.normed.set(m.hidden);
        rmsnormInPlace(m.normed, L.ffnNorm, m.eps);
        if (!L.moe) {
            denseFfn(m, L);
        } else {
            const rec = m.routes || m.payloads;
            const eng = { nExperts: m.nExperts, nExpertsUsed: m.nExpertsUsed, bufNormed: m.normed,
                          bufHidden: m.hidden, bufMoEOut: m.moeOut, expertMask: m.expertMask,
                          onRouterUpdate: rec ? function (r) {
                              if (m.routes) m.routes.push(r.selected);
                              if (m.payloads) m.payloads.push(r);
                          } : null };
            M.moEFFN(eng, li, L);
        }
        if (tm) tm.block(li, now() - ta);
    }
    if (skipLogits) return null;
    const th = tm ? now() : 0;
    rmsnormInPlace(m.hidden, m.outputNorm, m.eps);
    const out = M.matmulGeneric(m.output, m.hidden);
    if (tm) tm.head(now() - th);
    return out;
}

function loadJob(path) {
    const job = JSON.parse(fs.readFileSync(path, 'utf8'));
    const b = fs.readFileSync(job.gguf);
    const buf = b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength);
    const metas = {};
    for (const name of Object.keys(job.tensors)) {
        const t = job.tensors[name];
        metas[name] = { buffer: buf, offset: t.offset, shape: t.shape, type: t.type };
    }
    return { job: job, model: buildModel(job.kv, metas) };
}

function run(path) {
    const o = loadJob(path), job = o.job, m = o.model;
    m.routes = [];
    if (job.out_payloads) m.payloads = [];
    if (job.mask) m.expertMask = new Set(job.mask);
    const V = m.nVocab, T = job.tokens.length;
    const logits = new Float32Array(T * V);
    for (let t = 0; t < T; t++) logits.set(forward(m, job.tokens[t], job.start + t, false), t * V);
    fs.writeFileSync(job.out_logits, Buffer.from(logits.buffer));
    fs.writeFileSync(job.out_routes, JSON.stringify(m.routes));
    if (job.out_payloads) fs.writeFileSync(job.out_payloads, JSON.stringify(m.payloads));
}

// Times tokens through the model, per block and for the output head, so a
// model of a few full-width blocks can stand for a deeper one.
function bench(path, seconds) {
    const m = loadJob(path).model;
    const blockMs = new Array(m.nLayers).fill(0);
    let headMs = 0, n = 0;
    const tm = { block: function (li, ms) { blockMs[li] += ms; }, head: function (ms) { headMs += ms; } };
    const t0 = process.hrtime.bigint();
    let el = 0;
    while (el < seconds || n < 1) {
        forward(m, (n * 7919) % m.nVocab, n % m.maxCtx, false, tm);
        n++;
        el = Number(process.hrtime.bigint() - t0) / 1e9;
    }
    process.stdout.write(JSON.stringify({
        tokens: n, seconds: el, tokens_per_s: n / el, threads: 1, node: process.version,
        blocks: m.layers.map(function (L, i) {
            return { kind: (L.rec ? 'conv' : 'attn') + '+' + (L.moe ? 'moe' : 'dense'), ms: blockMs[i] / n };
        }),
        head_ms: headMs / n }) + '\n');
}

module.exports = { buildModel, forward, embedRow, rmsnormInPlace, headNormInPlace, ropeInPlace,
                   convKernelF32, shortConv, attention };

if (require.main === module) {
    const cmd = process.argv[2];
    if (cmd === 'run') run(process.argv[3]);
    else if (cmd === 'bench') bench(process.argv[3], Number(process.argv[4] || 10));
    else {
        process.stderr.write('usage: node lfm2_ref.js run <job.json> | bench <job.json> <seconds>\n');
        process.exit(2);
    }
}
