'use strict';
// moe_ref.js -- Node 12 restatement of the reference's CPU MoE path.
//
// TEST INFRASTRUCTURE ONLY: the CPU baseline that bench.py times and a second
// checker (compared bit for bit with oracle/qq_oracle.c by the tests).  It is
// never loaded by the product path.
//
// Same semantics and floating-point operation order as the reference:
//   matmulQ80xF32   src/tensor.js:26-53   (dot += x * q * d, float64, one fp32 store)
//   matmulF32xF32   src/tensor.js:469-482
//   matmulGeneric   src/tensor.js:485-496
//   _readWeightF32  src/tensor.js:80-100
//   siluInPlace / mulInPlace / addVec   src/tensor.js:167-185
//   _expertSlice    src/lfm2-engine.js:489-505
//   _moEFFN         src/lfm2-engine.js:413-487 (sigmoid + expert bias gating)
//   softmaxF32      src/tensor.js:150-164 (softmaxInPlace)
//   Qwen3 _moEFFN   src/qwen3-engine.js:304-363 (softmax gating, no bias)
// Node 12 has no DataView.getFloat16, so binary16 is decoded in closed form.
//
// CLI:
//   node moe_ref.js run <job.json>     run a job written by tests/ (inputs and
//                                      outputs are raw little-endian files)
//   node moe_ref.js bench <seconds>    time single-token MoE-layer calls on a
//                                      seeded LFM2-8B-A1B-shaped layer; prints JSON
//   node moe_ref.js bench-matvec <s>   time matmulQ80xF32 on a 1024 -> 3072 weight
//   node moe_ref.js bench-job <job.json> <runs> <s>
//                                      time single-token calls of a job's layer
//                                      (or matvec) over its input rows: the rate
//                                      of each of <runs> runs of <s> seconds and
//                                      their median (the CPU baseline)

const fs = require('fs');

const QK = 32;
const QBLOCK = 34;

function halfToNumber(bits) {
    const sign = (bits & 0x8000) ? -1 : 1;
    const exp = (bits >>> 10) & 0x1f;
    const man = bits & 0x3ff;
    if (exp === 0) return sign * man * Math.pow(2, -24);
    if (exp === 31) return man ? NaN : sign * Infinity;
    return sign * (1024 + man) * Math.pow(2, exp - 25);
}

// Typed-array views cached on the meta, as the reference does.
function viewsOf(meta) {
    if (!meta._qqI8) {
        meta._qqI8 = new Int8Array(meta.buffer);
        meta._qqU8 = new Uint8Array(meta.buffer);
    }
    return meta;
}

function scaleAt(u8, off) {
    return halfToNumber(u8[off] | (u8[off + 1] << 8));
}

function matmulQ80xF32(meta, input) {
    const inDim = meta.shape[0];
    const outDim = meta.shape[1];
    const nb = Math.ceil(inDim / QK);
    const m = viewsOf(meta);
    const i8 = m._qqI8, u8 = m._qqU8;
    const out = new Float32Array(outDim);
    for (let c = 0; c < outDim; c++) {
        let acc = 0;
        let p = meta.offset + c * nb * QBLOCK;
        for (let b = 0; b < nb; b++, p += QBLOCK) {
            const d = scaleAt(u8, p);
            const base = b * QK;
            const lim = Math.min(QK, inDim - base);
            for (let i = 0; i < lim; i++) acc += input[base + i] * i8[p + 2 + i] * d;
        }
        out[c] = acc;
    }
    return out;
}

function matmulF32xF32(meta, input) {
    const inDim = meta.shape[0];
    const outDim = meta.shape[1];
    const dv = new DataView(meta.buffer);
    const out = new Float32Array(outDim);
    for (let c = 0; c < outDim; c++) {
        let acc = 0;
        const base = meta.offset + c * inDim * 4;
        for (let i = 0; i < inDim; i++) acc += input[i] * dv.getFloat32(base + 4 * i, true);
        out[c] = acc;
    }
    return out;
}

function matmulGeneric(meta, input) {
    if (meta.type === 8) return matmulQ80xF32(meta, input);
    if (meta.type === 0) return matmulF32xF32(meta, input);
    throw new Error('Unsupported tensor type for matmul: ' + meta.type);
}

function readWeightF32(meta, n) {
    if (meta.type === 0) return new Float32Array(meta.buffer, meta.offset, n);
    if (meta.type === 8) {
        const m = viewsOf(meta);
        const out = new Float32Array(n);
        for (let b = 0; b < Math.ceil(n / QK); b++) {
            const p = meta.offset + b * QBLOCK;
            const d = scaleAt(m._qqU8, p);
            for (let i = 0; i < QK && b * QK + i < n; i++) out[b * QK + i] = m._qqI8[p + 2 + i] * d;
        }
        return out;
    }
    throw new Error('Unsupported weight type for norm: ' + meta.type);
}

function siluInPlace(a) {
    for (let i = 0; i < a.length; i++) a[i] *= 1.0 / (1.0 + Math.exp(-a[i]));
}

function mulInPlace(a, b) {
    for (let i = 0; i < a.length; i++) a[i] *= b[i];
}

function addVec(a, b) {
    for (let i = 0; i < a.length; i++) a[i] += b[i];
}

function expertSlice(meta, e) {
    const inDim = meta.shape[0], hidDim = meta.shape[1];
    const colBytes = Math.ceil(inDim / QK) * QBLOCK;
    return { buffer: meta.buffer, offset: meta.offset + e * hidDim * colBytes,
             nbytes: hidDim * colBytes, shape: [inDim, hidDim], type: meta.type };
}

// One token through one MoE layer.  `eng` carries bufNormed, bufHidden,
// bufMoEOut, nExperts, nExpertsUsed, onRouterUpdate, expertMask.
function moEFFN(eng, layerIdx, layer) {
    const E = eng.nExperts, K = eng.nExpertsUsed;
    const logits = matmulGeneric(layer.routerWeight, eng.bufNormed);
    const probs = new Float32Array(E);
    for (let e = 0; e < E; e++) probs[e] = 1.0 / (1.0 + Math.exp(-logits[e]));
    const score = new Float32Array(probs);
    if (layer.expProbsBias) {
        const bias = readWeightF32(layer.expProbsBias, E);
        for (let e = 0; e < E; e++) score[e] += bias[e];
    }
    const order = Array.from(score).map(function (v, i) { return [v, i]; });
    order.sort(function (a, b) { return b[0] - a[0]; });
    const chosen = [], chosenP = [];
    for (let k = 0; k < K; k++) {
        chosen.push(order[k][1]);
        chosenP.push(probs[order[k][1]]);
    }
    let sum = 1e-6;
    for (let k = 0; k < K; k++) sum += chosenP[k];
    const inv = 1.0 / sum;
    if (eng.onRouterUpdate) {
        eng.onRouterUpdate({ layer: layerIdx, probs: Array.from(probs), selected: chosen,
                             weights: chosenP.map(function (p) { return p * inv; }) });
    }
    eng.bufMoEOut.fill(0);
    for (let k = 0; k < K; k++) {
        const e = chosen[k];
        if (eng.expertMask && eng.expertMask.has(e)) continue;
        const wk = chosenP[k] * inv;
        const g = matmulGeneric(expertSlice(layer.ffnGateExps, e), eng.bufNormed);
        siluInPlace(g);
        const u = matmulGeneric(expertSlice(layer.ffnUpExps, e), eng.bufNormed);
        mulInPlace(g, u);
        const y = matmulGeneric(expertSlice(layer.ffnDownExps, e), g);
        for (let i = 0; i < y.length; i++) eng.bufMoEOut[i] += wk * y[i];
    }
    addVec(eng.bufHidden, eng.bufMoEOut);
}

// Normalised exponentials of the fp32 row[lo, hi), in place, with the float
// operations of src/tensor.js:150-164 in the same order: the shift is the
// first largest entry (a strict compare); each exponential is taken in
// binary64 of (entry - shift), stored back to fp32, and the stored values
// are summed in binary64 in index order; one binary64 reciprocal of the
// sum; every entry times it, stored to fp32.
function softmaxF32(row, lo, hi) {
    let peak = row[lo];
    for (let j = lo + 1; j < hi; j++) peak = row[j] > peak ? row[j] : peak;
    let total = 0;
    for (let j = lo; j < hi; j++) {
        row[j] = Math.exp(row[j] - peak);   // the store rounds to fp32 ...
        total += row[j];                    // ... and the sum takes the stored value
    }
    const scale = 1.0 / total;
    for (let j = lo; j < hi; j++) row[j] = row[j] * scale;
}

// The Qwen3-MoE block: softmax over the router logits, top-K by probability,
// weights renormalised from 0 (no 1e-6, no bias).  Top-K comes from the layer
// (src/qwen3-engine.js:73, 310), not the engine.
function moEFFNSoftmax(eng, layerIdx, layer) {
    const K = layer.nExpertsUsed;
    const probs = matmulGeneric(layer.routerWeight, eng.bufNormed);
    softmaxF32(probs, 0, probs.length);
    const order = Array.from(probs).map(function (v, i) { return [v, i]; });
    order.sort(function (a, b) { return b[0] - a[0]; });
    const chosen = [], chosenP = [];
    for (let k = 0; k < K; k++) {
        chosen.push(order[k][1]);
        chosenP.push(order[k][0]);
    }
    let sum = 0;
    for (let k = 0; k < K; k++) sum += chosenP[k];
    const inv = sum > 0 ? 1 / sum : 0;
    if (eng.onRouterUpdate) {
        eng.onRouterUpdate({ layer: layerIdx, probs: Array.from(probs), selected: chosen,
                             weights: chosenP.map(function (p) { return p * inv; }) });
    }
    eng.bufMoEOut.fill(0);
    for (let k = 0; k < K; k++) {
        const e = chosen[k];
        if (eng.expertMask && eng.expertMask.has(e)) continue;
        const wk = chosenP[k] * inv;
        const g = matmulGeneric(expertSlice(layer.ffnGateExps, e), eng.bufNormed);
        siluInPlace(g);
        const u = matmulGeneric(expertSlice(layer.ffnUpExps, e), eng.bufNormed);
        mulInPlace(g, u);
        const y = matmulGeneric(expertSlice(layer.ffnDownExps, e), g);
        for (let i = 0; i < y.length; i++) eng.bufMoEOut[i] += wk * y[i];
    }
    addVec(eng.bufHidden, eng.bufMoEOut);
}

// ---------------------------------------------------------------- CLI helpers

function readRaw(path) {
    const b = fs.readFileSync(path);
    return b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength);
}

function writeRaw(path, typed) {
    fs.writeFileSync(path, Buffer.from(typed.buffer, typed.byteOffset, typed.byteLength));
}

function runJob(jobPath) {
    const job = JSON.parse(fs.readFileSync(jobPath, 'utf8'));
    if (job.kind === 'matvec') {
        const meta = { buffer: readRaw(job.weight), offset: job.offset || 0,
                       shape: [job.in_dim, job.out_dim], type: job.type };
        const x = new Float32Array(readRaw(job.x));
        writeRaw(job.y, matmulGeneric(meta, x));
        return;
    }
    // kind === 'moe'
    const H = job.H, F = job.F, E = job.E, K = job.K, T = job.T;
    const tensor = function (path, shape, type) {
        return { buffer: readRaw(path), offset: 0, shape: shape, type: type };
    };
    const layer = {
        routerWeight: tensor(job.router, [H, E], job.router_type),
        expProbsBias: job.bias ? tensor(job.bias, [E], 0) : null,
        ffnGateExps: tensor(job.gate, [H, F, E], 8),
        ffnUpExps: tensor(job.up, [H, F, E], 8),
        ffnDownExps: tensor(job.down, [F, H, E], 8),
        nExpertsUsed: K,
    };
    const X = new Float32Array(readRaw(job.x));
    const hid = new Float32Array(readRaw(job.hidden));
    const idx = new Int32Array(T * K), w = new Float64Array(T * K), probs = new Float32Array(T * E);
    const eng = { nExperts: E, nExpertsUsed: K, bufNormed: new Float32Array(H),
                  bufHidden: new Float32Array(H), bufMoEOut: new Float32Array(H),
                  expertMask: job.mask ? new Set(job.mask) : null, onRouterUpdate: null };
    for (let t = 0; t < T; t++) {
        eng.bufNormed.set(X.subarray(t * H, (t + 1) * H));
        eng.bufHidden.set(hid.subarray(t * H, (t + 1) * H));
        eng.onRouterUpdate = function (info) {
            for (let k = 0; k < K; k++) { idx[t * K + k] = info.selected[k]; w[t * K + k] = info.weights[k]; }
            for (let e = 0; e < E; e++) probs[t * E + e] = info.probs[e];
        };
        if (job.gating === 'softmax') moEFFNSoftmax(eng, job.layer || 0, layer);
        else moEFFN(eng, job.layer || 0, layer);
        hid.set(eng.bufHidden, t * H);
    }
    writeRaw(job.out_hidden, hid);
    writeRaw(job.out_idx, idx);
    writeRaw(job.out_w, w);
    writeRaw(job.out_probs, probs);
}

// xorshift32 (seeded, deterministic); quality is irrelevant for timing
function rng(seed) {
    let s = seed >>> 0 || 1;
    return function () {
        s ^= s << 13; s >>>= 0;
        s ^= s >>> 17;
        s ^= s << 5; s >>>= 0;
        return s;
    };
}

function q8Tensor(next, inDim, outDim, nMats) {
    const nb = Math.ceil(inDim / QK);
    const nBlocks = nMats * outDim * nb;
    const u8 = new Uint8Array(nBlocks * QBLOCK);
    const halfOf = [0x1c19, 0x1e69, 0x1a3d, 0x2041];  // fp16 scales near 0.001..0.005
    for (let i = 0; i < nBlocks; i++) {
        const p = i * QBLOCK;
        const h = halfOf[next() & 3];
        u8[p] = h & 0xff;
        u8[p + 1] = h >> 8;
        for (let j = 0; j < QK; j += 4) {
            const r = next();
            u8[p + 2 + j] = r & 0xff; u8[p + 3 + j] = (r >> 8) & 0xff;
            u8[p + 4 + j] = (r >> 16) & 0xff; u8[p + 5 + j] = (r >>> 24) & 0xff;
        }
    }
    return u8.buffer;
}

function bench(seconds, qwen3) {
    // LFM2-8B-A1B MoE layer shape, or (qwen3) the Qwen3-30B-A3B one with softmax routing
    const H = 2048, F = qwen3 ? 768 : 1792, E = qwen3 ? 128 : 32, K = qwen3 ? 8 : 4;
    const next = rng(12345);
    const router = new Float32Array(E * H);
    for (let i = 0; i < router.length; i++) router[i] = ((next() & 0xffff) / 65536 - 0.5) * 0.04;
    const bias = new Float32Array(E);
    for (let e = 0; e < E; e++) bias[e] = ((next() & 0xffff) / 65536 - 0.5) * 0.02;
    const layer = {
        routerWeight: { buffer: router.buffer, offset: 0, shape: [H, E], type: 0 },
        expProbsBias: { buffer: bias.buffer, offset: 0, shape: [E], type: 0 },
        ffnGateExps: { buffer: q8Tensor(next, H, F, E), offset: 0, shape: [H, F, E], type: 8 },
        ffnUpExps: { buffer: q8Tensor(next, H, F, E), offset: 0, shape: [H, F, E], type: 8 },
        ffnDownExps: { buffer: q8Tensor(next, F, H, E), offset: 0, shape: [F, H, E], type: 8 },
        nExpertsUsed: K,
    };
    if (qwen3) layer.expProbsBias = null;
    const eng = { nExperts: E, nExpertsUsed: K, bufNormed: new Float32Array(H),
                  bufHidden: new Float32Array(H), bufMoEOut: new Float32Array(H),
                  expertMask: null, onRouterUpdate: null };
    const token = function () {
        for (let i = 0; i < H; i++) eng.bufNormed[i] = ((next() & 0xffff) / 65536 - 0.5) * 3.4;
        if (qwen3) moEFFNSoftmax(eng, 0, layer);
        else moEFFN(eng, 0, layer);
    };
    token();   // warm-up (JIT)
    let n = 0;
    const t0 = process.hrtime.bigint();
    let el = 0;
    while (el < seconds) {
        token();
        n++;
        el = Number(process.hrtime.bigint() - t0) / 1e9;
    }
    process.stdout.write(JSON.stringify({ tokens: n, seconds: el, tokens_per_s: n / el,
                                          threads: 1, node: process.version }) + '\n');
}

// matmulQ80xF32 on a 1024 -> 3072 Q8_0 weight (the Qwen3-0.6B FFN up-proj
// shape), one thread: matvecs per second.
function benchMatvec(seconds) {
    const IN = 1024, OUT = 3072;
    const next = rng(777);
    const meta = { buffer: q8Tensor(next, IN, OUT, 1), offset: 0, shape: [IN, OUT], type: 8 };
    const x = new Float32Array(IN);
    for (let i = 0; i < IN; i++) x[i] = ((next() & 0xffff) / 65536 - 0.5) * 3.4;
    matmulQ80xF32(meta, x);   // warm-up (JIT)
    let n = 0;
    const t0 = process.hrtime.bigint();
    let el = 0;
    while (el < seconds) {
        x[n & 1023] += 1e-3;
        matmulQ80xF32(meta, x);
        n++;
        el = Number(process.hrtime.bigint() - t0) / 1e9;
    }
    process.stdout.write(JSON.stringify({ matvecs: n, seconds: el, matvecs_per_s: n / el,
                                          threads: 1, node: process.version }) + '\n');
}

// The CPU baseline: single-token calls of a job's layer (or matvec) over its
// input rows, in `runs` runs of `seconds` each after a warm-up call; prints
// the rate of every run and their median.  Tokens are independent in the
// reference (src/lfm2-engine.js:550-555), so the per-token rate is the rate
// at any batch.
function benchJob(jobPath, runs, seconds) {
    const job = JSON.parse(fs.readFileSync(jobPath, 'utf8'));
    let step;
    if (job.kind === 'matvec') {
        const meta = { buffer: readRaw(job.weight), offset: 0, shape: [job.in_dim, job.out_dim], type: 8 };
        const X = new Float32Array(readRaw(job.x));
        const n = X.length / job.in_dim;
        step = function (i) {
            const r = i % n;
            matmulQ80xF32(meta, X.subarray(r * job.in_dim, (r + 1) * job.in_dim));
        };
    } else {
        const H = job.H, F = job.F, E = job.E, K = job.K;
        const tensor = function (path, shape, type) {
            return { buffer: readRaw(path), offset: 0, shape: shape, type: type };
        };
        const layer = {
            routerWeight: tensor(job.router, [H, E], job.router_type),
            expProbsBias: job.bias ? tensor(job.bias, [E], 0) : null,
            ffnGateExps: tensor(job.gate, [H, F, E], 8),
            ffnUpExps: tensor(job.up, [H, F, E], 8),
            ffnDownExps: tensor(job.down, [F, H, E], 8),
            nExpertsUsed: K,
        };
        const X = new Float32Array(readRaw(job.x));
        const hid = new Float32Array(readRaw(job.hidden));
        const n = X.length / H;
        const eng = { nExperts: E, nExpertsUsed: K, bufNormed: new Float32Array(H),
                      bufHidden: new Float32Array(H), bufMoEOut: new Float32Array(H),
                      expertMask: null, onRouterUpdate: null };
        step = function (i) {
            const r = i % n;
            eng.bufNormed.set(X.subarray(r * H, (r + 1) * H));
            eng.bufHidden.set(hid.subarray(r * H, (r + 1) * H));
            if (job.gating === 'softmax') moEFFNSoftmax(eng, 0, layer);
            else moEFFN(eng, 0, layer);
        };
    }
    step(0);   // warm-up (JIT)
    const rates = [];
    let calls = 1;
    for (let r = 0; r < runs; r++) {
        let n = 0, el = 0;
        const t0 = process.hrtime.bigint();
        while (el < seconds) {
            step(calls++);
            n++;
            el = Number(process.hrtime.bigint() - t0) / 1e9;
        }
        rates.push(n / el);
    }
    const sorted = rates.slice().sort(function (a, b) { return a - b; });
    const med = sorted.length % 2 ? sorted[(sorted.length - 1) / 2]
                                  : 0.5 * (sorted[sorted.length / 2 - 1] + sorted[sorted.length / 2]);
    process.stdout.write(JSON.stringify({ runs: rates, median_per_s: med, calls: calls - 1,
                                          seconds_per_run: seconds, threads: 1, node: process.version }) + '\n');
}

module.exports = { halfToNumber, matmulQ80xF32, matmulF32xF32, matmulGeneric, readWeightF32,
                   siluInPlace, mulInPlace, addVec, expertSlice, moEFFN, softmaxF32,
                   moEFFNSoftmax };

if (require.main === module) {
    const cmd = process.argv[2];
    if (cmd === 'run') runJob(process.argv[3]);
    else if (cmd === 'bench') bench(Number(process.argv[3] || 10), false);
    else if (cmd === 'bench-qwen3') bench(Number(process.argv[3] || 10), true);
    else if (cmd === 'bench-matvec') benchMatvec(Number(process.argv[3] || 10));
    else if (cmd === 'bench-job') benchJob(process.argv[3], Number(process.argv[4] || 5), Number(process.argv[5] || 2));
    else {
        process.stderr.write('usage: node moe_ref.js run <job.json> | bench <seconds> | bench-qwen3 <seconds> | ' +
                             'bench-matvec <seconds> | bench-job <job.json> <runs> <seconds per run>\n');
        process.exit(2);
    }
}
