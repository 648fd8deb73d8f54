'use strict';
// GPU check of the WebGPU-engine drop-in (qwenqwen3.js_amd/js): the
// _moEFFNGPU / _readbackRoutingData rebinding of Lfm2GPUEngine and
// Qwen3GPUEngine for an engine whose buffers are DeviceBuffers, against the
// Node restatement of the CPU engine (oracle/moe_ref.js) on the same seeded
// tensors.  Prints one JSON line; exits 1 on any failure.
//   node gpu_engine_check.js <H> <F> <E> <K> <tokens> [sigmoid|softmax]
const path = require('path');
const ref = require(path.join(__dirname, '..', '..', 'oracle', 'moe_ref.js'));
const qq = require(path.join(__dirname, '..', '..', 'qwenqwen3.js_amd', 'js'));

const H = Number(process.argv[2] || 256), F = Number(process.argv[3] || 96);
const E = Number(process.argv[4] || 16), K = Number(process.argv[5] || 4);
const NT = Number(process.argv[6] || 3);
const SOFTMAX = process.argv[7] === 'softmax';
const ABS = [1, 2, 4];          // absolute layer index of each MoE layer
const EPS = 1e-5;

let s = 0x2545f491;
function next() { s ^= s << 13; s >>>= 0; s ^= s >>> 17; s ^= s << 5; s >>>= 0; return s; }
function gauss() {
    const u = ((next() >>> 8) + 1) / 16777217, v = (next() >>> 8) / 16777216;
    return Math.sqrt(-2 * Math.log(u)) * Math.cos(2 * Math.PI * v);
}
function q8(inDim, outDim, nMats) {
    const nb = Math.ceil(inDim / 32), n = nMats * outDim * nb;
    const u8 = new Uint8Array(n * 34), dv = new DataView(u8.buffer);
    const f = new Float32Array(1), bits = new Uint32Array(f.buffer);
    for (let i = 0; i < n; i++) {
        f[0] = Math.abs(gauss()) * 0.002;
        const b = bits[0], e = ((b >>> 23) & 0xff) - 127 + 15;
        dv.setUint16(i * 34, e <= 0 ? 0 : (e << 10) | ((b >>> 13) & 0x3ff), true);
        for (let j = 0; j < 32; j++) u8[i * 34 + 2 + j] = (next() % 255) - 127;
    }
    return u8.buffer;
}
function relL2(a, b) {
    let num = 0, den = 0;
    for (let i = 0; i < a.length; i++) { const d = a[i] - b[i]; num += d * d; den += b[i] * b[i]; }
    return Math.sqrt(num / (den || 1));
}
// rmsnorm of src/tensor.js:103-114 (binary64 sum of squares, one fp32 store)
function rmsnorm(x, w) {
    let ss = 0;
    for (let i = 0; i < x.length; i++) ss += x[i] * x[i];
    const inv = 1 / Math.sqrt(ss / x.length + EPS);
    const out = new Float32Array(x.length);
    for (let i = 0; i < x.length; i++) out[i] = w[i] * (x[i] * inv);
    return out;
}
function makeLayer() {
    const router = new Float32Array(E * H);
    for (let i = 0; i < router.length; i++) router[i] = gauss() * (SOFTMAX ? 0.05 : 0.02);
    const bias = new Float32Array(E);
    for (let e = 0; e < E; e++) bias[e] = gauss() * 0.005;
    const nw = new Float32Array(H);
    for (let i = 0; i < H; i++) nw[i] = 1 + 0.1 * gauss();
    return {
        routerWeight: { buffer: router.buffer, offset: 0, shape: [H, E], type: 0 },
        expProbsBias: SOFTMAX ? null : { buffer: bias.buffer, offset: 0, shape: [E], type: 0 },
        ffnGateExps: { buffer: q8(H, F, E), offset: 0, shape: [H, F, E], type: 8 },
        ffnUpExps: { buffer: q8(H, F, E), offset: 0, shape: [H, F, E], type: 8 },
        ffnDownExps: { buffer: q8(F, H, E), offset: 0, shape: [F, H, E], type: 8 },
        nExpertsUsed: K,
        normW: nw,
    };
}
const layers = ABS.map(makeLayer);

// The WebGPU engine classes of the scope: their own methods stand for the
// WGSL path and must run only for engines that are not on the device.
let webgpuCalls = 0;
let resets = 0;
class Lfm2GPUEngine {
    _moEFFNGPU() { webgpuCalls++; }
    _readbackRoutingData() { webgpuCalls++; return Promise.resolve(); }
    _resetGPUState() { resets++; }
    resetKVCache() { this._resetGPUState(); }
}
class Qwen3GPUEngine extends Lfm2GPUEngine {}
const scope = { matmulGeneric: ref.matmulGeneric, Lfm2GPUEngine: Lfm2GPUEngine, Qwen3GPUEngine: Qwen3GPUEngine };
const dev = qq.install(scope, { device: 0 });
const Cls = SOFTMAX ? Qwen3GPUEngine : Lfm2GPUEngine;

const result = { ok: true, tokens: NT, H: H, F: F, E: E, K: K, max_rel_l2: 0, checks: [] };
function check(name, cond, extra) {
    result.checks.push(Object.assign({ name: name, ok: !!cond }, extra || {}));
    if (!cond) result.ok = false;
}

// an engine object laid out as the WebGPU engines are (src/webgpu.js:1470-1500,
// 1605-1640; Qwen3 keeps nExperts / nExpertsUsed itself, :498-530)
function makeEngine(sharedRecords) {
    const eng = Object.create(Cls.prototype);
    eng._gpu = dev;
    if (SOFTMAX) { eng.nExperts = E; eng.nExpertsUsed = K; }
    else eng._cpu = { nExperts: E, nExpertsUsed: K, layers: layers };
    eng._buf = { normed: dev.createBuffer(H * 4), hidden: dev.createBuffer(H * 4) };
    eng._moeAbsLayerIndices = ABS.slice();
    eng.batchRouterUpdate = true;
    eng.expertMask = null;
    eng.onRouterUpdate = null;
    if (sharedRecords) dev.routingBuffers(eng, ABS.length);
    else eng._gpuRoutingBufs = ABS.map(function () { return dev.createBuffer((2 * K + E) * 4); });
    return eng;
}
class HostEngine {   // the CPU engine's fields moEFFN reads (src/lfm2-engine.js:413-487)
    constructor() {
        this.nExperts = E; this.nExpertsUsed = SOFTMAX ? 0 : K;
        this.bufNormed = new Float32Array(H); this.bufHidden = new Float32Array(H);
        this.bufMoEOut = new Float32Array(H); this.expertMask = null; this.onRouterUpdate = null;
    }
}
function hostBlock(h, l, normed, hidden) {
    h.bufNormed.set(normed); h.bufHidden.set(hidden);
    if (SOFTMAX) ref.moEFFNSoftmax(h, ABS[l], layers[l]); else ref.moEFFN(h, ABS[l], layers[l]);
    return Float32Array.from(h.bufHidden);
}

// ---- 1. each block from host-written normed / hidden: routing exact ----
for (const shared of [true, false]) {
    const eng = makeEngine(shared);
    const host = new HostEngine();
    const tag = shared ? 'one record allocation' : 'per-layer records';
    for (let t = 0; t < NT; t++) {
        const want = [], got = [];
        host.onRouterUpdate = function (r) { want.push(r); };
        eng.onRouterUpdate = function (r) { got.push(r); };
        if (t === NT - 1) { host.expertMask = new Set([1, 3]); eng.expertMask = new Set([1, 3]); }
        let err = 0;
        for (let l = 0; l < ABS.length; l++) {
            const hid = new Float32Array(H), x = new Float32Array(H);
            for (let i = 0; i < H; i++) { hid[i] = gauss(); x[i] = gauss(); }
            dev.writeBuffer(eng._buf.hidden, 0, hid);
            dev.writeBuffer(eng._buf.normed, 0, x);
            eng._moEFFNGPU(ABS[l], { _moeIdx: l }, layers[l]);
            const hd = dev.readF32Sync(eng._buf.hidden, H);
            const hr = hostBlock(host, l, x, hid);
            err = Math.max(err, relL2(hd.map(function (v, i) { return v - hid[i]; }),
                                      hr.map(function (v, i) { return v - hid[i]; })));
        }
        eng._readbackRoutingData();
        result.max_rel_l2 = Math.max(result.max_rel_l2, err);
        check(tag + ' token ' + t + ' hidden', err < 1e-4, { rel_l2: err });
        check(tag + ' token ' + t + ' payload count', got.length === ABS.length && want.length === ABS.length);
        for (let l = 0; l < Math.min(got.length, want.length); l++) {
            const g = got[l], w = want[l];
            check(tag + ' token ' + t + ' layer ' + l, g.layer === w.layer &&
                  JSON.stringify(g.selected) === JSON.stringify(w.selected) &&
                  // the record holds weights rounded to fp32 (the shaders' result buffer is f32)
                  JSON.stringify(g.weights) === JSON.stringify(w.weights.map(Math.fround)) &&
                  JSON.stringify(g.probs) === JSON.stringify(w.probs),
                  { dev: g.selected, ref: w.selected });
        }
    }
}
check('WebGPU methods not called for device engines', webgpuCalls === 0, { calls: webgpuCalls });

// ---- 2. a token chained on the device: rmsnorm + block per layer, no host copy between ----
{
    const eng = makeEngine(true);
    const host = new HostEngine();
    const got = [], want = [];
    eng.onRouterUpdate = function (r) { got.push(r); };
    host.onRouterUpdate = function (r) { want.push(r); };
    const h0 = new Float32Array(H);
    for (let i = 0; i < H; i++) h0[i] = gauss();
    const nws = layers.map(function (L) { return dev.uploadBuffer(L.normW); });
    dev.writeBuffer(eng._buf.hidden, 0, h0);
    let hr = Float32Array.from(h0);
    for (let l = 0; l < ABS.length; l++) {
        dev.rmsnormDev(eng._buf.hidden, nws[l], eng._buf.normed, 1, H, EPS);
        eng._moEFFNGPU(ABS[l], { _moeIdx: l }, layers[l]);
        hr = hostBlock(host, l, rmsnorm(hr, layers[l].normW), hr);
    }
    eng._readbackRoutingData();
    const hd = dev.readF32Sync(eng._buf.hidden, H);
    const err = relL2(hd.map(function (v, i) { return v - h0[i]; }), hr.map(function (v, i) { return v - h0[i]; }));
    result.max_rel_l2 = Math.max(result.max_rel_l2, err);
    check('chained hidden', err < 1e-4, { rel_l2: err });
    check('chained selected', got.length === ABS.length && got.every(function (g, l) {
        return JSON.stringify(g.selected) === JSON.stringify(want[l].selected) && g.layer === ABS[l];
    }));
    check('chained probs', got.every(function (g, l) { return relL2(g.probs, want[l].probs) < 1e-5; }));
}

// ---- 3. an engine whose buffers are not on the device keeps its own methods ----
{
    const other = Object.create(Cls.prototype);
    other._buf = { normed: {}, hidden: {} };
    other.onRouterUpdate = function () {};
    other._moEFFNGPU(1, { _moeIdx: 0 }, layers[0]);
    other._readbackRoutingData();
    check('other engines delegate to their own methods', webgpuCalls === 2, { calls: webgpuCalls });
}

// ---- 4. T rows at once with the record (the batched router path) ----
{
    const T = 5;
    const X = new Float32Array(T * H), hid = new Float32Array(T * H);
    for (let i = 0; i < X.length; i++) { X[i] = gauss(); hid[i] = gauss(); }
    const xb = dev.uploadBuffer(X), hb = dev.uploadBuffer(hid), rb = dev.createBuffer(T * (2 * K + E) * 4);
    dev.moeForwardDev(layers[0], xb, hb, T, { K: K, gating: SOFTMAX ? qq.GATING_SOFTMAX : qq.GATING_SIGMOID_BIAS,
                                             record: rb });
    const hd = dev.readF32Sync(hb, T * H), rec = dev.readF32Sync(rb, T * (2 * K + E));
    const host = new HostEngine();
    let r = null;
    host.onRouterUpdate = function (p) { r = p; };
    for (let t = 0; t < T; t++) {
        const hr = hostBlock(host, 0, X.subarray(t * H, (t + 1) * H), hid.subarray(t * H, (t + 1) * H));
        const rr = rec.subarray(t * (2 * K + E), (t + 1) * (2 * K + E));
        const err = relL2(hd.subarray(t * H, (t + 1) * H).map(function (v, i) { return v - hid[t * H + i]; }),
                          hr.map(function (v, i) { return v - hid[t * H + i]; }));
        result.max_rel_l2 = Math.max(result.max_rel_l2, err);
        check('rows ' + t + ' hidden', err < 1e-4, { rel_l2: err });
        check('rows ' + t + ' record',
              JSON.stringify(Array.from(rr.subarray(0, K))) === JSON.stringify(r.selected) &&
              JSON.stringify(Array.from(rr.subarray(K, 2 * K))) === JSON.stringify(r.weights.map(Math.fround)) &&
              JSON.stringify(Array.from(rr.subarray(2 * K))) === JSON.stringify(r.probs));
    }
    let range = false;
    try { dev.moeForwardDev(layers[0], xb, hb, T + 1, { K: K, gating: SOFTMAX ? qq.GATING_SOFTMAX : qq.GATING_SIGMOID_BIAS }); }
    catch (e) { range = e instanceof RangeError; }
    check('rows past the buffer are a RangeError', range);
}

// ---- 5. a timed-out device wait (forced from the host with a zero bound)
// leaves the engine's residual stream half updated: _moEFFNGPU refuses until
// resetKVCache(), then runs exactly again ----
{
    const eng = makeEngine(true);
    const host = new HostEngine();
    const hid = new Float32Array(H), x = new Float32Array(H);
    for (let i = 0; i < H; i++) { hid[i] = gauss(); x[i] = gauss(); }
    dev.setWaitLimit(0);
    let timedOut = false;
    for (let t = 0; t < 4 && !timedOut; t++) {
        dev.writeBuffer(eng._buf.hidden, 0, hid);
        dev.writeBuffer(eng._buf.normed, 0, x);
        eng._moEFFNGPU(ABS[0], { _moeIdx: 0 }, layers[0]);
        try { dev.readF32Sync(eng._buf.hidden, H); } catch (e) { timedOut = /timed out/.test(e.message); }
    }
    dev.setWaitLimit(50000);
    check('zero wait bound times out', timedOut);
    let refused = false;
    try { eng._moEFFNGPU(ABS[0], { _moeIdx: 0 }, layers[0]); } catch (e) { refused = /resetKVCache/.test(e.message); }
    check('engine refuses after a timeout', refused);
    eng.resetKVCache();
    check('resetKVCache reached the engine', resets === 1, { resets: resets });
    dev.writeBuffer(eng._buf.hidden, 0, hid);
    dev.writeBuffer(eng._buf.normed, 0, x);
    eng._moEFFNGPU(ABS[0], { _moeIdx: 0 }, layers[0]);
    const hd = dev.readF32Sync(eng._buf.hidden, H);
    const hr = hostBlock(host, 0, x, hid);
    const err = relL2(hd.map(function (v, i) { return v - hid[i]; }), hr.map(function (v, i) { return v - hid[i]; }));
    check('exact again after resetKVCache', err < 1e-4, { rel_l2: err });
    // an engine made after the timeout starts valid
    let fresh = true;
    try { makeEngine(true)._moEFFNGPU(ABS[0], { _moeIdx: 0 }, layers[0]); dev.synchronize(); } catch (e) { fresh = false; }
    check('an engine made after the timeout runs', fresh);
}

dev.release();
console.log(JSON.stringify(result));
process.exit(result.ok ? 0 : 1);
