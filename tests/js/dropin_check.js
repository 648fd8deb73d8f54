'use strict';
// GPU check of the JavaScript drop-in (qwenqwen3.js_amd/js) against the Node
// restatement of the reference (oracle/moe_ref.js), in one process, on the
// same seeded tensors.  Prints one JSON line; exits 1 on any failure.
//   node dropin_check.js <H> <F> <E> <K> <tokens> [sigmoid|softmax]
// "softmax" checks Qwen3Engine._moEFFN (no bias tensor, K from the layer)
// instead of Lfm2Engine._moEFFN.
const path = require('path');
const ref = require(path.join(__dirname, '..', '..', 'oracle', 'moe_ref.js'));
const qq = require(path.join(__dirname, '..', '..', 'qwenqwen3.js_amd', 'js'));

const H = Number(process.argv[2] || 256), F = Number(process.argv[3] || 96);
const E = Number(process.argv[4] || 16), K = Number(process.argv[5] || 4);
const NT = Number(process.argv[6] || 6);
const SOFTMAX = process.argv[7] === 'softmax';

let s = 0x9e3779b9;
function next() { s ^= s << 13; s >>>= 0; s ^= s >>> 17; s ^= s << 5; s >>>= 0; return s; }
function gauss() {   // Box-Muller from the xorshift stream
    const u = ((next() >>> 8) + 1) / 16777217, v = (next() >>> 8) / 16777216;
    return Math.sqrt(-2 * Math.log(u)) * Math.cos(2 * Math.PI * v);
}
function q8(inDim, outDim, nMats) {
    const nb = Math.ceil(inDim / 32), n = nMats * outDim * nb;
    const u8 = new Uint8Array(n * 34), dv = new DataView(u8.buffer);
    const f16 = new Float32Array(1), bits = new Uint32Array(f16.buffer);
    for (let i = 0; i < n; i++) {
        f16[0] = Math.abs(gauss()) * 0.002;   // to fp16 by truncation: any fp16 value will do
        const b = bits[0], e = ((b >>> 23) & 0xff) - 127 + 15;
        const h = e <= 0 ? 0 : (e << 10) | ((b >>> 13) & 0x3ff);
        dv.setUint16(i * 34, h, true);
        for (let j = 0; j < 32; j++) u8[i * 34 + 2 + j] = (next() % 255) - 127;
    }
    return u8.buffer;
}
function relL2(a, b) {
    let num = 0, den = 0;
    for (let i = 0; i < a.length; i++) { const d = a[i] - b[i]; num += d * d; den += b[i] * b[i]; }
    return Math.sqrt(num / (den || 1));
}

const router = new Float32Array(E * H);
for (let i = 0; i < router.length; i++) router[i] = gauss() * (SOFTMAX ? 0.05 : 0.02);
const bias = new Float32Array(E);
for (let e = 0; e < E; e++) bias[e] = (gauss()) * 0.005;
const layer = {
    routerWeight: { buffer: router.buffer, offset: 0, shape: [H, E], type: 0 },
    expProbsBias: SOFTMAX ? null : { buffer: bias.buffer, offset: 0, shape: [E], type: 0 },
    ffnGateExps: { buffer: q8(H, F, E), offset: 0, shape: [H, F, E], type: 8 },
    ffnUpExps: { buffer: q8(H, F, E), offset: 0, shape: [H, F, E], type: 8 },
    ffnDownExps: { buffer: q8(F, H, E), offset: 0, shape: [F, H, E], type: 8 },
    nExpertsUsed: K,
};

class FakeEngine {
    constructor() {
        this.nExperts = E; this.nExpertsUsed = SOFTMAX ? 0 : K;   // Qwen3 reads K from the layer
        this.bufNormed = new Float32Array(H); this.bufHidden = new Float32Array(H);
        this.bufMoEOut = new Float32Array(H); this.expertMask = null; this.onRouterUpdate = null;
    }
    _moEFFN(l, layer) { return SOFTMAX ? ref.moEFFNSoftmax(this, l, layer) : ref.moEFFN(this, l, layer); }
}
class DevEngine extends FakeEngine {}

const scope = { matmulGeneric: ref.matmulGeneric };
scope[SOFTMAX ? 'Qwen3Engine' : 'Lfm2Engine'] = DevEngine;
const dev = qq.install(scope, { device: 0 });
const result = { ok: true, tokens: NT, H: H, F: F, E: E, K: K, max_rel_l2: 0, checks: [] };
function check(name, cond, extra) {
    result.checks.push(Object.assign({ name: name, ok: !!cond }, extra || {}));
    if (!cond) result.ok = false;
}

// ---- per-token _moEFFN through the patched prototype ----
const a = new FakeEngine(), b = new DevEngine();
let ra = null, rb = null;
a.onRouterUpdate = function (r) { ra = r; };
b.onRouterUpdate = function (r) { rb = r; };
for (let t = 0; t < NT; t++) {
    for (let i = 0; i < H; i++) { const v = gauss(); a.bufNormed[i] = v; b.bufNormed[i] = v; }
    for (let i = 0; i < H; i++) { const v = gauss(); a.bufHidden[i] = v; b.bufHidden[i] = v; }
    const h0 = Float32Array.from(a.bufHidden);
    if (t === NT - 1) { a.expertMask = new Set([2, 5]); b.expertMask = new Set([2, 5]); }
    a._moEFFN(3, layer);
    b._moEFFN(3, layer);
    const da = a.bufHidden.map(function (v, i) { return v - h0[i]; });
    const db = b.bufHidden.map(function (v, i) { return v - h0[i]; });
    const err = relL2(db, da);
    result.max_rel_l2 = Math.max(result.max_rel_l2, err);
    check('token ' + t + ' selected', JSON.stringify(ra.selected) === JSON.stringify(rb.selected),
          { ref: ra.selected, dev: rb.selected });
    check('token ' + t + ' weights', JSON.stringify(ra.weights) === JSON.stringify(rb.weights));
    check('token ' + t + ' probs', JSON.stringify(ra.probs) === JSON.stringify(rb.probs));
    check('token ' + t + ' layer', ra.layer === 3 && rb.layer === 3);
    check('token ' + t + ' hidden', err < 1e-4, { rel_l2: err });
}

// ---- batched entry point = per-token reference ----
const T = 5, X = new Float32Array(T * H), hid = new Float32Array(T * H);
for (let i = 0; i < X.length; i++) { X[i] = gauss(); hid[i] = gauss(); }
const hidDev = Float32Array.from(hid);
const rbat = dev.moeForward(layer, X, hidDev, T,
                            { K: K, gating: SOFTMAX ? qq.GATING_SOFTMAX : qq.GATING_SIGMOID_BIAS,
                              wantProbs: true });
const c = new FakeEngine();
let rc = null;
c.onRouterUpdate = function (r) { rc = r; };
for (let t = 0; t < T; t++) {
    c.bufNormed.set(X.subarray(t * H, (t + 1) * H));
    c.bufHidden.set(hid.subarray(t * H, (t + 1) * H));
    c._moEFFN(0, layer);
    check('batch ' + t + ' selected', JSON.stringify(Array.from(rbat.idx.subarray(t * K, (t + 1) * K))) === JSON.stringify(rc.selected));
    const dref = c.bufHidden.map(function (v, i) { return v - hid[t * H + i]; });
    const ddev = hidDev.subarray(t * H, (t + 1) * H).map(function (v, i) { return v - hid[t * H + i]; });
    const err = relL2(ddev, dref);
    result.max_rel_l2 = Math.max(result.max_rel_l2, err);
    check('batch ' + t + ' hidden', err < 1e-4, { rel_l2: err });
}

// ---- matmulQ80xF32 / matmulGeneric drop-ins ----
const wmeta = { buffer: q8(1024, 3072, 1), offset: 0, shape: [1024, 3072], type: 8 };
const xv = new Float32Array(Math.max(1024, H));
for (let i = 0; i < xv.length; i++) xv[i] = gauss();
const x1k = xv.subarray(0, 1024);
const ym = scope.matmulQ80xF32(wmeta, x1k), yr = ref.matmulQ80xF32(wmeta, x1k);
check('matmulQ80xF32', ym.length === 3072 && relL2(ym, yr) < 1e-4, { rel_l2: relL2(ym, yr) });
const slice = ref.expertSlice(layer.ffnGateExps, Math.min(7, E - 1));
const ys = scope.matmulGeneric(slice, xv.subarray(0, H)), ysr = ref.matmulGeneric(slice, xv.subarray(0, H));
check('matmulGeneric expert slice', relL2(ys, ysr) < 1e-4, { rel_l2: relL2(ys, ysr) });
const yf = scope.matmulGeneric(layer.routerWeight, xv.subarray(0, H));
const yfr = ref.matmulF32xF32(layer.routerWeight, xv.subarray(0, H));
check('matmulGeneric F32 delegates', JSON.stringify(Array.from(yf)) === JSON.stringify(Array.from(yfr)));
let threw = false;
try { scope.matmulGeneric({ buffer: wmeta.buffer, offset: 0, shape: [1024, 8], type: 13 }, x1k); }
catch (e) { threw = /Unsupported tensor type for matmul: 13/.test(String(e)); }
check('unknown type throws like the reference', threw);
let short = false;
try { scope.matmulQ80xF32(wmeta, new Float32Array(100)); }
catch (e) { short = e instanceof RangeError; }
check('short input is a RangeError', short);

process.stdout.write(JSON.stringify(result) + '\n');
process.exit(result.ok ? 0 : 1);
