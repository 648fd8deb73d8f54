'use strict';
// GPU check of MoEDevice.attachGGUF: the engine's _moEFFN on layers bound from
// a GGUF file by the native reader, against the Node restatement of the
// reference (oracle/moe_ref.js) on metas over the same file bytes.  Prints one
// JSON line; exits 1 on any failure.
//   node gguf_check.js <file.gguf> <sigmoid|softmax> <tokens>
const fs = require('fs');
const path = require('path');
const ref = require(path.join(__dirname, '..', '..', 'oracle', 'moe_ref.js'));
const qq = require(path.join(__dirname, '..', '..', 'qwenqwen3.js_amd', 'js'));

const file = process.argv[2];
const SOFTMAX = process.argv[3] === 'softmax';
const NT = Number(process.argv[4] || 3);

const bytes = fs.readFileSync(file);
const buffer = bytes.buffer.slice(bytes.byteOffset, bytes.byteOffset + bytes.byteLength);
const scope = { matmulGeneric: ref.matmulGeneric };
class FakeEngine {
    constructor(H, E, K) {
        this.nExperts = E; this.nExpertsUsed = SOFTMAX ? 0 : K;
        this.bufNormed = new Float32Array(H); this.bufHidden = new Float32Array(H);
        this.bufMoEOut = new Float32Array(H); this.expertMask = null; this.onRouterUpdate = null;
    }
    _moEFFN(l, layer) { return SOFTMAX ? ref.moEFFNSoftmax(this, l, layer) : ref.moEFFN(this, l, layer); }
}
class DevEngine extends FakeEngine {}
scope[SOFTMAX ? 'Qwen3Engine' : 'Lfm2Engine'] = DevEngine;
const dev = qq.install(scope, { device: 0 });
const table = dev.attachGGUF(file);
const meta = function (name) {     // getTensorMetaByName over the whole-file buffer
    for (const t of table) if (t.name === name) return { buffer: buffer, offset: t.offset, nbytes: t.nbytes,
                                                         shape: t.shape, type: t.type };
    return null;
};

const result = { ok: true, checks: [], max_rel_l2: 0 };
function check(name, cond, extra) {
    result.checks.push(Object.assign({ name: name, ok: !!cond }, extra || {}));
    if (!cond) result.ok = false;
}
function relL2(a, b) {
    let num = 0, den = 0;
    for (let i = 0; i < a.length; i++) { const d = a[i] - b[i]; num += d * d; den += b[i] * b[i]; }
    return Math.sqrt(num / (den || 1));
}
let s = 12345;
function rnd() { s = (s * 1103515245 + 12345) >>> 0; return (s / 4294967296) * 2 - 1; }

for (let l = 0; meta('blk.' + l + '.ffn_gate_inp.weight'); l++) {
    const p = 'blk.' + l + '.';
    const g = meta(p + 'ffn_gate_exps.weight');
    const H = g.shape[0], E = g.shape[2];
    const K = dev.native.ggufMoeParams(dev._gguf, l, 0, SOFTMAX ? 1 : 0).K;
    const layer = { routerWeight: meta(p + 'ffn_gate_inp.weight'),
                    expProbsBias: SOFTMAX ? null : meta(p + 'exp_probs_b.bias'),
                    ffnGateExps: g, ffnUpExps: meta(p + 'ffn_up_exps.weight'),
                    ffnDownExps: meta(p + 'ffn_down_exps.weight'), nExpertsUsed: K };
    const a = new FakeEngine(H, E, K), b = new DevEngine(H, E, K);
    let ra = null, rb = null;
    a.onRouterUpdate = function (r) { ra = r; };
    b.onRouterUpdate = function (r) { rb = r; };
    for (let t = 0; t < NT; t++) {
        for (let i = 0; i < H; i++) { const v = rnd() * 2; a.bufNormed[i] = v; b.bufNormed[i] = v; }
        for (let i = 0; i < H; i++) { const v = rnd(); a.bufHidden[i] = v; b.bufHidden[i] = v; }
        const h0 = Float32Array.from(a.bufHidden);
        a._moEFFN(l, layer);
        b._moEFFN(l, layer);
        const err = relL2(b.bufHidden.map(function (v, i) { return v - h0[i]; }),
                          a.bufHidden.map(function (v, i) { return v - h0[i]; }));
        result.max_rel_l2 = Math.max(result.max_rel_l2, err);
        const tag = 'block ' + l + ' token ' + t;
        check(tag + ' selected', JSON.stringify(ra.selected) === JSON.stringify(rb.selected));
        check(tag + ' weights', JSON.stringify(ra.weights) === JSON.stringify(rb.weights));
        check(tag + ' probs', JSON.stringify(ra.probs) === JSON.stringify(rb.probs));
        check(tag + ' hidden', err < 1e-4, { rel_l2: err });
    }
    check('block ' + l + ' bound from the file', layer._qqMoe && layer._qqMoe.K === K);
}
check('blocks seen', result.checks.length > 0);
dev.release();
process.stdout.write(JSON.stringify(result) + '\n');
process.exit(result.ok ? 0 : 1);
