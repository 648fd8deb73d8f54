'use strict';
// GPU check of MoEDevice.attachLfm2Forward (the whole-token device forward
// behind the reference's Lfm2Engine.forward surface) against
// oracle/lfm2_ref.js on the same model file.
//   node lfm2_check.js <job.json>     (job as tests/_lfm2.py writes it)
// Prints one JSON line {ok, checks, max_rel_l2}.
const path = require('path');
const ROOT = path.join(__dirname, '..', '..');
const ref = require(path.join(ROOT, 'oracle', 'lfm2_ref.js'));
const qq = require(path.join(ROOT, 'qwenqwen3.js_amd', 'js', 'index.js'));
const fs = require('fs');

function relL2(a, b) {
    let num = 0, den = 0;
    for (let i = 0; i < b.length; i++) {
        num += (a[i] - b[i]) * (a[i] - b[i]);
        den += b[i] * b[i];
    }
    return Math.sqrt(num / (den > 0 ? den : 1));
}

const job = JSON.parse(fs.readFileSync(process.argv[2], 'utf8'));
const b = fs.readFileSync(job.gguf);
const buf = b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength);
const metas = {};
for (const name of Object.keys(job.tensors)) {
    const t = job.tensors[name];
    metas[name] = { buffer: buf, offset: t.offset, shape: t.shape, type: t.type };
}
const m = ref.buildModel(job.kv, metas);
const dev = new qq.MoEDevice(0);
dev.attachGGUF(job.gguf);
const engine = {};
const info = dev.attachLfm2Forward(engine);
const checks = [];
let maxErr = 0;
checks.push({ what: 'info', ok: info.nVocab === m.nVocab && info.nLayers === m.nLayers &&
              info.nAttnLayers === m.nAttn });
const first = [];
job.tokens.forEach(function (tok, t) {
    const want = ref.forward(m, tok, t, false);
    const got = engine.forward(tok, t, false);
    const err = relL2(got, want);
    maxErr = Math.max(maxErr, err);
    checks.push({ what: 'token ' + t, ok: got === engine.bufLogits && err < 1e-4, err: err });
    if (t < 2) first.push(Float32Array.from(got));
});
checks.push({ what: 'skipLogits', ok: engine.forward(job.tokens[0], job.tokens.length, true) === null });
engine.resetKVCache();
for (let t = 0; t < first.length; t++) {
    const again = engine.forward(job.tokens[t], t, false);
    let same = true;
    for (let i = 0; i < again.length; i++) if (again[i] !== first[t][i]) same = false;
    checks.push({ what: 'reset replay ' + t, ok: same });
}
// onRouterUpdate of every MoE block and expertMask, against the reference's
// forward run with the same mask (src/lfm2-engine.js:449-464)
engine.resetKVCache();
// (fresh oracle models: each keeps its own caches)
const m2 = ref.buildModel(job.kv, metas);
const sel0 = [];
m2.routes = sel0;
ref.forward(m2, job.tokens[0], 0, true);
const mask = new Set([sel0[0][0], sel0[sel0.length - 1][1]]);
const m3 = ref.buildModel(job.kv, metas);
m3.expertMask = mask;
m3.payloads = [];
const got = [];
engine.expertMask = mask;
engine.onRouterUpdate = function (r) { got.push(r); };
let payOk = true, maskErr = 0;
job.tokens.slice(0, 3).forEach(function (tok, t) {
    const want = ref.forward(m3, tok, t, false);
    const logits = engine.forward(tok, t, false);
    maskErr = Math.max(maskErr, relL2(logits, want));
});
// (selected experts equal; weights and probabilities to 1e-5 relative: past the
// first block the device's hidden state differs from the oracle's in the last
// bits, and with it every later router's logits)
let payErr = 0;
payOk = got.length === m3.payloads.length && got.every(function (r, i) {
    const p = m3.payloads[i];
    payErr = Math.max(payErr, relL2(r.weights, p.weights), relL2(r.probs, p.probs));
    return r.layer === p.layer && JSON.stringify(r.selected) === JSON.stringify(p.selected) &&
        r.weights.length === p.weights.length && r.probs.length === p.probs.length;
}) && payErr < 1e-5;
checks.push({ what: 'onRouterUpdate payloads', ok: payOk && got.length > 0, n: got.length, err: payErr });
checks.push({ what: 'expertMask logits', ok: maskErr < 1e-4, err: maskErr });
engine.expertMask = null;
engine.onRouterUpdate = null;
// a second engine gets its own model; the first keeps working
const engine2 = {};
dev.attachLfm2Forward(engine2);
engine.resetKVCache();
engine2.resetKVCache();
const a1 = Float32Array.from(engine.forward(job.tokens[0], 0, false));
const a2 = Float32Array.from(engine2.forward(job.tokens[0], 0, false));
checks.push({ what: 'two engines', ok: relL2(a1, a2) === 0 });
let threw = false;
try { engine.forward(m.nVocab, 0, false); } catch (e) { threw = /token/.test(String(e.message)); }
checks.push({ what: 'bad token throws', ok: threw });
dev.release();
process.stdout.write(JSON.stringify({ ok: checks.every(function (c) { return c.ok; }), checks: checks,
                                      max_rel_l2: maxErr }) + '\n');
