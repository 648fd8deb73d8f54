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
let threw = false;
try { engine.forward(m.nVocab, 0, false); } catch (e) { threw = /token/.test(String(e.message)); }
checks.push({ what: 'bad token throws', ok: threw });
dev.release();
process.stdout.write(JSON.stringify({ ok: checks.every(function (c) { return c.ok; }), checks: checks,
                                      max_rel_l2: maxErr }) + '\n');
