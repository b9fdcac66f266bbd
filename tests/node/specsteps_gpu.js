'use strict';
// GPU run of specSteps / specStepsAsync (specChain's rounds with acceptSpec's
// commit on the device), driven by tests/test_gpu_node.py: reads a case
// directory (specsteps.json and each round's verify and draft rows), runs
// the chain with host and then device logits, and writes the round log, the
// final state and the windows after.
const fs = require('fs');
const path = require('path');
const sas = require(path.join(__dirname, '..', '..', 'shared_amd', 'js'));

const dir = process.argv[2];
function read(name, Type) {
  const b = fs.readFileSync(path.join(dir, name));
  const copy = new Uint8Array(b.byteLength);
  copy.set(b);
  return new Type(copy.buffer);
}
function step(msg) { console.log('[node] ' + msg); }

const meta = JSON.parse(fs.readFileSync(path.join(dir, 'specsteps.json'), 'utf8'));
const R = meta.rounds;
const targets = [], drafts = [];
for (let r = 0; r < R; r++) {
  targets.push(read('target_' + r + '.f32', Float32Array));
  drafts.push(read('draft_' + r + '.f32', Float32Array));
}

function windows() {
  return meta.windows.map(function (h) {
    const w = new sas.PenaltyWindow(meta.windowSize);
    for (let i = 0; i < h.length; i++) w.note(h[i]);
    return w;
  });
}

async function main() {
  const s = new sas.Sampler(0);
  try {
    const base = { vocab: meta.vocab, seqs: meta.seqs, draftLen: meta.drafts, rounds: R, params: meta.params,
      windowSize: meta.windowSize };
    const w1 = windows();
    const res = s.specSteps(Object.assign({}, base, { windows: w1, logits: function (r) {
      return { target: targets[r], draft: drafts[r] };
    } }));
    res.windows = w1.map(function (x) { return x.genIds; });
    fs.writeFileSync(path.join(dir, 'js_specsteps.json'), JSON.stringify(res));
    step('specSteps (host logits) done');

    const tb = targets.map(function (t) { return s.alloc(t.byteLength).upload(t); });
    const db = drafts.map(function (t) { return s.alloc(t.byteLength).upload(t); });
    const w2 = windows();
    const res2 = await s.specStepsAsync(Object.assign({}, base, { windows: w2, logits: function (r) {
      return Promise.resolve({ target: tb[r], draft: db[r] });
    } }));
    res2.windows = w2.map(function (x) { return x.genIds; });
    fs.writeFileSync(path.join(dir, 'js_specsteps_async.json'), JSON.stringify(res2));
    step('specStepsAsync (device logits) done');

    let msg = '';
    try { s.specSteps(Object.assign({}, base, { rounds: 0, logits: function () { return null; } })); } catch (e) {
      msg = e.message;
    }
    if (msg !== 'rounds must be >= 1') throw new Error('rounds check: ' + msg);
    tb.concat(db).forEach(function (b) { b.free(); });
  } finally {
    await s.close();
  }
}

main().then(function () { step('all done'); }, function (e) { console.error(e); process.exit(1); });
