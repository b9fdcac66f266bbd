'use strict';
// GPU run of specExact / specExactAsync (the reference's exact-match
// speculative round), driven by tests/test_gpu_node.py: reads spec.json +
// spec_target.f32 + spec_draft.f32, runs one round with the draft head's
// logits and PenaltyWindows, then the same round async with the drafts
// given and plain history lists, and writes both results.
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

const meta = JSON.parse(fs.readFileSync(path.join(dir, 'spec.json'), 'utf8'));
const target = read('spec_target.f32', Float32Array);
const draft = read('spec_draft.f32', Float32Array);

async function main() {
  const s = new sas.Sampler(0);
  try {
    const windows = meta.history.map(function (h) {
      const w = new sas.PenaltyWindow(512);
      for (let i = 0; i < h.length; i++) w.note(h[i]);
      return w;
    });
    const base = { vocab: meta.vocab, seqs: meta.seqs, draftLen: meta.drafts, params: meta.params,
      round: meta.round, target: target };
    const r1 = s.specExact(Object.assign({}, base, { draft: draft, windows: windows }));
    fs.writeFileSync(path.join(dir, 'js_spec.json'), JSON.stringify({
      results: r1, windows: windows.map(function (w) { return w.genIds; }) }));
    step('specExact (draft head) done');

    const ids = new Uint32Array(meta.seqs * meta.drafts);
    for (let q = 0; q < meta.seqs; q++) for (let j = 0; j < meta.drafts; j++) ids[q * meta.drafts + j] = r1[q].drafts[j];
    const r2 = await s.specExactAsync(Object.assign({}, base, { draftIds: ids, history: meta.history }));
    fs.writeFileSync(path.join(dir, 'js_spec_async.json'), JSON.stringify({ results: r2 }));
    step('specExactAsync (given drafts) done');
  } finally {
    await s.close();
  }
}

main().then(function () { step('all done'); }, function (e) { console.error(e); process.exit(1); });
