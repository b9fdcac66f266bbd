'use strict';
// GPU run of decodeStepsWithHead / decodeStepsWithHeadAsync (the k-step
// loop with the LM head fused and the token fed back on the device), driven
// by tests/test_gpu_node.py: reads a case directory (headsteps.json, the
// hidden states of every step [k][rows][dim] and a GGUF Q6_K head), runs the
// loop with host and then device hidden states, and writes the per-row
// results, the tokens each step was fed and the windows after.
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

const meta = JSON.parse(fs.readFileSync(path.join(dir, 'headsteps.json'), 'utf8'));
const rows = meta.rows, vocab = meta.vocab, k = meta.k, dim = meta.dim;
const hidden = read('hs.f32', Float32Array);
const head = read('head.u8', Uint8Array);
const mask = read('mask.u32', Uint32Array);
const first = read('first.u32', Uint32Array);
const n = rows * dim;

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
    const w = s.alloc(head.byteLength).upload(head);
    const base = { rows: rows, vocab: vocab, k: k, params: meta.params, mask: mask, firstTokens: first,
      windowSize: meta.windowSize, head: { weight: w, dim: dim, format: 'q6_k' } };
    const w1 = windows();
    const fed = [];
    const res = s.decodeStepsWithHead(Object.assign({}, base, { windows: w1, hidden: function (i, next) {
      fed.push(Array.from(next.download(new Uint32Array(rows))));
      return hidden.subarray(i * n, (i + 1) * n);
    } }));
    fs.writeFileSync(path.join(dir, 'js_headsteps.json'), JSON.stringify({
      results: res, fed: fed, windows: w1.map(function (x) { return x.genIds; }) }));
    step('decodeStepsWithHead (host hidden) done');

    const bufs = [];
    for (let i = 0; i < k; i++) bufs.push(s.alloc(n * 4).upload(hidden.subarray(i * n, (i + 1) * n)));
    const w2 = windows();
    const res2 = await s.decodeStepsWithHeadAsync(Object.assign({}, base, { windows: w2, hidden: function (i) {
      return Promise.resolve(bufs[i]);
    } }));
    fs.writeFileSync(path.join(dir, 'js_headsteps_async.json'), JSON.stringify({
      results: res2, windows: w2.map(function (x) { return x.genIds; }) }));
    step('decodeStepsWithHeadAsync (device hidden) done');

    let msg = '';
    try { s.decodeStepsWithHead(Object.assign({}, base, { hidden: null })); } catch (e) { msg = e.message; }
    if (msg !== 'hidden must be a function (step, nextTokens)') throw new Error('hidden check: ' + msg);
    for (let i = 0; i < k; i++) bufs[i].free();
    w.free();
  } finally {
    await s.close();
  }
}

main().then(function () { step('all done'); }, function (e) { console.error(e); process.exit(1); });
