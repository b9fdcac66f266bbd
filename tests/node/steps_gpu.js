'use strict';
// GPU run of decodeSteps / decodeStepsAsync (the k-step loop with the token
// fed back on the device), driven by tests/test_gpu_node.py: reads a case
// directory (steps.json + step_logits.f32 [k][rows][vocab] + first.u32),
// runs the loop over device-resident and then host logits, and writes the
// per-row results, the tokens each step was fed and the windows after.
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

const meta = JSON.parse(fs.readFileSync(path.join(dir, 'steps.json'), 'utf8'));
const rows = meta.rows, vocab = meta.vocab, k = meta.k;
const logits = read('step_logits.f32', Float32Array);
const first = read('first.u32', Uint32Array);
const n = rows * vocab;

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
    const bufs = [];
    for (let i = 0; i < k; i++) bufs.push(s.alloc(n * 4).upload(logits.subarray(i * n, (i + 1) * n)));
    const base = { rows: rows, vocab: vocab, k: k, params: meta.params, firstTokens: first,
      windowSize: meta.windowSize };
    const w1 = windows();
    const fed = [];
    const res = s.decodeSteps(Object.assign({}, base, { windows: w1, logits: function (i, next) {
      fed.push(Array.from(next.download(new Uint32Array(rows))));
      return bufs[i];
    } }));
    fs.writeFileSync(path.join(dir, 'js_steps.json'), JSON.stringify({
      results: res, fed: fed, windows: w1.map(function (w) { return w.genIds; }) }));
    step('decodeSteps (device logits) done');

    const w2 = windows();
    const res2 = await s.decodeStepsAsync(Object.assign({}, base, { windows: w2, logits: function (i) {
      return Promise.resolve(logits.subarray(i * n, (i + 1) * n));
    } }));
    fs.writeFileSync(path.join(dir, 'js_steps_async.json'), JSON.stringify({
      results: res2, windows: w2.map(function (w) { return w.genIds; }) }));
    step('decodeStepsAsync (host logits) done');

    let msg = '';
    try { s.decodeSteps(Object.assign({}, base, { k: 0, logits: function (i) { return bufs[i]; } })); } catch (e) {
      msg = e.message;
    }
    if (msg !== 'k must be >= 1') throw new Error('k check: ' + msg);
    for (let i = 0; i < k; i++) bufs[i].free();
  } finally {
    await s.close();
  }
}

main().then(function () { step('all done'); }, function (e) { console.error(e); process.exit(1); });
