'use strict';
// Host hand-over cost of the Node API on the GPU, per call: sampleRows with
// logits in a host Float32Array (uploaded by the call) against the same
// logits already resident in device memory, and the reference's CPU
// sample(cands) signature, whose candidates become a dense device row.
// Synthetic C3P-shaped inputs (fp32 logits, a packed mask, 512 history ids
// per row, top-k 50 / top-p 0.9, penalties).  Usage:
//   node shared_amd/js/bench_host.js [rows] [vocab] [reps]
const sas = require('./index.js');

const rows = parseInt(process.argv[2] || '128', 10);
const vocab = parseInt(process.argv[3] || '262144', 10);
const reps = parseInt(process.argv[4] || '20', 10);

// xorshift32: deterministic inputs
let seed = 0x9E3779B9;
function rnd() {
  seed ^= seed << 13; seed >>>= 0;
  seed ^= seed >>> 17;
  seed ^= seed << 5; seed >>>= 0;
  return seed / 4294967296;
}
function normal() {
  const u = Math.max(rnd(), 1e-12), v = rnd();
  return Math.sqrt(-2 * Math.log(u)) * Math.cos(2 * Math.PI * v);
}

function time(name, n, fn) {
  fn();
  const t0 = process.hrtime.bigint();
  for (let i = 0; i < n; i++) fn();
  const us = Number(process.hrtime.bigint() - t0) / 1e3 / n;
  console.log(name.padEnd(64) + us.toFixed(1).padStart(10) + ' us');
  return us;
}

const logits = new Float32Array(rows * vocab);
for (let i = 0; i < logits.length; i++) logits[i] = 4 * normal();
const nwords = Math.ceil(vocab / 32);
const mask = new Uint32Array(rows * nwords);
for (let r = 0; r < rows; r++) {
  const density = 0.005 + 0.195 * rnd();
  for (let id = 0; id < vocab; id++) {
    if (rnd() < density) mask[r * nwords + (id >> 5)] |= (1 << (id & 31)) >>> 0;
  }
  mask[r * nwords] |= 1;
}
const history = [];
for (let r = 0; r < rows; r++) {
  const h = new Uint32Array(512);
  for (let i = 0; i < h.length; i++) h[i] = Math.floor(rnd() * vocab);
  history.push(h);
}
const uniforms = new Float64Array(rows);
for (let r = 0; r < rows; r++) uniforms[r] = rnd();
const params = {
  temperature: 1.0, topK: 50, topP: 0.9, repetitionPenalty: 1.1, presencePenalty: 0.5, frequencyPenalty: 0.3,
};

const s = new sas.Sampler(0);
try {
  s.reserve(rows, vocab);
  const base = { rows: rows, vocab: vocab, mask: mask, params: params, history: history, uniforms: uniforms };
  console.log(rows + ' rows x ' + vocab + ' vocab (' + (logits.byteLength / 1e6).toFixed(1) + ' MB of logits per call)');
  const host = time('sampleRows, host Float32Array logits (upload included)', reps, function () {
    s.sampleRows(Object.assign({ logits: logits }, base));
  });
  const dev = s.alloc(logits.byteLength).upload(logits);
  const resident = time('sampleRows, device-resident logits', reps, function () {
    s.sampleRows(Object.assign({ logits: dev }, base));
  });
  console.log('host hand-over: ' + (host - resident).toFixed(1) + ' us per call, ' +
    (logits.byteLength / (host - resident) / 1e3).toFixed(1) + ' GB/s for the logits upload');
  dev.free();
  // sample(cands): the reference's candidate list, [id, value] pairs over
  // NBLK x 20 blocks (kernels.js:1389-1449): Gemma 256 x 20, Qwen 243 x 20
  [[262144, 256], [151936, 243]].forEach(function (vb) {
    const v = vb[0], nblk = vb[1];
    const n = nblk * 20;
    const ids = new Uint32Array(2 * n), vals = new Float32Array(2 * n);
    for (let b = 0; b < nblk; b++) {
      for (let j = 0; j < 20; j++) {
        const i = b * 20 + j;
        ids[2 * i] = Math.min(b * 1024 + Math.floor(rnd() * 1024), v - 1);
        vals[2 * i + 1] = 4 * normal();
      }
    }
    const recent = new Set();
    for (let i = 0; i < 512; i++) recent.add(Math.floor(rnd() * v));
    time('sample(cands), ' + n + ' candidates, vocab ' + v, reps * 5, function () {
      s.sample({ ids: ids, vals: vals }, { temperature: 0.6, topK: 20, topP: 0.95, presencePenalty: 0.5,
        recentIds: recent, uniform: 0.5 });
    });
  });
} finally {
  s.close();
}
