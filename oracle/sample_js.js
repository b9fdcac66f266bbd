'use strict';
/*
 * sample_js.js - Node restatement of the reference sampling path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline that
 * bench.py times on the host cores.  The product never loads it.
 *
 * It keeps the reference's two-stage CPU structure:
 *   1. per 1024-id block: mask test per element (kernels.js:1422-1426), the
 *      history penalties, then the block's top-K by (value desc, id asc)
 *      with K = max(20, top_k) (kernels.js:1428-1448 emits top-20);
 *   2. sample() over the concatenated block lists exactly as
 *      lib/webgpu-llm/tokenizer.js:151-178 does, with the host-supplied
 *      uniform in place of Math.random() and the penalties already applied.
 * Arithmetic is V8's: doubles, Math.exp, a stable Array.prototype.sort.
 * Plain ES2017 so it runs on Node 12 (no ?? / ?. / private fields).
 */
var fs = require('fs');
var path = require('path');

var BLOCK = 1024;
var MAX_TOP_K = 128;

function clampTopK(k) {
  if (!(k >= 1)) return 1;
  return k > MAX_TOP_K ? MAX_TOP_K : Math.floor(k);
}

/* tanh rounded once to fp32 from a double evaluation (the same expression
 * the C oracle and the GPU use); Math.exp is fdlibm's exp in V8. */
function tanhF32(x) {
  var ax = Math.abs(x), r;
  if (ax !== ax) return x;
  if (ax >= 9.5) r = 1;
  else if (ax < 0.001953125) {
    var x2 = ax * ax;
    r = ax * (1 - x2 * (1 / 3 - x2 * (2 / 15 - x2 * (17 / 315))));
  } else {
    var t = Math.exp(2 * ax);
    r = (t - 1) / (t + 1);
  }
  r = Math.fround(r);
  return (x < 0 || (x === 0 && 1 / x < 0)) ? -r : r;
}

function softcap(x, cap) {
  var q = Math.fround(x / cap);
  return Math.fround(cap * tanhF32(q));
}

function penalize(v, count, p) {
  if (count === 0) return v;
  var r = p.repetition_penalty;
  v = v > 0 ? v / r : v * r;
  v = v - p.frequency_penalty * count;
  v = v - p.presence_penalty;
  return v;
}

/* Stage 1 for one row: the concatenated per-block candidate lists. */
function blockCandidates(logits, off, vocab, mask, moff, counts, p, K) {
  var cand = [];
  var bi = new Int32Array(K), bv = new Float64Array(K);
  for (var base = 0; base < vocab; base += BLOCK) {
    var n = 0;
    var end = Math.min(vocab, base + BLOCK);
    for (var g = base; g < end; g++) {
      if (mask && !((mask[moff + (g >>> 5)] >>> (g & 31)) & 1)) continue;
      var x = logits[off + g];
      if (p.softcap > 0) x = softcap(x, Math.fround(p.softcap));
      if (x !== x) continue;
      var v = counts ? penalize(x, counts[g], p) : x;
      if (v !== v) continue;
      // insertion into the block's descending list; equal values keep the
      // earlier (lower) id first, as the strict '>' scan of kernels.js:1433
      if (n === K && !(v > bv[K - 1])) continue;
      var j = n < K ? n++ : K - 1;
      while (j > 0 && v > bv[j - 1]) { bv[j] = bv[j - 1]; bi[j] = bi[j - 1]; j--; }
      bv[j] = v; bi[j] = g;
    }
    for (var t = 0; t < n; t++) cand.push([bi[t], bv[t]]);
  }
  return cand;
}

/* Stage 2: tokenizer.js:151-178 with U for Math.random(). */
function sampleCands(cand, temperature, topK, topP, U) {
  cand.sort(function (a, b) { return b[1] - a[1]; });
  var k = Math.min(topK, cand.length);
  if (temperature <= 0) return { id: cand[0][0], k: 0, cut: 0, probs: [], ids: [] };
  var mx = cand[0][1];
  var probs = [], sum = 0;
  for (var i = 0; i < k; i++) {
    var pr = Math.exp((cand[i][1] - mx) / temperature);
    probs.push(pr); sum += pr;
  }
  var cum = 0, cut = k;
  for (i = 0; i < k; i++) {
    cum += probs[i] / sum;
    if (cum >= topP) { cut = i + 1; break; }
  }
  var r = U * probs.slice(0, cut).reduce(function (a, b) { return a + b; }, 0);
  var id = cand[cut - 1][0];
  for (i = 0; i < cut; i++) { r -= probs[i]; if (r <= 0) { id = cand[i][0]; break; } }
  var ids = [], pn = [];
  for (i = 0; i < k; i++) { ids.push(cand[i][0]); pn.push(probs[i] / sum); }
  return { id: id, k: k, cut: cut, probs: pn, ids: ids };
}

/* One row end to end.  Returns {id, k, cut, probs, ids}. */
function sampleRow(inp, r, p, counts) {
  var greedy = !(p.temperature > 0);
  var kreq = greedy ? 1 : clampTopK(p.top_k);
  var K = Math.max(20, kreq);
  var cand = blockCandidates(inp.logits, r * inp.stride, inp.vocab, inp.mask,
                             r * inp.maskStride, counts, p, K);
  if (cand.length === 0) return { id: 0xFFFFFFFF, k: 0, cut: 0, probs: [], ids: [] };
  return sampleCands(cand, greedy ? 0 : p.temperature, kreq, p.top_p,
                     inp.uniforms ? inp.uniforms[r] : 0);
}

function historyCounts(inp, r, scratch) {
  if (!inp.hist) return null;
  var a = inp.histOff[r], b = inp.histOff[r + 1];
  if (b <= a) return null;
  scratch.fill(0);
  for (var i = a; i < b; i++) { var id = inp.hist[i]; if (id < inp.vocab) scratch[id]++; }
  return scratch;
}

function runRows(inp, r0, r1, out) {
  var scratch = inp.hist ? new Uint32Array(inp.vocab) : null;
  for (var r = r0; r < r1; r++) {
    var counts = historyCounts(inp, r, scratch);
    var res = sampleRow(inp, r, inp.params, counts);
    out.ids[r] = res.id >>> 0;
    out.counts[2 * r] = res.k; out.counts[2 * r + 1] = res.cut;
    for (var i = 0; i < res.k; i++) {
      out.probs[r * MAX_TOP_K + i] = res.probs[i];
      out.cand[r * MAX_TOP_K + i] = res.ids[i];
    }
  }
}

/* ------------------------------------------------------------- file I/O -- */
/* A case directory holds meta.json plus raw little-endian arrays:
 *   logits.f32 [rows*stride], mask.u32 [rows*maskStride] (optional),
 *   hist.u32 + hist_off.i32 (optional), uniforms.f64 (optional). */
function readArray(dir, name, Ctor, shared) {
  var f = path.join(dir, name);
  if (!fs.existsSync(f)) return null;
  var buf = fs.readFileSync(f);
  var bytes = buf.length;
  var sab = shared ? new SharedArrayBuffer(bytes) : new ArrayBuffer(bytes);
  new Uint8Array(sab).set(buf);
  return new Ctor(sab);
}

function loadCase(dir, shared) {
  var meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
  return {
    meta: meta,
    rows: meta.rows, vocab: meta.vocab, stride: meta.stride || meta.vocab,
    maskStride: meta.mask_stride || Math.ceil(meta.vocab / 32),
    params: meta.params,
    logits: readArray(dir, 'logits.f32', Float32Array, shared),
    mask: readArray(dir, 'mask.u32', Uint32Array, shared),
    hist: readArray(dir, 'hist.u32', Uint32Array, shared),
    histOff: readArray(dir, 'hist_off.i32', Int32Array, shared),
    uniforms: readArray(dir, 'uniforms.f64', Float64Array, shared)
  };
}

function makeOut(rows, shared) {
  function mk(Ctor, n) {
    var b = shared ? new SharedArrayBuffer(n * Ctor.BYTES_PER_ELEMENT) : new ArrayBuffer(n * Ctor.BYTES_PER_ELEMENT);
    return new Ctor(b);
  }
  var out = { ids: mk(Uint32Array, rows), counts: mk(Int32Array, 2 * rows),
              probs: mk(Float64Array, rows * MAX_TOP_K), cand: mk(Uint32Array, rows * MAX_TOP_K) };
  out.cand.fill(0xFFFFFFFF);  // unused candidate slots hold the no-token id
  return out;
}

function writeOut(dir, out) {
  fs.writeFileSync(path.join(dir, 'out_ids.u32'), Buffer.from(out.ids.buffer));
  fs.writeFileSync(path.join(dir, 'out_counts.i32'), Buffer.from(out.counts.buffer));
  fs.writeFileSync(path.join(dir, 'out_probs.f64'), Buffer.from(out.probs.buffer));
  fs.writeFileSync(path.join(dir, 'out_cand.u32'), Buffer.from(out.cand.buffer));
}

/* ------------------------------------------------------------------ CLI -- */
/* node sample_js.js <case_dir> [--threads N] [--repeat R]
 * Writes out_*.* into the case dir and prints one JSON line of timings. */
function main() {
  var args = process.argv.slice(2);
  var dir = args[0];
  var threads = 1, repeat = 1;
  for (var i = 1; i < args.length; i++) {
    if (args[i] === '--threads') threads = parseInt(args[++i], 10);
    else if (args[i] === '--repeat') repeat = parseInt(args[++i], 10);
  }
  var os = require('os');
  var cpus = os.cpus();
  if (threads <= 0) threads = cpus.length;
  if (threads === 1) {
    var inp = loadCase(dir, false);
    var out = makeOut(inp.rows, false);
    var times = [];
    for (var rep = 0; rep < repeat; rep++) {
      var t0 = process.hrtime.bigint();
      runRows(inp, 0, inp.rows, out);
      times.push(Number(process.hrtime.bigint() - t0) / 1e9);
    }
    writeOut(dir, out);
    report(times, inp.rows, 1, cpus);
    return;
  }
  var wt = require('worker_threads');
  var inp2 = loadCase(dir, true);
  var out2 = makeOut(inp2.rows, true);
  var workers = [], ready = 0, done = 0, times2 = [], t1 = 0n, rep2 = 0;
  var n = Math.min(threads, Math.max(1, inp2.rows));
  function go() {
    done = 0;
    t1 = process.hrtime.bigint();
    for (var w = 0; w < n; w++) workers[w].postMessage('go');
  }
  for (var w = 0; w < n; w++) {
    var r0 = Math.floor(inp2.rows * w / n), r1 = Math.floor(inp2.rows * (w + 1) / n);
    var wk = new wt.Worker(__filename, { workerData: { inp: inp2, out: out2, r0: r0, r1: r1 } });
    wk.on('message', function (m) {
      if (m === 'ready') { if (++ready === n) go(); return; }
      if (++done === n) {
        times2.push(Number(process.hrtime.bigint() - t1) / 1e9);
        if (++rep2 < repeat) { go(); return; }
        for (var q = 0; q < n; q++) workers[q].postMessage('exit');
        writeOut(dir, out2);
        report(times2, inp2.rows, n, cpus);
      }
    });
    workers.push(wk);
  }
}

function report(times, rows, threads, cpus) {
  var sorted = times.slice().sort(function (a, b) { return a - b; });
  var med = sorted[Math.floor(sorted.length / 2)];
  process.stdout.write(JSON.stringify({
    rows: rows, threads: threads, repeat: times.length, median_s: med, min_s: sorted[0],
    rows_per_s: rows / med, cpu_model: cpus.length ? cpus[0].model : '', host_cpus: cpus.length,
    node: process.version
  }) + '\n');
}

function workerMain() {
  var wt = require('worker_threads');
  var d = wt.workerData;
  d.inp.params = d.inp.meta.params;
  wt.parentPort.on('message', function (m) {
    if (m === 'exit') { process.exit(0); }
    runRows(d.inp, d.r0, d.r1, d.out);
    wt.parentPort.postMessage('done');
  });
  wt.parentPort.postMessage('ready');
}

module.exports = { sampleRow: sampleRow, sampleCands: sampleCands, blockCandidates: blockCandidates,
                   penalize: penalize, softcap: softcap, loadCase: loadCase, runRows: runRows,
                   makeOut: makeOut, MAX_TOP_K: MAX_TOP_K };

if (require.main === module) {
  var wtm = null;
  try { wtm = require('worker_threads'); } catch (e) { wtm = null; }
  if (wtm && !wtm.isMainThread) workerMain(); else main();
}
