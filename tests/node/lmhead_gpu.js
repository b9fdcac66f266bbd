'use strict';
// GPU run of Sampler#lmHeadSample, driven by tests/test_gpu_node.py: reads a
// case directory (meta.json, the hidden states, the bf16 head and the usual
// sampling inputs), runs the fused head through the JS API (host and device
// hidden states, sync and async, with and without out_logits) and writes
// each result back for the Python side to compare with the oracle.
const fs = require('fs');
const path = require('path');
const sas = require(path.join(__dirname, '..', '..', 'shared_amd', 'js'));

const dir = process.argv[2];
function read(name, Type) {
  const f = path.join(dir, name);
  if (!fs.existsSync(f)) return null;
  const b = fs.readFileSync(f);
  const copy = new Uint8Array(b.byteLength);
  copy.set(b);
  return new Type(copy.buffer);
}
function write(name, typed) {
  fs.writeFileSync(path.join(dir, name), Buffer.from(typed.buffer, typed.byteOffset, typed.byteLength));
}
function step(msg) { console.log('[node] ' + msg); }

const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
const rows = meta.rows;
const vocab = meta.vocab;
const dim = meta.dim;
const p = meta.params;
const params = {
  temperature: p.temperature, topK: p.top_k, topP: p.top_p, repetitionPenalty: p.repetition_penalty,
  presencePenalty: p.presence_penalty, frequencyPenalty: p.frequency_penalty, softcap: p.softcap,
};
const hidden = read('hidden.f32', Float32Array);
const weight = read('weight.u16', Uint16Array);
const mask = read('mask.u32', Uint32Array);
const hist = read('hist.u32', Uint32Array);
const histOff = read('hist_off.i32', Int32Array);
const uniforms = read('uniforms.f64', Float64Array);
const history = [];
for (let r = 0; r < rows; r++) history.push(hist.subarray(histOff[r], histOff[r + 1]));

async function main() {
  const s = new sas.Sampler(0);
  try {
    const w = s.alloc(weight.byteLength).upload(weight);
    const logits = s.alloc(rows * vocab * 4);
    const base = { rows: rows, vocab: vocab, mask: mask, params: params, history: history, uniforms: uniforms };

    const a = s.lmHeadSample(Object.assign({ full: true, head: { hidden: hidden, weight: w, dim: dim, outLogits: logits } }, base));
    write('lmh_sync_ids.u32', a.ids);
    write('lmh_sync_probs.f64', a.probs);
    write('lmh_sync_cand.u32', a.candIds);
    write('lmh_logits.f32', logits.download(new Float32Array(rows * vocab)));
    step('lmHeadSample (host hidden, out_logits) done');

    const hdev = s.alloc(hidden.byteLength).upload(hidden);
    const b = await s.lmHeadSampleAsync(Object.assign({ head: { hidden: hdev, weight: w, dim: dim } }, base));
    write('lmh_async_ids.u32', b.ids);
    step('lmHeadSampleAsync (device hidden) done');

    // the unfused path over the head's own logits
    const c = s.sampleRows(Object.assign({ logits: logits }, base));
    write('lmh_unfused_ids.u32', c.ids);
    step('sampleRows over the written logits done');

    // a GGUF Q6_K head (the Qwen head's format) with the same rows and inputs
    const q6k = read('q6k.u8', Uint8Array);
    if (q6k) {
      const wq = s.alloc(q6k.byteLength).upload(q6k);
      const qlog = s.alloc(rows * vocab * 4);
      const qd = await s.lmHeadSampleAsync(Object.assign({ full: true,
        head: { hidden: hidden, weight: wq, dim: dim, format: 'q6_k', outLogits: qlog } }, base));
      write('lmh_q6k_ids.u32', qd.ids);
      write('lmh_q6k_probs.f64', qd.probs);
      write('lmh_q6k_logits.f32', qlog.download(new Float32Array(rows * vocab)));
      let bad = '';
      try {
        s.lmHeadSample(Object.assign({ head: { hidden: hidden, weight: wq, dim: dim, format: 'q5_k' } }, base));
      } catch (e) { bad = String(e.message); }
      if (!/format/.test(bad)) throw new Error('an unknown head format did not throw: ' + bad);
      wq.free();
      qlog.free();
      step('lmHeadSampleAsync (Q6_K head) done');
    }

    let threw = '';
    try {
      s.lmHeadSample(Object.assign({ head: { hidden: hdev, weight: w, dim: dim + 64 } }, base));
    } catch (e) {
      threw = String(e.message);
    }
    if (!/dim|multiple/.test(threw)) throw new Error('a dim that is not a multiple of 256 did not throw: ' + threw);
    step('bad dim rejected: ' + threw);
    hdev.free();
    logits.free();
    w.free();
  } finally {
    await s.close();
  }
}

main().then(function () { step('ok'); }, function (e) { console.error(e && e.stack || e); process.exit(1); });
