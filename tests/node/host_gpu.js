'use strict';
// GPU run of the Node host layer, driven by tests/test_gpu_node.py: reads a
// case directory (meta.json + raw little-endian arrays), samples it through
// every entry of the JS API and writes each result back next to the inputs
// for the Python side to compare with the oracle.  Prints a line per step.
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
const p = meta.params;
const params = {
  temperature: p.temperature, topK: p.top_k, topP: p.top_p, repetitionPenalty: p.repetition_penalty,
  presencePenalty: p.presence_penalty, frequencyPenalty: p.frequency_penalty, softcap: p.softcap,
};
const logits = read('logits.f32', Float32Array);
const mask = read('mask.u32', Uint32Array);
const hist = read('hist.u32', Uint32Array);
const histOff = read('hist_off.i32', Int32Array);
const uniforms = read('uniforms.f64', Float64Array);
let history = null;
if (hist) {
  history = [];
  for (let r = 0; r < rows; r++) history.push(hist.subarray(histOff[r], histOff[r + 1]));
}

async function main() {
  const s = new sas.Sampler(0);
  try {
    s.reserve(rows, vocab);
    const base = { rows: rows, vocab: vocab, mask: mask, params: params, history: history, uniforms: uniforms };

    const a = s.sampleRows(Object.assign({ logits: logits, full: true }, base));
    write('js_sync_ids.u32', a.ids);
    write('js_sync_probs.f64', a.probs);
    write('js_sync_cand.u32', a.candIds);
    write('js_sync_counts.i32', a.counts);
    step('sampleRows (host logits) done');

    const b = await s.sampleRowsAsync(Object.assign({ logits: logits }, base));
    write('js_async_ids.u32', b.ids);
    step('sampleRowsAsync done');

    const dev = s.alloc(logits.byteLength).upload(logits);
    const c = s.sampleRows(Object.assign({}, base, { logits: dev }));
    write('js_dev_ids.u32', c.ids);
    dev.free();
    step('sampleRows (device-resident logits) done');

    // per-row params as an array: the same values for every row
    const perRow = [];
    for (let r = 0; r < rows; r++) perRow.push(params);
    const d = s.sampleRows(Object.assign({}, base, { logits: logits, params: perRow }));
    write('js_rowparams_ids.u32', d.ids);
    step('sampleRows (per-row params) done');

    const allow = read('tokmask_allow.u32', Uint32Array);
    if (allow) {
      const state = s.createTokenMaskState(vocab);
      const tm = { kind: 'allow', tokenIds: allow };
      sas.updateTokenMaskState(state, tm);
      sas.updateTokenMaskState(state, tm);          // same object: no second upload
      if (state.uploads !== 1) throw new Error('mask uploaded ' + state.uploads + ' times');
      const e = s.sampleRows(Object.assign({}, base, { logits: logits, mask: state }));
      write('js_tokmask_ids.u32', e.ids);
      const e2 = s.sampleRows(Object.assign({}, base, { logits: logits, mask: tm }));
      write('js_tokmask2_ids.u32', e2.ids);
      step('sampleRows (TokenMask) done');
    }

    if (allow) {
      // the packed producer: MaskBuilder words (set algebra on words) through
      // updateTokenMaskState, then packedToolMask over a ToolConstraint-shaped
      // object whose mask() wraps one cached array in a new object per call
      // (tool-constraint.ts:286-293, 653-661): packed once, uploaded once
      const mb = new sas.MaskBuilder(vocab, 8);
      const wstate = s.createTokenMaskState(vocab);
      const words = mb.andNot(mb.allow(allow), mb.allow(allow.subarray(0, 100)));
      sas.updateTokenMaskState(wstate, { kind: 'words', words: words });
      const g1 = s.sampleRows(Object.assign({}, base, { logits: logits, mask: wstate }));
      write('js_words_ids.u32', g1.ids);
      const constraint = { mask: function () { return { kind: 'allow', tokenIds: allow }; } };
      const pm1 = sas.packedToolMask(constraint, '', null, mb);
      sas.updateTokenMaskState(wstate, pm1);
      const up = wstate.uploads;
      const pm2 = sas.packedToolMask(constraint, '', null, mb);
      if (pm2.words !== pm1.words) throw new Error('packedToolMask packed the same tokenIds again');
      sas.updateTokenMaskState(wstate, pm2);
      if (wstate.uploads !== up) throw new Error('the same words were uploaded again');
      const g2 = s.sampleRows(Object.assign({}, base, { logits: logits, mask: wstate }));
      write('js_tool_ids.u32', g2.ids);
      step('sampleRows (MaskBuilder words, packedToolMask) done');
    }

    if (allow) {
      // Qwen's SampleParams.allowedTokenIds (model.js:661-666): one list for
      // every row, then rows with and without one
      const qp = Object.assign({}, params, { allowedTokenIds: allow });
      const f = s.sampleRows(Object.assign({}, base, { logits: logits, mask: null, params: qp }));
      write('js_allowed_ids.u32', f.ids);
      const mixed = [];
      for (let r = 0; r < rows; r++) mixed.push(r % 2 ? params : qp);
      const f2 = s.sampleRows(Object.assign({}, base, { logits: logits, mask: null, params: mixed }));
      write('js_allowed_mixed_ids.u32', f2.ids);
      let msg = '';
      try {
        s.sampleRows(Object.assign({}, base, { logits: logits, mask: null,
          params: Object.assign({}, params, { allowedTokenIds: new Uint32Array(vocab + 1) }) }));
      } catch (e) { msg = e.message; }
      if (msg !== 'Tool constraint has too many allowed token IDs.') throw new Error('allow-list check: ' + msg);
      step('sampleRows (allowedTokenIds) done');
    }

    // decodeBatch's result shape over PenaltyWindows seeded with the history;
    // the stop ids are two of the tokens the rows draw
    const want = read('want_ids.u32', Uint32Array);
    if (want && history) {
      const windows = history.map(function (h) {
        const w = new sas.PenaltyWindow(512);
        for (let i = 0; i < h.length; i++) w.note(h[i]);
        return w;
      });
      const sp = Object.assign({}, params, { stopIds: [want[0], want[1]] });
      const res = s.decodeRows(Object.assign({}, base, { logits: logits, params: sp, history: null, windows: windows }));
      fs.writeFileSync(path.join(dir, 'js_decode.json'), JSON.stringify({
        results: res, lens: windows.map(function (w) { return w.genIds.length; }),
        last: windows.map(function (w) { return w.genIds[w.genIds.length - 1]; }),
      }));
      step('decodeRows done');
    }

    // a synchronous call while an async one is pending throws; close() after
    // an async call waits for it, then the handle is closed
    {
      const s2 = new sas.Sampler(0);
      const pend = s2.sampleRowsAsync(Object.assign({ logits: logits }, base));
      let msg = '';
      try { s2.sampleRows(Object.assign({ logits: logits }, base)); } catch (e) { msg = e.message; }
      if (!/pending/.test(msg)) throw new Error('sync during async did not throw: ' + msg);
      const pend2 = s2.sampleRowsAsync(Object.assign({ logits: logits }, base, { uniforms: uniforms }));
      const closing = s2.close();
      msg = '';
      try { s2.sampleRowsAsync(Object.assign({ logits: logits }, base)); } catch (e) { msg = e.message; }
      if (msg !== 'sampler is closed') throw new Error('call after close did not throw: ' + msg);
      const r1 = await pend;
      const r2 = await pend2;
      await closing;
      if (s2._h !== null) throw new Error('handle not released after close');
      write('js_conc1_ids.u32', r1.ids);
      write('js_conc2_ids.u32', r2.ids);
      step('async queue, sync guard and deferred close done');
    }

    const candsPath = path.join(dir, 'cands.json');
    if (fs.existsSync(candsPath)) {
      const cc = JSON.parse(fs.readFileSync(candsPath, 'utf8'));
      const buf = new ArrayBuffer(cc.ids.length * 8);
      const ids = new Uint32Array(buf);
      const vals = new Float32Array(buf);
      for (let i = 0; i < cc.ids.length; i++) {
        ids[i * 2] = cc.ids[i];
        vals[i * 2 + 1] = cc.vals[i];
      }
      const out = [];
      for (let t = 0; t < cc.uniforms.length; t++) {
        out.push(s.sample({ ids: ids, vals: vals }, {
          temperature: cc.temperature, topK: cc.topK, topP: cc.topP, presencePenalty: cc.presencePenalty,
          recentIds: new Set(cc.recent), uniform: cc.uniforms[t],
        }));
      }
      fs.writeFileSync(path.join(dir, 'js_compat.json'), JSON.stringify(out));
      step('sample(cands, opts) done');
    }

    const vmeta = path.join(dir, 'verify.json');
    if (fs.existsSync(vmeta)) {
      const v = JSON.parse(fs.readFileSync(vmeta, 'utf8'));
      const opts = {
        target: read('v_target.f32', Float32Array), draft: read('v_draft.f32', Float32Array), vocab: v.vocab,
        seqs: v.seqs, draftLen: v.drafts, draftIds: read('v_ids.u32', Uint32Array),
        uniforms: read('v_u.f64', Float64Array), temperature: v.temperature, mask: read('v_mask.u32', Uint32Array),
      };
      const r1 = s.verify(opts);
      write('js_v_tokens.u32', r1.tokens);
      write('js_v_acc.i32', r1.accepted);
      const r2 = await s.verifyAsync(opts);
      write('js_v2_tokens.u32', r2.tokens);
      step('verify done');
    }
  } finally {
    s.close();
  }
  step('all done');
}

main().catch(function (e) {
  console.error(e && e.stack ? e.stack : e);
  process.exit(1);
});
