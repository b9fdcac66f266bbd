'use strict';
// CPU checks of the Node host layer (no GPU): the mask state mirrors the
// reference's updateTokenMaskState behaviour and messages
// (lib/webgpu-llm/token-mask-state.js:8-31, tests/token-mask-state.test.ts:21-46),
// the parameter packer its validation (lib/webgpu-llm/model.js:401-426), and
// the addon's host helpers.  Prints "ok <name>" per check; exits non-zero on
// the first failure.
const assert = require('assert');
const path = require('path');
// SAS_JS_DIR: another build of the module (the sanitizer build in tests/sanitize)
const sas = require(process.env.SAS_JS_DIR || path.join(__dirname, '..', '..', 'shared_amd', 'js'));

function check(name, fn) {
  fn();
  console.log('ok ' + name);
}

function fakeMaskState(vocab) {
  const state = {
    cfg: { text: { vocab: vocab } },
    allowedCount: 0,
    tokenMaskKind: 'all',
    tokenMaskIds: null,
    uploads: [],
    upload: function (w) { this.uploads.push(Uint32Array.from(w)); },
  };
  return state;
}

check('mask uploads once per distinct immutable mask', function () {
  const state = fakeMaskState(32);
  const tokenIds = Uint32Array.of(1, 2, 3);
  const mask = { kind: 'deny', tokenIds: tokenIds };
  sas.updateTokenMaskState(state, mask);
  assert.strictEqual(state.uploads.length, 1);
  sas.updateTokenMaskState(state, mask);
  sas.updateTokenMaskState(state, { kind: 'deny', tokenIds: tokenIds });
  assert.strictEqual(state.uploads.length, 1);
  // a new array with the same ids: the reference uploads it again; its words
  // equal the ones on the device, so this build does not
  sas.updateTokenMaskState(state, { kind: 'deny', tokenIds: Uint32Array.of(1, 2, 3) });
  assert.strictEqual(state.uploads.length, 1);
  sas.updateTokenMaskState(state, { kind: 'deny', tokenIds: Uint32Array.of(1, 2, 4) });
  assert.strictEqual(state.uploads.length, 2);
  sas.updateTokenMaskState(state, undefined);
  assert.strictEqual(state.uploads.length, 2);      // 'all' needs no words
  assert.strictEqual(state.tokenMaskKind, 'all');
  assert.strictEqual(state.allowedCount, 0);
  // deny {1,2,3} over 32 ids: every bit but 1..3
  assert.strictEqual(state.uploads[0][0] >>> 0, (~0xE) >>> 0);
});

check('packed words masks: uploaded once per content, counted', function () {
  const state = fakeMaskState(40);
  const w = new Uint32Array(2);
  w[0] = 0x0000000F; w[1] = 0x81;
  sas.updateTokenMaskState(state, { kind: 'words', words: w });
  assert.strictEqual(state.uploads.length, 1);
  assert.strictEqual(state.allowedTokens, 6);
  sas.updateTokenMaskState(state, { kind: 'words', words: w });
  sas.updateTokenMaskState(state, { kind: 'words', words: Uint32Array.from(w) });
  assert.strictEqual(state.uploads.length, 1);
  sas.updateTokenMaskState(state, { kind: 'allow', tokenIds: Uint32Array.of(0, 1, 2, 3, 32, 39) });
  assert.strictEqual(state.uploads.length, 1);      // the same words as ids
  sas.updateTokenMaskState(state, { kind: 'allow', tokenIds: Uint32Array.of(5) });
  assert.strictEqual(state.uploads.length, 2);
  assert.throws(function () { sas.updateTokenMaskState(state, { kind: 'words', words: new Uint32Array(1) }); },
    /^Error: A words token mask requires Uint32Array words of ceil\(vocab \/ 32\) entries\.$/);
});

check('MaskBuilder: words equal the brute-force masks; equal lists hit its cache', function () {
  const V = 1000;
  const b = new sas.MaskBuilder(V, 16);
  const bits = function (w) { const o = []; for (let i = 0; i < V; i++) if ((w[i >> 5] >>> (i & 31)) & 1) o.push(i); return o; };
  const ids = Uint32Array.of(3, 999, 64, 3, 1000, 500);
  assert.deepStrictEqual(bits(b.allow(ids)), [3, 64, 500, 999]);
  const d = bits(b.deny(ids));
  assert.strictEqual(d.length, V - 4);
  assert.ok(d.indexOf(3) < 0 && d.indexOf(998) >= 0);
  assert.strictEqual(b.count(b.all()), V);
  assert.strictEqual(b.count(b.none()), 0);
  const u = b.or(b.allow(Uint32Array.of(1, 2)), b.allow(Uint32Array.of(2, 7)));
  assert.deepStrictEqual(bits(u), [1, 2, 7]);
  assert.deepStrictEqual(bits(b.and(u, b.deny(Uint32Array.of(2)))), [1, 7]);
  assert.deepStrictEqual(bits(b.andNot(b.all(), b.deny(Uint32Array.of(9, 10)))), [9, 10]);
  const hits = b.hits;
  b.allow(Uint32Array.of(3, 999, 64, 3, 1000, 500));   // a new array, the same ids
  assert.strictEqual(b.hits, hits + 1);
  assert.deepStrictEqual(bits(b.fromTokenMask({ kind: 'deny', tokenIds: Uint32Array.of(0) })).length, V - 1);
  // packedToolMask: a ToolConstraint-like producer's TokenMask, packed once per object
  const cached = { kind: 'deny', tokenIds: Uint32Array.of(5, 6) };
  const tc = { mask: function (raw) { return raw === 'x' ? cached : { kind: 'allow', tokenIds: Uint32Array.of(7) }; } };
  const m1 = sas.packedToolMask(tc, 'x', null, b), m2 = sas.packedToolMask(tc, 'x', null, b);
  assert.strictEqual(m1.kind, 'words');
  assert.strictEqual(m1.words, m2.words);
  assert.deepStrictEqual(bits(sas.packedToolMask(tc, 'y', null, b).words), [7]);
  // Qwen's mask(): the same cached array in a new {kind: 'allow'} object per
  // call (tool-constraint.ts:286-293, 653-661) packs once, a long list too
  const big = Uint32Array.from({ length: 900 }, function (_, i) { return i; });
  const long = new sas.MaskBuilder(V, 16);
  const qwen = { mask: function () { return { kind: 'allow', tokenIds: big }; } };
  const q1 = sas.packedToolMask(qwen, 'a', null, long);
  const misses = long.misses;
  const q2 = sas.packedToolMask(qwen, 'b', null, long);
  assert.strictEqual(q1.words, q2.words);
  assert.strictEqual(long.misses, misses);
  assert.strictEqual(long.count(q1.words), 900);
  // 'all' masks share one array; arrays that are not Uint32Arrays are not memoized
  const all1 = sas.packedToolMask({ mask: function () { return { kind: 'all' }; } }, '', null, long).words;
  const all2 = sas.packedToolMask({ mask: function () { return { kind: 'all' }; } }, '', null, long).words;
  assert.strictEqual(all1, all2);
  assert.strictEqual(long.count(all1), V);
  const plain = [1, 2, 3];
  const p1 = long.allow(plain);
  plain.push(4);
  assert.deepStrictEqual(bits(long.allow(plain)), [1, 2, 3, 4]);
  assert.deepStrictEqual(bits(p1), [1, 2, 3]);
});

check('empty allow mask is kept as an empty constraint', function () {
  const state = fakeMaskState(32);
  sas.updateTokenMaskState(state, { kind: 'allow', tokenIds: new Uint32Array() });
  assert.strictEqual(state.tokenMaskKind, 'allow');
  assert.strictEqual(state.uploads.length, 1);
  assert.strictEqual(state.uploads[0][0], 0);       // no id allowed
  assert.strictEqual(state.allowedTokens, 0);
});

check('mask errors carry the reference messages', function () {
  const state = fakeMaskState(4);
  assert.throws(function () { sas.updateTokenMaskState(state, { kind: 'maybe' }); },
    /^Error: Unknown token mask kind: maybe$/);
  assert.throws(function () { sas.updateTokenMaskState(state, { kind: 'allow', tokenIds: [1, 2] }); },
    /^Error: A allow token mask requires Uint32Array tokenIds\.$/);
  assert.throws(function () { sas.updateTokenMaskState(state, { kind: 'deny', tokenIds: new Uint32Array(5) }); },
    /^Error: Tool constraint has too many token IDs\.$/);
  assert.strictEqual(state.uploads.length, 0);
});

check('allow and deny produce complementary words', function () {
  const ids = Uint32Array.of(0, 31, 32, 99, 150, 7);
  const a = sas.maskFromIds(1, ids, 151);
  const d = sas.maskFromIds(2, ids, 151);
  assert.strictEqual(a.allowed, 6);
  assert.strictEqual(d.allowed, 151 - 6);
  for (let w = 0; w < a.words.length; w++) {
    const valid = w < 4 ? 0xFFFFFFFF : (1 << (151 - 128)) - 1;
    assert.strictEqual((a.words[w] ^ d.words[w]) >>> 0, valid >>> 0, 'word ' + w);
  }
});

check('packer validates stop ids like the reference', function () {
  assert.throws(function () { sas.packSamplerParams({ stopIds: 5 }); }, /^Error: stopIds must be an array$/);
  assert.throws(function () { sas.packSamplerParams({ stopIds: [1, 2, 3, 4, 5] }); },
    /^Error: stopIds supports at most 4 ids$/);
  assert.throws(function () { sas.packSamplerParams({ stopIds: [1.5] }); }, /^Error: invalid stop token id: 1.5$/);
  const p = sas.packSamplerParams({ eosId: 7 });
  assert.deepStrictEqual(p.stopIds, [7]);
  assert.deepStrictEqual(p.paddedStopIds, [7, sas.STOP_PAD, sas.STOP_PAD, sas.STOP_PAD]);
  assert.strictEqual(p.seed, 1);
});

check('packer clamps like model.js:418-423 and lifts the top-k cap to 128', function () {
  const c = sas.packSamplerParams({ temperature: NaN, topP: 3, topK: 0, presencePenalty: 50 }).params;
  assert.strictEqual(c.temperature, 0);
  assert.strictEqual(c.topP, 1);
  assert.strictEqual(c.topK, 1);
  assert.strictEqual(c.presencePenalty, 10);
  assert.strictEqual(sas.packSamplerParams({ topK: 400 }).params.topK, sas.MAX_TOP_K);
  assert.strictEqual(sas.packSamplerParams({}).params.topK, 20);
  assert.strictEqual(sas.packSamplerParams({ temperature: -2 }).params.temperature, 0);
  const g = sas.packSamplerParams({}, { temperature: 0.6, topP: 0.95 }).params;
  assert.strictEqual(g.temperature, 0.6);
  assert.strictEqual(g.topP, 0.95);
});

check('pcg uniform matches the reference hash', function () {
  // kernels.js:91-95, 181: (pcg(seed ^ it * 0x9E3779B9) & 0xFFFFFF) / 2^24
  function pcg(x) {
    let h = (Math.imul(x >>> 0, 747796405) + 2891336453) >>> 0;
    h = Math.imul(((h >>> ((h >>> 28) + 4)) ^ h) >>> 0, 277803737) >>> 0;
    return ((h >>> 22) ^ h) >>> 0;
  }
  const cases = [[1, 0, 0], [12345, 7, 0], [0xDEADBEEF, 99, 3]];
  for (let i = 0; i < cases.length; i++) {
    const s = cases[i][0], it = cases[i][1], row = cases[i][2];
    const x = (s ^ Math.imul(it, 0x9E3779B9) ^ Math.imul(row, 0x85EBCA6B)) >>> 0;
    assert.strictEqual(sas.pcgUniform(s, it, row), (pcg(x) & 0xFFFFFF) / 16777216);
  }
});

check('allowedTokenIds: checked and carried like decodeBatch (model.js:661-666)', function () {
  assert.throws(function () { sas.packSamplerParams({ allowedTokenIds: [1, 2] }); },
    /^TypeError: allowedTokenIds must be a Uint32Array$/);
  const ids = Uint32Array.of(3, 9);
  const p = sas.packSamplerParams({ allowedTokenIds: ids });
  assert.strictEqual(p.allowedTokenIds, ids);                 // identity kept for the upload dedupe
  assert.strictEqual(sas.packSamplerParams({ allowedTokenIds: new Uint32Array() }).allowedTokenIds, null);
  assert.strictEqual(sas.packSamplerParams({}).allowedTokenIds, null);
  // more ids than the vocabulary: the reference's message
  const big = sas.packSamplerParams({ allowedTokenIds: new Uint32Array(11) });
  assert.throws(function () { sas.allowedLists([big], 10, false); },
    /^Error: Tool constraint has too many allowed token IDs\.$/);
  assert.deepStrictEqual(sas.allowedLists([p, sas.packSamplerParams({})], 10, false), [ids, null]);
  assert.throws(function () { sas.allowedLists([p], 10, true); }, /cannot both be given/);
  assert.deepStrictEqual(sas.allowedLists([sas.packSamplerParams({})], 10, true), [null]);
});

check('eos id: Qwen takes the first stop id, Gemma only an explicit eosId', function () {
  assert.strictEqual(sas.packSamplerParams({ stopIds: [7, 9] }).eosId, 7);
  assert.strictEqual(sas.packSamplerParams({}).eosId, sas.STOP_PAD);
  assert.strictEqual(sas.packSamplerParams({ stopIds: [7, 9], eosId: 9 }).eosId, 9);
  const g = sas.PACKER_DEFAULTS.gemma;
  assert.strictEqual(sas.packSamplerParams({ stopIds: [7, 9] }, g).eosId, null);
  assert.strictEqual(sas.packSamplerParams({ stopIds: [7, 9], eosId: 9 }, g).eosId, 9);
  const gp = sas.packSamplerParams({}, g);
  assert.strictEqual(gp.params.temperature, 0.6);
  assert.strictEqual(gp.params.topP, 0.95);
  assert.ok(Number.isInteger(gp.seed) && gp.seed >= 0 && gp.seed <= 0xFFFFFFFF);
});

check('request clamps and defaults (completions.ts:268-273, gemma-completions.ts:212-217)', function () {
  assert.deepStrictEqual(sas.requestSamplingParams({}),
    { temperature: 0.6, topP: 0.95, topK: 20, presencePenalty: 1.5 });
  assert.deepStrictEqual(sas.requestSamplingParams({}, 'gemma'),
    { temperature: 1.0, topP: 0.95, topK: 20, presencePenalty: 0 });
  assert.deepStrictEqual(sas.requestSamplingParams({ temperature: 5, top_p: 0.01, top_k: 300.6, presence_penalty: -1 }),
    { temperature: 2, topP: 0.05, topK: 128, presencePenalty: 0 });
  assert.strictEqual(sas.requestSamplingParams({ top_k: 0.4 }).topK, 1);
  assert.strictEqual(sas.requestSamplingParams({ top_k: 40.5 }).topK, 41);   // Math.round
  assert.ok(Number.isNaN(sas.requestSamplingParams({ temperature: NaN }).temperature));
  // NaN then meets the packer's non-finite rule: greedy for Qwen, 0.6 for Gemma
  assert.strictEqual(sas.packSamplerParams(sas.requestSamplingParams({ temperature: NaN })).params.temperature, 0);
  assert.strictEqual(sas.packSamplerParams(sas.requestSamplingParams({ temperature: NaN }, 'gemma'),
    sas.PACKER_DEFAULTS.gemma).params.temperature, 0.6);
});

check('penalty window: last 512, rewind by sampled count (token-mask-state.test.ts:58-70)', function () {
  const w = new sas.PenaltyWindow();
  [1, 2, 3, 4, 5].forEach(function (x) { w.note(x); });
  w.rewind(2);
  assert.deepStrictEqual(w.genIds, [1, 2, 3]);
  w.rewind(0);
  assert.deepStrictEqual(w.genIds, [1, 2, 3]);
  const big = new sas.PenaltyWindow();
  for (let i = 0; i < 600; i++) big.note(i);
  const r = big.recent();
  assert.strictEqual(r.length, 512);
  assert.strictEqual(r[0], 88);
  assert.strictEqual(r[511], 599);
  assert.ok(big.recentSet().has(599) && !big.recentSet().has(87));
  big.reset();
  assert.strictEqual(big.recent().length, 0);
});

check('a sampler needs a HIP device and says so', function () {
  assert.throws(function () { return new sas.Sampler(0); }, /no HIP device/);
});

check('lmHeadSample describes its head and rejects bad ones on the host', function () {
  const self = Object.create(sas.Sampler.prototype);
  const fake = function (ptr) { const b = Object.create(sas.DeviceBuffer.prototype); b.ptr = ptr; return b; };
  const hd = self._describeHead({ rows: 2, head: { hidden: fake(16n), weight: fake(4096n), dim: 512, outLogits: fake(8192n) } });
  assert.deepStrictEqual(hd, { dim: 512, hiddenStride: 512, weightStride: 512, format: 0, hidden: 16n, weight: 4096n,
    outLogits: 8192n });
  // GGUF heads: the format code and the row's bytes as the default stride
  const q6 = self._describeHead({ rows: 1, head: { hidden: fake(16n), weight: fake(64n), dim: 2560, format: 'q6_k' } });
  assert.strictEqual(q6.format, 3);
  assert.strictEqual(q6.weightStride, 2100);
  assert.strictEqual(self._describeHead({ rows: 1, head: { hidden: fake(16n), weight: fake(64n), dim: 512, format: 'q8_0' } })
    .weightStride, 544);
  assert.strictEqual(self._describeHead({ rows: 1, head: { hidden: fake(16n), weight: fake(64n), dim: 512, format: 'q4_0' } })
    .weightStride, 288);
  assert.throws(function () { self._describeHead({ rows: 1, head: { hidden: fake(16n), weight: fake(64n), dim: 256, format: 'q5_k' } }); },
    /head.format must be one of bf16, q8_0, q4_0, q6_k/);
  const hs = self._describeHead({ rows: 1, head: { hidden: fake(16n), weight: fake(32n), dim: 256, hiddenStride: 300, weightStride: 264 } });
  assert.strictEqual(hs.hiddenStride, 300);
  assert.strictEqual(hs.weightStride, 264);
  assert.strictEqual(hs.outLogits, undefined);
  assert.throws(function () { self._describeHead({ rows: 1 }); }, TypeError);
  assert.throws(function () { self._describeHead({ rows: 1, head: { hidden: fake(16n), weight: fake(32n), dim: 1.5 } }); }, RangeError);
  assert.throws(function () { self._describeHead({ rows: 1, head: { hidden: fake(16n), weight: new Uint16Array(256), dim: 256 } }); },
    /head.weight must be a DeviceBuffer/);
  assert.throws(function () { self._describeHead({ rows: 2, head: { hidden: new Float32Array(256), weight: fake(32n), dim: 256 } }); },
    /fewer than rows \* hiddenStride/);
  assert.throws(function () { self._describeHead({ rows: 1, head: { hidden: [1, 2], weight: fake(32n), dim: 256 } }); }, TypeError);
  assert.strictEqual(sas.LMH_MAX_ROWS, 4);
});

check('version names the target', function () {
  assert.ok(/^shared_amd_sampler \d+ gfx950$/.test(sas.version()));
});
console.log('all ok');
