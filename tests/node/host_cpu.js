'use strict';
// CPU checks of the Node host layer (no GPU): the mask state mirrors the
// reference's updateTokenMaskState behaviour and messages
// (lib/webgpu-llm/token-mask-state.js:8-31, tests/token-mask-state.test.ts:21-46),
// the parameter packer its validation (lib/webgpu-llm/model.js:401-426), and
// the addon's host helpers.  Prints "ok <name>" per check; exits non-zero on
// the first failure.
const assert = require('assert');
const path = require('path');
const sas = require(path.join(__dirname, '..', '..', 'shared_amd', 'js'));

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
  sas.updateTokenMaskState(state, { kind: 'deny', tokenIds: Uint32Array.of(1, 2, 3) });
  assert.strictEqual(state.uploads.length, 2);
  sas.updateTokenMaskState(state, undefined);
  assert.strictEqual(state.uploads.length, 2);      // 'all' needs no words
  assert.strictEqual(state.tokenMaskKind, 'all');
  assert.strictEqual(state.allowedCount, 0);
  // deny {1,2,3} over 32 ids: every bit but 1..3
  assert.strictEqual(state.uploads[0][0] >>> 0, (~0xE) >>> 0);
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

check('a sampler needs a HIP device and says so', function () {
  assert.throws(function () { return new sas.Sampler(0); }, /no HIP device/);
});

check('version names the target', function () {
  assert.ok(/^shared_amd_sampler \d+ gfx950$/.test(sas.version()));
});
console.log('all ok');
