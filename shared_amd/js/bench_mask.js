'use strict';
// Host cost of the grammar mask's wire format, per decode step (no GPU):
// packing a TokenMask into bitmask words from its id list, a MaskBuilder
// cache hit for an equal list rebuilt as a new array, and a packed-words
// mask checked against the words already uploaded.  Usage:
//   node shared_amd/js/bench_mask.js [vocab]
const sas = require('./index.js');

const vocab = parseInt(process.argv[2] || '151936', 10);
function time(name, reps, fn) {
  fn();
  const t0 = process.hrtime.bigint();
  for (let i = 0; i < reps; i++) fn();
  const us = Number(process.hrtime.bigint() - t0) / 1e3 / reps;
  console.log(name.padEnd(58) + us.toFixed(1).padStart(9) + ' us');
  return us;
}
const all = Uint32Array.from({ length: vocab }, function (_, i) { return i; });
const unrestricted = all.filter(function (id) { return id !== 151645 && id % 1000 !== 7; });
const small = Uint32Array.of(1, 2, 3, 42, 9000, 100000 % vocab);
const b = new sas.MaskBuilder(vocab, 64);
const state = { cfg: { text: { vocab: vocab } }, allowedCount: 0, tokenMaskKind: 'all', tokenMaskIds: null,
  lastWords: null, uploads: 0, upload: function () { this.uploads++; } };
console.log('vocab ' + vocab + ', allow list of ' + unrestricted.length + ' ids (an unrestricted Qwen state)');
time('maskFromIds: allow list -> words (conversion)', 200, function () {
  sas.maskFromIds(1, unrestricted, vocab);
});
time('MaskBuilder.allow: the list (packed directly: above 4,096 ids)', 200, function () {
  b.allow(unrestricted);
});
const mid = unrestricted.subarray(0, 4000);
time('maskFromIds: a 4,000-id list', 500, function () { sas.maskFromIds(1, mid, vocab); });
time('MaskBuilder.allow: the same 4,000 ids in a new array (cache hit)', 500, function () { b.allow(mid.slice()); });
time('  of which copying the 4,000 ids', 500, function () { mid.slice(); });
time('MaskBuilder.allow: a 6-id list (cache hit)', 2000, function () { b.allow(Uint32Array.of(1, 2, 3, 42, 9000, 100000 % vocab)); });
time('maskFromIds: a 6-id list', 2000, function () { sas.maskFromIds(1, small, vocab); });
// Qwen's ToolConstraint.mask(): its cached unrestricted() array in a new
// {kind: 'allow'} object every step (tool-constraint.ts:286-293, 653-661)
const constraint = { mask: function () { return { kind: 'allow', tokenIds: unrestricted }; } };
const b2 = new sas.MaskBuilder(vocab, 64);
time('packedToolMask: repeated unrestricted Qwen state (new object)', 2000, function () {
  sas.packedToolMask(constraint, '', null, b2);
});
const w = b.allow(unrestricted);
time('updateTokenMaskState, words equal to the uploaded ones', 2000, function () {
  sas.updateTokenMaskState(state, { kind: 'words', words: Uint32Array.from(w) });
});
console.log('uploads: ' + state.uploads + ' (one for the first call)');
