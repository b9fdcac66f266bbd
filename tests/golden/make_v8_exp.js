'use strict';
/*
 * Writes tests/golden/v8_math_exp.json: inputs and outputs of V8's own
 * Math.exp, as IEEE-754 bit patterns in hex.  sample() computes its
 * weights with Math.exp (lib/webgpu-llm/tokenizer.js:165), so these vectors
 * pin the oracle's exp and the GPU kernel's exp to the engine the reference
 * runs on, bit for bit.
 *
 *   node tests/golden/make_v8_exp.js > tests/golden/v8_math_exp.json
 */
var buf = new ArrayBuffer(8);
var f64 = new Float64Array(buf);
var u32 = new Uint32Array(buf);

function hex(x) {
  f64[0] = x;
  return ('00000000' + u32[1].toString(16)).slice(-8) + ('00000000' + u32[0].toString(16)).slice(-8);
}

function fromBits(hi, lo) {
  u32[1] = hi >>> 0;
  u32[0] = lo >>> 0;
  return f64[0];
}

// xorshift32, fixed seed: the vectors are reproducible
var s = 0x2545F491;
function rnd() {
  s ^= s << 13; s >>>= 0;
  s ^= s >>> 17;
  s ^= s << 5; s >>>= 0;
  return s / 4294967296;
}

var xs = [0, -0, 1, -1, 0.5, -0.5, 2, -2, 10, -10, 100, -100, 700, -700, 709.7, 709.8, -745.1, -745.2,
          -708.5, -720, -740, 1e-300, -1e-300, 1e-9, -1e-9, Infinity, -Infinity, NaN,
          Math.LN2 / 2, -Math.LN2 / 2, 1.5 * Math.LN2, -1.5 * Math.LN2, Math.pow(2, -28), -Math.pow(2, -28)];
// neighbours of fdlibm's branch points (high words 0x3fd62e42, 0x3ff0a2b2,
// 0x3e300000, 0x40862e42) on both sides and both signs
[0x3fd62e42, 0x3ff0a2b2, 0x3e300000, 0x40862e42].forEach(function (hi) {
  [hi - 1, hi, hi + 1].forEach(function (h) {
    [0, 1, 0xfefa39ef, 0xffffffff].forEach(function (lo) {
      xs.push(fromBits(h, lo));
      xs.push(fromBits((h | 0x80000000) >>> 0, lo));
    });
  });
});
var i;
// the domain sample() feeds it: (v_i - v_0) / T <= 0
for (i = 0; i < 3000; i++) xs.push(-60 * rnd());
for (i = 0; i < 1000; i++) xs.push(-rnd() * rnd());
// the whole finite range
for (i = 0; i < 1000; i++) xs.push(-745 + 1455 * rnd());
for (i = 0; i < 500; i++) xs.push((rnd() - 0.5) * Math.pow(2, -40 * rnd()));

var cases = xs.map(function (x) { return [hex(x), hex(Math.exp(x))]; });
process.stdout.write(JSON.stringify({
  source: 'Math.exp of Node ' + process.version + ' (V8 ' + process.versions.v8 + ')',
  format: '[input bits, output bits], IEEE-754 binary64, big-endian hex',
  cases: cases
}) + '\n');
