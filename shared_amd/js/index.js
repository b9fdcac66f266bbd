'use strict';
// Node host side of the MI355X sampling path: the sampler / token-mask API of
// lib/webgpu-llm kept as a drop-in, over the C ABI through the N-API addon.
//
//   TokenMask + updateTokenMaskState  <- lib/webgpu-llm/tool-constraint.ts:39-42,
//                                        lib/webgpu-llm/token-mask-state.js:8-31
//   packSamplerParams                 <- lib/webgpu-llm/model.js:401-426,
//                                        lib/webgpu-llm/gemma-model.js:900-919
//   Sampler#sample(cands, opts)       <- sample(), lib/webgpu-llm/tokenizer.js:151-178
//   Sampler#sampleRows                <- the topk + sampler WGSL pair,
//                                        lib/webgpu-llm/kernels.js:65-201, 1389-1449
//   Sampler#lmHeadSample              <- the decode head and the topk pass after it,
//                                        lib/webgpu-llm/model.js:466-471, gemma-model.js:786-799
//   Sampler#verify                    <- acceptSpec, lib/webgpu-llm/kernels.js:211-369
//   Sampler#decodeRows                <- the sampling tail of decodeBatch, lib/webgpu-llm/model.js:656-742,
//                                        lib/webgpu-llm/gemma-model.js:921-992 ({ids, fed, eos, stopped, stopId})
//   PenaltyWindow                     <- genIds / recentSet / rewindDecode, lib/webgpu-llm/model.js:386-399,
//                                        lib/webgpu-llm/gemma-model.js:817-839
//   requestSamplingParams             <- request defaults and ranges, lib/completions.ts:268-273,
//                                        lib/gemma-completions.ts:212-217
//
// Grammar state stays on the host: a TokenMask becomes the packed u32
// bitmask (bit id & 31 of word id >> 5 = allowed) once per distinct
// immutable mask, and only those words cross to the GPU.  Written for
// Node >= 12 (no optional chaining, no class fields).

const addon = require('./sas_napi.node');

const MAX_STOP_IDS = 4;
const STOP_PAD = 0xFFFFFFFF;
const PARAMS_BYTES = addon.PARAMS_BYTES;
const KIND_CODE = { all: addon.MASK_ALL, allow: addon.MASK_ALLOW, deny: addon.MASK_DENY };

function orDefault(v, d) { return v === undefined || v === null ? d : v; }

function popcount32(x) {
  x = x - ((x >>> 1) & 0x55555555);
  x = (x & 0x33333333) + ((x >>> 2) & 0x33333333);
  return (((x + (x >>> 4)) & 0x0F0F0F0F) * 0x01010101) >>> 24;
}

function sameWords(a, b) {
  return !!a && !!b && (a === b || addon.u32Equal(a, b));
}

/**
 * Apply an immutable TokenMask to a mask state, as the reference does: the
 * same checks and messages (token-mask-state.js:9-20), and nothing is
 * re-uploaded for the same kind and the same Uint32Array object (:21).
 * A changed mask is packed into bitmask words on the host and handed to
 * state.upload(words), unless the words equal the ones last uploaded (a
 * grammar state rebuilt as a new but equal list).  Kind 'all' needs no
 * words: rows sample unmasked.  Beyond the reference's kinds, a producer
 * that already has packed words passes {kind: 'words', words} (ceil(vocab /
 * 32) words, bit id & 31 of word id >> 5 = allowed): no id list is built
 * or converted.
 */
function updateTokenMaskState(state, mask) {
  const kind = orDefault(mask ? mask.kind : undefined, 'all');
  if (kind !== 'all' && kind !== 'allow' && kind !== 'deny' && kind !== 'words') {
    throw new Error('Unknown token mask kind: ' + kind);
  }
  const vocab = state.cfg.text.vocab;
  const nwords = Math.ceil(vocab / 32);
  if (kind === 'words') {
    const w = mask.words;
    if (!(w instanceof Uint32Array) || w.length < nwords) {
      throw new Error('A words token mask requires Uint32Array words of ceil(vocab / 32) entries.');
    }
    if (state.tokenMaskKind === 'words' && w === state.tokenMaskIds) return;
    const words = w.length === nwords ? w : w.subarray(0, nwords);
    let allowed = 0;
    for (let i = 0; i < nwords; i++) allowed += popcount32(words[i]);
    if (!sameWords(words, state.lastWords)) {
      state.upload(words);
      state.lastWords = Uint32Array.from(words);
    }
    state.allowedTokens = allowed;
    state.allowedCount = allowed;
    state.tokenMaskKind = kind;
    state.tokenMaskIds = w;
    return;
  }
  const ids = kind === 'all' ? null : (mask ? mask.tokenIds : undefined);
  if (kind !== 'all' && !(ids instanceof Uint32Array)) {
    throw new Error('A ' + kind + ' token mask requires Uint32Array tokenIds.');
  }
  const count = ids ? ids.length : 0;
  if (count > vocab) {
    throw new Error('Tool constraint has too many token IDs.');
  }
  if (kind === state.tokenMaskKind && ids === state.tokenMaskIds) return;
  if (kind !== 'all') {
    const packed = addon.maskFromIds(KIND_CODE[kind], ids, vocab);
    if (!sameWords(packed.words, state.lastWords)) {
      state.upload(packed.words);
      state.lastWords = packed.words;
    }
    state.allowedTokens = packed.allowed;
  } else {
    state.allowedTokens = vocab;
    state.lastWords = null;
  }
  state.allowedCount = count;
  state.tokenMaskKind = kind;
  state.tokenMaskIds = ids;
}

/**
 * Packed-bitmask producer for grammar code (the host side of the mask's
 * wire format): masks as words from the start, set algebra on words, and a
 * content-keyed cache so that a grammar state rebuilt each step as a new but
 * equal id list costs a hash and a compare, not a conversion.  Every result
 * is a Uint32Array of ceil(vocab / 32) words, to be treated as immutable (a
 * cache hit returns the same array, which updateTokenMaskState then skips
 * by identity); wrap it as {kind: 'words', words} for updateTokenMaskState
 * or pass it as a sampleRows mask.
 */
class MaskBuilder {
  constructor(vocab, cacheSize) {
    if (!(vocab >= 1 && vocab <= addon.MAX_VOCAB)) throw new RangeError('vocab must be in [1, MAX_VOCAB]');
    this.vocab = vocab;
    this.nwords = Math.ceil(vocab / 32);
    this.cacheSize = cacheSize || 64;
    this.cache = new Map();   // content key -> {ids copy, words}; insertion order = age
    this.hits = 0;
    this.misses = 0;
    this._all = addon.maskFromIds(addon.MASK_ALL, null, vocab).words;
    // words by id-list object: a TokenMask's tokenIds are immutable and
    // compared by identity (token-mask-state.js:21), so the same array
    // packs once, whatever its length
    this._byIds = new WeakMap();
  }
  /** Every id allowed (a fresh copy). */
  all() { return Uint32Array.from(this._all); }
  /** No id allowed. */
  none() { return new Uint32Array(this.nwords); }
  /** Only `ids` (ids past the vocabulary are ignored). */
  allow(ids) { return this._fromIds(addon.MASK_ALLOW, toU32(ids), ids); }
  /** Every id but `ids`. */
  deny(ids) { return this._fromIds(addon.MASK_DENY, toU32(ids), ids); }
  /** The words of a TokenMask ({kind: 'all' | 'allow' | 'deny', tokenIds} or {kind: 'words', words}). */
  fromTokenMask(mask) {
    const kind = orDefault(mask ? mask.kind : undefined, 'all');
    if (kind === 'all') return this.all();
    if (kind === 'words') return Uint32Array.from(mask.words.subarray(0, this.nwords));
    if (kind !== 'allow' && kind !== 'deny') throw new Error('Unknown token mask kind: ' + kind);
    return kind === 'allow' ? this.allow(mask.tokenIds) : this.deny(mask.tokenIds);
  }
  or(a, b) { return this._zip(a, b, function (x, y) { return x | y; }); }
  and(a, b) { return this._zip(a, b, function (x, y) { return x & y; }); }
  andNot(a, b) { return this._zip(a, b, function (x, y) { return x & ~y; }); }
  /** Number of allowed ids. */
  count(w) {
    let n = 0;
    for (let i = 0; i < this.nwords; i++) n += popcount32(w[i]);
    return n;
  }
  _zip(a, b, op) {
    const out = new Uint32Array(this.nwords);
    for (let i = 0; i < this.nwords; i++) out[i] = op(a[i], b[i]) >>> 0;
    const tail = this.vocab & 31;
    if (tail) out[this.nwords - 1] &= (1 << tail) - 1 >>> 0;
    return out;
  }
  _fromIds(code, ids, original) {
    // the same Uint32Array again (a TokenMask's tokenIds): its words, with
    // no work per id.  Other lists (arrays, sets) are converted per call.
    const owner = original instanceof Uint32Array ? original : null;
    let byCode = owner ? this._byIds.get(owner) : undefined;
    if (byCode && byCode[code]) {
      this.hits++;
      return byCode[code];
    }
    let words;
    if (ids.length > 4096) {
      // past a few thousand ids, hashing and comparing a list costs as much
      // as packing it (about 1 ns per id each): pack it directly
      this.misses++;
      words = addon.maskFromIds(code, ids, this.vocab).words;
    } else {
      const key = code + ':' + addon.idsKey(ids);
      const hit = this.cache.get(key);
      if (hit && sameWords(hit.ids, ids)) {
        this.cache.delete(key);
        this.cache.set(key, hit);
        this.hits++;
        words = hit.words;
      } else {
        this.misses++;
        words = addon.maskFromIds(code, ids, this.vocab).words;
        this.cache.set(key, { ids: Uint32Array.from(ids), words: words });
        if (this.cache.size > this.cacheSize) this.cache.delete(this.cache.keys().next().value);
      }
    }
    if (owner) {
      if (!byCode) {
        byCode = {};
        this._byIds.set(owner, byCode);
      }
      byCode[code] = words;
    }
    return words;
  }
}

/**
 * The reference's ToolConstraint (tool-constraint.ts:653-661) as a packed
 * mask producer: its TokenMask for `raw` as {kind: 'words', words} through
 * `builder`; the same TokenMask object (its cached unrestricted masks) is
 * packed once.
 */
function packedToolMask(constraint, raw, parseArguments, builder) {
  const mask = constraint.mask(raw, parseArguments);
  const kind = orDefault(mask ? mask.kind : undefined, 'all');
  let words;
  if (kind === 'all') {
    // one immutable all-allowed array for every 'all' mask
    words = builder._allShared || (builder._allShared = builder.all());
  } else if (kind === 'allow' || kind === 'deny') {
    // keyed by the tokenIds array: Qwen's mask() wraps its cached
    // unrestricted() list in a new {kind: 'allow'} object every step
    // (tool-constraint.ts:286-293, 653-661), and the same array is packed once
    words = builder.fromTokenMask(mask);
  } else {
    const memo = builder._byMask || (builder._byMask = new WeakMap());
    words = memo.get(mask);
    if (!words) {
      words = builder.fromTokenMask(mask);
      memo.set(mask, words);
    }
  }
  return { kind: 'words', words: words };
}

/**
 * Packer defaults of the two model families.  Qwen (model.js:401-426):
 * greedy unless a temperature is given, seed 1, and the first stop id is the
 * end-of-sequence id.  Gemma (gemma-model.js:900-919): temperature 0.6,
 * top-p 0.95, a random seed, and eos only when eosId is given.
 */
// LM head formats (sas_lm_head.format): bf16, and the GGUF block types the
// reference loads (gguf/parser.js:29-36) with their values and bytes per block.
const HEAD_FORMATS = {
  bf16: { id: 0, values: 1, bytesPer: 0 },
  q8_0: { id: 1, values: 32, bytesPer: 34 },
  q4_0: { id: 2, values: 32, bytesPer: 18 },
  q6_k: { id: 3, values: 256, bytesPer: 210 },
};

const PACKER_DEFAULTS = {
  qwen: { temperature: 0, topP: 1, topK: 20, seed: 1, eosFromStops: true },
  gemma: { temperature: 0.6, topP: 0.95, topK: 20, seed: null, eosFromStops: false },
};

/**
 * The reference packer's validation and clamps (model.js:401-426): stop ids
 * are checked and padded, and every numeric field is clamped by
 * sas_clamp_params.  top_k may go to 128 here (the request API's range,
 * completions.ts:271) where the reference GPU path stopped at 20.
 * `defaults` is PACKER_DEFAULTS.qwen (the default) or .gemma, or a partial
 * object of the same fields.  SampleParams.allowedTokenIds (model.d.ts:15)
 * is checked and carried through: a non-empty Uint32Array constrains the
 * draw to those ids; an empty one or none leaves the row unconstrained, as
 * the reference's allowedCount of 0 does (model.js:660-666).
 */
function packSamplerParams(sp, defaults) {
  sp = sp || {};
  defaults = defaults || PACKER_DEFAULTS.qwen;
  const rawStopIds = sp.stopIds !== undefined ? sp.stopIds
    : (sp.eosId !== undefined ? [sp.eosId] : []);
  if (!Array.isArray(rawStopIds)) throw new Error('stopIds must be an array');
  if (rawStopIds.length > MAX_STOP_IDS) throw new Error('stopIds supports at most ' + MAX_STOP_IDS + ' ids');
  const stopIds = rawStopIds.map(function (id) {
    if (!Number.isInteger(id)) throw new Error('invalid stop token id: ' + id);
    return id >>> 0;
  });
  const allowed = sp.allowedTokenIds;
  if (allowed !== undefined && allowed !== null && !(allowed instanceof Uint32Array)) {
    throw new TypeError('allowedTokenIds must be a Uint32Array');
  }
  const pick = function (name, d) { return Number.isFinite(sp[name]) ? sp[name] : orDefault(defaults[name], d); };
  const params = addon.clampParams({
    temperature: pick('temperature', 0),
    topP: pick('topP', 1),
    topK: Number.isFinite(sp.topK) ? Math.floor(sp.topK) : orDefault(defaults.topK, 20),
    presencePenalty: pick('presencePenalty', 0),
    repetitionPenalty: pick('repetitionPenalty', 1),
    frequencyPenalty: pick('frequencyPenalty', 0),
    softcap: pick('softcap', 0),
  });
  let seed;
  if (sp.seed !== undefined && sp.seed !== null) seed = sp.seed >>> 0;
  else if (defaults.seed === null) seed = (Math.random() * 0xffffffff) >>> 0;
  else seed = orDefault(defaults.seed, 1) >>> 0;
  const padded = [];
  for (let i = 0; i < MAX_STOP_IDS; i++) padded.push(i < stopIds.length ? stopIds[i] : STOP_PAD);
  const eosFromStops = defaults.eosFromStops !== undefined ? defaults.eosFromStops : true;
  let eosId = null;
  if (sp.eosId !== undefined) eosId = sp.eosId >>> 0;
  else if (eosFromStops) eosId = stopIds.length ? stopIds[0] : STOP_PAD;
  return {
    params: params, seed: seed, stopIds: stopIds, paddedStopIds: padded, stopSet: new Set(stopIds),
    eosId: eosId, allowedTokenIds: allowed && allowed.length ? allowed : null,
  };
}

/**
 * The rows' allowedTokenIds lists (null = unconstrained) from packed
 * params, checked as decodeBatch checks them (model.js:661-664): a list
 * longer than the vocabulary throws the reference's message.  A list cannot
 * be combined with a mask (the reference's two model families take one or
 * the other).
 */
function allowedLists(packed, vocab, hasMask) {
  const lists = packed.map(function (p) { return p.allowedTokenIds; });
  let any = false;
  for (let i = 0; i < lists.length; i++) {
    if (lists[i] === null) continue;
    any = true;
    if (lists[i].length > vocab) throw new Error('Tool constraint has too many allowed token IDs.');
  }
  if (any && hasMask) throw new Error('allowedTokenIds and mask cannot both be given');
  return lists;
}

/**
 * Request-level sampling defaults and ranges of the completion endpoints:
 * Qwen (completions.ts:268-273) temperature 0.6 in [0, 2], top_p 0.95 in
 * [0.05, 1], top_k 20 rounded in [1, 128], presence 1.5 in [0, 2]; Gemma
 * (gemma-completions.ts:212-217) the same with temperature 1.0 and presence
 * 0.  Math.min/Math.max as the reference's clamp(), so NaN stays NaN and the
 * packer then applies its own non-finite defaults.
 */
function requestSamplingParams(request, grammar) {
  request = request || {};
  const clamp = function (v, lo, hi) { return Math.min(hi, Math.max(lo, v)); };
  const gemma = grammar === 'gemma';
  return {
    temperature: clamp(orDefault(request.temperature, gemma ? 1.0 : 0.6), 0, 2),
    topP: clamp(orDefault(request.top_p, 0.95), 0.05, 1),
    topK: Math.round(clamp(orDefault(request.top_k, 20), 1, 128)),
    presencePenalty: clamp(orDefault(request.presence_penalty, gemma ? 0 : 1.5), 0, 2),
  };
}

/**
 * The penalty window of one sequence: the tokens generated this turn
 * (model.js:386-389; gemma-model.js:817-827), the last `size` of them as
 * the history the penalties use (recentSet), and rewindDecode's removal of
 * discarded tokens (gemma-model.js:834-839).  Stop tokens never enter it.
 */
class PenaltyWindow {
  constructor(size) {
    this.size = size || 512;
    this.genIds = [];
  }
  reset() { this.genIds = []; }
  note(id) { this.genIds.push(id >>> 0); }
  /** The ids the next step penalizes: the last `size` generated tokens. */
  recent() { return Uint32Array.from(this.genIds.slice(-this.size)); }
  recentSet() { return new Set(this.genIds.slice(-this.size)); }
  /** rewindDecode(count, sampledCount): drop the last sampledCount tokens. */
  rewind(sampledCount) {
    const n = Math.max(0, Math.floor(sampledCount || 0));
    if (n) this.genIds.splice(Math.max(0, this.genIds.length - n), n);
  }
}

/** sas_params layout: five doubles, a float softcap, an int32 top_k (48 bytes). */
function writeParams(view, offset, p) {
  view.setFloat64(offset + 0, p.temperature, true);
  view.setFloat64(offset + 8, p.topP, true);
  view.setFloat64(offset + 16, p.repetitionPenalty, true);
  view.setFloat64(offset + 24, p.presencePenalty, true);
  view.setFloat64(offset + 32, p.frequencyPenalty, true);
  view.setFloat32(offset + 40, p.softcap, true);
  view.setInt32(offset + 44, p.topK, true);
}

function toU32(list) {
  if (list instanceof Uint32Array) return list;
  if (list instanceof Set) return Uint32Array.from(list);
  return Uint32Array.from(list || []);
}

class DeviceBuffer {
  constructor(sampler, bytes) {
    this.sampler = sampler;
    this.bytes = bytes;
    this.ptr = addon.alloc(sampler._idle('alloc'), bytes);
  }
  upload(typed) {
    if (typed.byteLength > this.bytes) throw new RangeError('upload larger than the device buffer');
    addon.copy(this.sampler._idle('upload'), this.ptr, typed, 0);
    return this;
  }
  download(typed) {
    if (typed.byteLength > this.bytes) throw new RangeError('download larger than the device buffer');
    addon.copy(this.sampler._idle('download'), this.ptr, typed, 1);
    return typed;
  }
  free() {
    if (this.ptr !== null && this.sampler._h !== null) addon.free(this.sampler._idle('free'), this.ptr);
    this.ptr = null;
  }
}

class Sampler {
  /** A sampler bound to HIP device `device`; throws when no device exists. */
  constructor(device) {
    this._h = addon.create(device || 0);
    this._scratch = {};
    this._queue = Promise.resolve();
    this._pending = 0;      // async calls queued or running
    this._running = false;  // the queue is executing one of them now
    this._inWorker = false; // ... and its launch is on a libuv worker thread
    this._closing = null;   // close() requested while async calls were pending
  }

  _handle() {
    if (this._h === null) throw new Error('sampler is closed');
    return this._h;
  }

  // The handle for a synchronous call.  A handle runs one call at a time
  // (its scratch and stream are shared): while async calls are pending, a
  // synchronous one would run beside them, so it throws; after close() was
  // asked for, every new call throws.  The queued call's own host steps
  // (before and after its worker) run with _running set and pass.
  _idle(what) {
    const h = this._handle();
    if (this._running && !this._inWorker) return h;
    if (this._closing) throw new Error('sampler is closed');
    if (this._pending > 0) {
      throw new Error('Sampler: ' + what + ' called while an async call is pending; await it first');
    }
    return h;
  }

  // Run an addon async call (a promise from a libuv worker) as the queue's
  // current job, flagging the worker phase.
  _worker(promise) {
    const self = this;
    this._inWorker = true;
    return promise.then(function (v) { self._inWorker = false; return v; },
      function (e) { self._inWorker = false; throw e; });
  }

  // Queue fn (which returns a promise) behind every earlier async call.
  _enqueue(fn) {
    const self = this;
    this._handle();
    if (this._closing) throw new Error('sampler is closed');
    this._pending++;
    const run = function () {
      self._running = true;
      let p;
      try {
        p = Promise.resolve(fn());
      } catch (e) {
        p = Promise.reject(e);
      }
      return p.then(function (v) { self._running = false; self._pending--; return v; },
        function (e) { self._running = false; self._pending--; throw e; });
    };
    const p = this._queue.then(run, run);
    this._queue = p.then(function () {}, function () {});
    return p;
  }

  _destroy() {
    if (this._h === null) return;
    const names = Object.keys(this._scratch);
    for (let i = 0; i < names.length; i++) {
      const b = this._scratch[names[i]];
      if (b.ptr !== null) addon.free(this._h, b.ptr);
      b.ptr = null;
    }
    this._scratch = {};
    addon.destroy(this._h);
    this._h = null;
  }

  /**
   * Release the handle.  With async calls pending, the handle stays alive
   * until they settle and the returned promise resolves after the release;
   * new calls throw from now on.
   */
  close() {
    if (this._h === null) return Promise.resolve();
    if (this._closing) return this._closing;
    if (this._pending > 0) {
      const self = this;
      this._closing = this._queue.then(function () { self._destroy(); });
      return this._closing;
    }
    this._destroy();
    return Promise.resolve();
  }

  // Pre-sizes the handle's device scratch (sas_reserve_for): calls of at
  // most these shapes then allocate nothing.  opts: {histIds, lmHeadRows,
  // verifySeqs, verifyDraftLen} (all 0 by default).
  reserve(rows, vocab, opts) {
    const o = opts || {};
    addon.reserve(this._idle('reserve'), rows, vocab, o.histIds || 0, o.lmHeadRows || 0, o.verifySeqs || 0,
      o.verifyDraftLen || 0);
  }

  /** Device memory owned by the caller (e.g. the LM head's logits). */
  alloc(bytes) { return new DeviceBuffer(this, bytes); }

  synchronize() { addon.synchronize(this._idle('synchronize')); }

  // Grow-only per-name scratch, so steady-state calls allocate nothing.
  _buf(name, bytes) {
    const have = this._scratch[name];
    if (have && have.bytes >= bytes) return have;
    if (have) have.free();
    const b = new DeviceBuffer(this, Math.max(256, bytes));
    this._scratch[name] = b;
    return b;
  }

  /**
   * Mask state that mirrors the reference's (cfg.text.vocab, tokenMaskKind,
   * tokenMaskIds, allowedCount) plus the device words it uploads to.
   */
  createTokenMaskState(vocab) {
    const self = this;
    const words = this.alloc(Math.ceil(vocab / 32) * 4);
    return {
      cfg: { text: { vocab: vocab } },
      allowedCount: 0,
      allowedTokens: vocab,
      tokenMaskKind: 'all',
      tokenMaskIds: null,
      lastWords: null,
      words: words,
      uploads: 0,
      upload: function (w) { words.upload(w); this.uploads++; },
      sampler: self,
    };
  }

  // The sas_rows descriptor of opts.  With `step` the history (the device
  // ring) and the uniforms (the device draw from each row's seed) are left
  // out: sas_sample_step brings them.
  _describe(opts, step) {
    const rows = opts.rows;
    const vocab = opts.vocab;
    const stride = orDefault(opts.stride, vocab);
    const d = { rows: rows, vocab: vocab, logitsStride: stride };
    // logits: device buffer (resident), or a host Float32Array staged up
    // (a step loop sets them per step)
    if (step || opts.head) {
      d.logits = null;
      if (opts.head) d.logitsStride = 0;
    } else if (opts.logits instanceof DeviceBuffer) {
      d.logits = opts.logits.ptr;
    } else if (opts.logits instanceof Float32Array) {
      d.logits = this._buf('logits', opts.logits.byteLength).upload(opts.logits).ptr;
    } else {
      throw new TypeError('logits must be a DeviceBuffer or a Float32Array');
    }
    // mask: a token-mask state (one grammar state for every row), a
    // TokenMask, host words [rows][ceil(vocab/32)], or a DeviceBuffer of them
    const nwords = Math.ceil(vocab / 32);
    const m = opts.mask;
    if (m && m.cfg && m.words) {
      if (m.tokenMaskKind !== 'all') { d.mask = m.words.ptr; d.maskStride = 0; }
    } else if (m && m.kind !== undefined) {
      if (m.kind !== 'all') {
        const st = this._maskState || (this._maskState = this.createTokenMaskState(vocab));
        if (st.cfg.text.vocab !== vocab) {
          st.words.free();
          this._maskState = this.createTokenMaskState(vocab);
        }
        updateTokenMaskState(this._maskState, m);
        d.mask = this._maskState.words.ptr;
        d.maskStride = 0;
      }
    } else if (m instanceof Uint32Array) {
      d.mask = this._buf('mask', m.byteLength).upload(m).ptr;
      d.maskStride = m.length === nwords ? 0 : nwords;
    } else if (m instanceof DeviceBuffer) {
      d.mask = m.ptr;
      d.maskStride = orDefault(opts.maskStride, nwords);
    }
    // params: one SampleParams for every row, or one per row
    const ps = Array.isArray(opts.params) ? opts.params : null;
    const packed = ps ? ps.map(function (p) { return packSamplerParams(p, opts.defaults); })
      : [packSamplerParams(opts.params, opts.defaults)];
    // SampleParams.allowedTokenIds (the Qwen path, model.js:661-666): each
    // distinct Uint32Array becomes an allow bitmask once
    const lists = allowedLists(packed, vocab, d.mask !== undefined);
    const firstList = lists.find(function (x) { return x !== null; });
    if (firstList !== undefined) {
      const shared = lists.every(function (x) { return x === firstList; });
      if (shared) {
        let st = this._allowState;
        if (!st || st.cfg.text.vocab !== vocab) {
          if (st) st.words.free();
          st = this._allowState = this.createTokenMaskState(vocab);
        }
        updateTokenMaskState(st, { kind: 'allow', tokenIds: firstList });
        d.mask = st.words.ptr;
        d.maskStride = 0;
      } else {
        // rows with different lists (rows without one are unconstrained)
        const cache = this._allowWords || (this._allowWords = new WeakMap());
        const allWords = addon.maskFromIds(addon.MASK_ALL, null, vocab).words;
        const words = new Uint32Array(rows * nwords);
        for (let r = 0; r < rows; r++) {
          const list = lists[r];
          let w = allWords;
          if (list !== null) {
            const hit = cache.get(list);
            if (hit && hit.vocab === vocab) {
              w = hit.words;
            } else {
              w = addon.maskFromIds(addon.MASK_ALLOW, list, vocab).words;
              cache.set(list, { vocab: vocab, words: w });
            }
          }
          words.set(w, r * nwords);
        }
        d.mask = this._buf('mask', words.byteLength).upload(words).ptr;
        d.maskStride = nwords;
      }
    }
    if (ps) {
      if (ps.length !== rows) throw new RangeError('params must have one entry per row');
      const ab = new ArrayBuffer(rows * PARAMS_BYTES);
      const view = new DataView(ab);
      for (let r = 0; r < rows; r++) writeParams(view, r * PARAMS_BYTES, packed[r].params);
      d.rowParams = this._buf('params', ab.byteLength).upload(new Uint8Array(ab)).ptr;
      d.params = packed[0].params;
      // the packer knows every row's values: without a softcap anywhere the
      // library may use its cheaper kernel variant
      d.rowHints = packed.every(function (p) { return !(p.params.softcap > 0); }) ? addon.HINT_NO_SOFTCAP : 0;
    } else {
      d.params = packed[0].params;
    }
    if (step) {
      d.outIds = this._buf('ids', rows * 4).ptr;
      return { desc: d, packed: packed };
    }
    // history: per-row lists (Array / Uint32Array / Set), or recentIds for every row
    let hist = opts.history;
    if (!hist && opts.windows) {
      if (opts.windows.length !== rows) throw new RangeError('windows must have one PenaltyWindow per row');
      hist = opts.windows.map(function (w) { return w.recent(); });
    }
    if (!hist && opts.recentIds) {
      hist = [];
      for (let r = 0; r < rows; r++) hist.push(opts.recentIds);
    }
    if (hist) this._history(d, hist, rows, 'row');
    // uniforms: host-supplied U per row, else the reference GPU sampler's
    // PCG draw from each row's seed (kernels.js:181, 320)
    let u = opts.uniforms;
    if (!u) {
      u = new Float64Array(rows);
      const it = orDefault(opts.iteration, 0) >>> 0;
      for (let r = 0; r < rows; r++) u[r] = addon.pcgUniform(packed[ps ? r : 0].seed, it, r);
    }
    if (!(u instanceof Float64Array) || u.length < rows) throw new TypeError('uniforms must be a Float64Array[rows]');
    d.uniforms = this._buf('uniforms', rows * 8).upload(u).ptr;
    d.outIds = this._buf('ids', rows * 4).ptr;
    if (opts.full) {
      d.outProbs = this._buf('probs', rows * addon.MAX_TOP_K * 8).ptr;
      d.outCandIds = this._buf('candIds', rows * addon.MAX_TOP_K * 4).ptr;
      d.outCounts = this._buf('counts', rows * 8).ptr;
      d.outFlags = this._buf('flags', rows * 4).ptr;
    }
    return { desc: d, packed: packed };
  }

  // Per-row (or per-sequence) id lists as the CSR history of descriptor d.
  _history(d, hist, rows, what) {
    if (hist.length !== rows) throw new RangeError('history must have one list per ' + what);
    const hl = hist.map(toU32);
    const offs = new Int32Array(rows + 1);
    for (let r = 0; r < rows; r++) {
      if (hl[r].length > addon.MAX_HISTORY) {
        throw new RangeError('history of ' + what + ' ' + r + ' holds ' + hl[r].length + ' ids; at most ' +
          addon.MAX_HISTORY + ' are supported');
      }
      if (offs[r] + hl[r].length > 0x7FFFFFFF) throw new RangeError('histories exceed 2^31 - 1 ids');
      offs[r + 1] = offs[r] + hl[r].length;
    }
    const flat = new Uint32Array(Math.max(1, offs[rows]));
    for (let r = 0; r < rows; r++) flat.set(hl[r], offs[r]);
    d.histIds = this._buf('hist', flat.byteLength).upload(flat).ptr;
    d.histCount = flat.length;
    d.histOffsets = this._buf('histOffsets', offs.byteLength).upload(offs).ptr;
  }

  _collect(opts, packed) {
    const rows = opts.rows;
    const ids = this._scratch.ids.download(new Uint32Array(rows));
    const stopped = [];
    const stopId = [];
    for (let r = 0; r < rows; r++) {
      const set = packed[packed.length > 1 ? r : 0].stopSet;
      const hit = set.has(ids[r]);
      stopped.push(hit);
      stopId.push(hit ? ids[r] : null);
    }
    const out = { ids: ids, stopped: stopped, stopId: stopId };
    if (opts.full) {
      out.probs = this._scratch.probs.download(new Float64Array(rows * addon.MAX_TOP_K));
      out.candIds = this._scratch.candIds.download(new Uint32Array(rows * addon.MAX_TOP_K));
      out.counts = this._scratch.counts.download(new Int32Array(rows * 2));
      out.flags = this._scratch.flags.download(new Uint32Array(rows));
    }
    return out;
  }

  /**
   * One token per row.  opts: {logits, rows, vocab, stride?, mask?, params,
   * history? | recentIds?, uniforms? | seeds via params, iteration?, full?}.
   * Returns {ids: Uint32Array, stopped, stopId[, probs, candIds, counts, flags]}.
   */
  sampleRows(opts) {
    this._idle('sampleRows');
    const r = this._describe(opts);
    addon.sample(this._handle(), r.desc);
    return this._collect(opts, r.packed);
  }

  /**
   * sampleRows with the launch and the wait on a worker thread.  Async calls
   * queue behind each other; synchronous calls throw until they settle.
   */
  sampleRowsAsync(opts) {
    const self = this;
    return this._enqueue(function () {
      const r = self._describe(opts);
      return self._worker(addon.sampleAsync(self._handle(), r.desc))
        .then(function () { return self._collect(opts, r.packed); });
    });
  }

  // The sas_lm_head descriptor of opts.head: {hidden, weight, dim, format?,
  // hiddenStride?, weightStride?, outLogits?}.  format: 'bf16' (default:
  // bits [vocab][weightStride elements]) or a GGUF type, 'q8_0', 'q4_0',
  // 'q6_k' (blocks [vocab][weightStride bytes], the row's bytes by
  // default).  The head must be device-resident; the hidden states may be a
  // host Float32Array [rows][hiddenStride], staged up per call.
  _describeHead(opts) {
    const h = opts.head;
    if (!h || typeof h !== 'object') throw new TypeError('head must be {hidden, weight, dim}');
    const dim = h.dim;
    if (!Number.isInteger(dim) || dim <= 0) throw new RangeError('head.dim must be a positive integer');
    const fmt = orDefault(h.format, 'bf16');
    if (!Object.prototype.hasOwnProperty.call(HEAD_FORMATS, fmt)) {
      throw new RangeError('head.format must be one of ' + Object.keys(HEAD_FORMATS).join(', '));
    }
    const code = HEAD_FORMATS[fmt];
    const rowDefault = code.bytesPer ? dim / code.values * code.bytesPer : dim;
    const hd = { dim: dim, hiddenStride: orDefault(h.hiddenStride, dim), weightStride: orDefault(h.weightStride, rowDefault),
      format: code.id };
    if (h.hidden instanceof DeviceBuffer) {
      hd.hidden = h.hidden.ptr;
    } else if (h.hidden instanceof Float32Array) {
      if (h.hidden.length < opts.rows * hd.hiddenStride) throw new RangeError('head.hidden holds fewer than rows * hiddenStride values');
      hd.hidden = this._buf('hidden', h.hidden.byteLength).upload(h.hidden).ptr;
    } else {
      throw new TypeError('head.hidden must be a DeviceBuffer or a Float32Array');
    }
    if (!(h.weight instanceof DeviceBuffer)) throw new TypeError('head.weight must be a DeviceBuffer');
    hd.weight = h.weight.ptr;
    if (h.outLogits !== undefined && h.outLogits !== null) {
      if (!(h.outLogits instanceof DeviceBuffer)) throw new TypeError('head.outLogits must be a DeviceBuffer');
      hd.outLogits = h.outLogits.ptr;
    }
    return hd;
  }

  /**
   * The LM head with the sampling step fused: logits = head.weight (bf16)
   * times head.hidden (f32) for each row, summed in the library's fixed
   * order, then sampled as sampleRows samples them.  opts as sampleRows
   * without logits, plus head: {hidden, weight, dim, hiddenStride?,
   * weightStride?, outLogits?}.  rows <= LMH_MAX_ROWS.
   */
  lmHeadSample(opts) {
    this._idle('lmHeadSample');
    const hd = this._describeHead(opts);
    const r = this._describe(opts);
    addon.lmHeadSample(this._handle(), r.desc, hd);
    return this._collect(opts, r.packed);
  }

  lmHeadSampleAsync(opts) {
    const self = this;
    return this._enqueue(function () {
      const hd = self._describeHead(opts);
      const r = self._describe(opts);
      return self._worker(addon.lmHeadSampleAsync(self._handle(), r.desc, hd))
        .then(function () { return self._collect(opts, r.packed); });
    });
  }

  // decodeBatch's per-row result for one step (model.js:727-741,
  // gemma-model.js:976-991), with each window's genIds mirror.
  _decodeResults(opts, out, packed) {
    const res = [];
    for (let r = 0; r < opts.rows; r++) {
      const pk = packed[packed.length > 1 ? r : 0];
      const id = out.ids[r];
      const stopped = pk.stopSet.has(id);
      if (opts.windows && !stopped && id !== addon.NO_TOKEN) opts.windows[r].note(id);
      res.push({ ids: [id], fed: 1, eos: stopped && pk.eosId !== null && id === pk.eosId, stopped: stopped,
        stopId: stopped ? id : null });
    }
    return res;
  }

  /**
   * One decode step over every row with decodeBatch's result shape
   * (model.d.ts:23-29): an array of {ids, fed, eos, stopped, stopId}, one
   * per row.  opts as sampleRows, plus windows: a PenaltyWindow per row whose
   * last tokens are the row's history and which receives the row's token
   * unless it is a stop id (model.js:733-734).
   */
  decodeRows(opts) {
    this._idle('decodeRows');
    const r = this._describe(opts);
    addon.sample(this._handle(), r.desc);
    return this._decodeResults(opts, this._collect(opts, r.packed), r.packed);
  }

  decodeRowsAsync(opts) {
    const self = this;
    return this._enqueue(function () {
      const r = self._describe(opts);
      return self._worker(addon.sampleAsync(self._handle(), r.desc))
        .then(function () { return self._decodeResults(opts, self._collect(opts, r.packed), r.packed); });
    });
  }

  // The device state of a k-step loop (kernels.js:63-200 per row): zeroed
  // {stopped, iteration}, the sampled tokens, the fed-back tokens (seeded
  // with opts.firstTokens), the penalty rings (seeded from opts.windows as
  // model.js:391-399 seeds its ring), the padded stop ids and the seeds.
  _stepState(opts, packed, k) {
    const rows = opts.rows;
    const W = Math.floor(orDefault(opts.windowSize, opts.windows && opts.windows.length ? opts.windows[0].size : 512));
    if (!(W >= 1 && W <= addon.MAX_HISTORY)) throw new RangeError('windowSize must be in [1, ' + addon.MAX_HISTORY + ']');
    const pk = function (r) { return packed[packed.length > 1 ? r : 0]; };
    const ring = new Uint32Array(rows * (1 + W));
    if (opts.windows) {
      if (opts.windows.length !== rows) throw new RangeError('windows must have one PenaltyWindow per row');
      for (let r = 0; r < rows; r++) {
        const g = opts.windows[r].genIds;
        const n = g.length;
        const base = r * (1 + W);
        ring[base] = n;
        for (let i = Math.max(0, n - W); i < n; i++) ring[base + 1 + (i % W)] = g[i];
      }
    }
    const stops = new Uint32Array(rows * 4);
    const seeds = new Uint32Array(rows);
    for (let r = 0; r < rows; r++) {
      stops.set(pk(r).paddedStopIds, r * 4);
      seeds[r] = pk(r).seed;
    }
    const next = new Uint32Array(rows);
    if (opts.firstTokens) {
      const f = toU32(opts.firstTokens);
      if (f.length !== rows) throw new RangeError('firstTokens must have one id per row');
      next.set(f);
    }
    return {
      state: this._buf('stState', rows * 8).upload(new Uint32Array(rows * 2)).ptr,
      sampled: this._buf('stSampled', rows * k * 4).ptr, maxSteps: k,
      nextTokens: this._buf('stNext', rows * 4).upload(next).ptr,
      ring: this._buf('stRing', ring.byteLength).upload(ring).ptr, ringLen: W,
      stopIds: this._buf('stStops', stops.byteLength).upload(stops).ptr,
      seeds: this._buf('stSeeds', seeds.byteLength).upload(seeds).ptr,
    };
  }

  // The logits of step i from the caller's producer (a DeviceBuffer or a
  // host Float32Array of [rows][stride]).
  _stepLogits(d, logits) {
    if (logits instanceof DeviceBuffer) d.logits = logits.ptr;
    else if (logits instanceof Float32Array) d.logits = this._buf('logits', logits.byteLength).upload(logits).ptr;
    else throw new TypeError('the logits producer must return a DeviceBuffer or a Float32Array');
  }

  // decodeBatch's result for each row after k steps (model.js:727-741): the
  // ids through the first stop, how many were fed, eos/stopped/stopId; the
  // windows receive the non-stop tokens as the device ring did.
  _stepResults(opts, packed, k) {
    const rows = opts.rows;
    const sampled = this._scratch.stSampled.download(new Uint32Array(rows * k));
    const res = [];
    for (let r = 0; r < rows; r++) {
      const pk = packed[packed.length > 1 ? r : 0];
      const ids = Array.from(sampled.subarray(r * k, (r + 1) * k));
      const stopAt = ids.findIndex(function (id) { return pk.stopSet.has(id) || id === addon.NO_TOKEN; });
      const stopped = stopAt >= 0;
      const stopId = stopped ? ids[stopAt] : null;
      if (opts.windows) {
        const kept = stopped ? ids.slice(0, stopAt) : ids;
        for (let i = 0; i < kept.length; i++) opts.windows[r].note(kept[i]);
      }
      res.push({ ids: stopped ? ids.slice(0, stopAt + 1) : ids, fed: stopped ? stopAt + 1 : k,
        eos: stopped && pk.eosId !== null && stopId === pk.eosId, stopped: stopped, stopId: stopId });
    }
    return res;
  }

  /**
   * decodeBatch's k-step loop (model.js:649-742) for opts.rows sequences,
   * each token fed back on the device: step i samples every live row from
   * opts.logits(i, nextTokens), the logits ([rows][stride], a DeviceBuffer
   * or a Float32Array) the caller's model computed from the tokens in
   * nextTokens (a DeviceBuffer of rows uint32: opts.firstTokens at step 0,
   * then the last step's tokens).  A row that samples one of its stop ids
   * freezes and emits its first stop id from then on; other tokens join its
   * device penalty ring (the last windowSize tokens, seeded from
   * opts.windows).  Draws use each row's seed at the row's iteration
   * (kernels.js:181).  opts as sampleRows otherwise, with k (>= 1) and no
   * history/uniforms.  Returns per row {ids, fed, eos, stopped, stopId}.
   */
  decodeSteps(opts) {
    this._idle('decodeSteps');
    const k = Math.floor(opts.k);
    if (!(k >= 1)) throw new RangeError('k must be >= 1');
    const r = this._describe(opts, true);
    const st = this._stepState(opts, r.packed, k);
    const next = this._scratch.stNext;
    for (let i = 0; i < k; i++) {
      this._stepLogits(r.desc, opts.logits(i, next));
      addon.sampleStep(this._handle(), r.desc, st);
    }
    return this._stepResults(opts, r.packed, k);
  }

  /** decodeSteps with each launch and wait on a worker thread; opts.logits may return a promise. */
  decodeStepsAsync(opts) {
    const self = this;
    return this._enqueue(function () {
      const k = Math.floor(opts.k);
      if (!(k >= 1)) throw new RangeError('k must be >= 1');
      const r = self._describe(opts, true);
      const st = self._stepState(opts, r.packed, k);
      const next = self._scratch.stNext;
      let chain = Promise.resolve();
      for (let i = 0; i < k; i++) {
        chain = chain.then(function () { return opts.logits(i, next); }).then(function (lg) {
          self._stepLogits(r.desc, lg);
          return self._worker(addon.sampleStepAsync(self._handle(), r.desc, st));
        });
      }
      return chain.then(function () { return self._stepResults(opts, r.packed, k); });
    });
  }

  /**
   * decodeSteps with the LM head fused into each step: the reference's
   * per-iteration lm -> topk -> sampler with tokens[0] fed back
   * (model.js:711-717, kernels.js:189-199).  Step i's logits are
   * opts.head.weight times opts.hidden(i, nextTokens): the final-normed
   * hidden states [rows][hiddenStride] (a DeviceBuffer or a Float32Array) the
   * caller's model computed from the tokens in nextTokens.  opts.head:
   * {weight, dim, format?, weightStride?, hiddenStride?} as for
   * lmHeadSample; rows <= LMH_MAX_ROWS.  Everything else, and the result, as
   * decodeSteps.
   */
  decodeStepsWithHead(opts) {
    this._idle('decodeStepsWithHead');
    const k = Math.floor(opts.k);
    if (!(k >= 1)) throw new RangeError('k must be >= 1');
    if (typeof opts.hidden !== 'function') throw new TypeError('hidden must be a function (step, nextTokens)');
    const r = this._describe(opts, true);
    const st = this._stepState(opts, r.packed, k);
    const next = this._scratch.stNext;
    for (let i = 0; i < k; i++) {
      const hd = this._describeHead({ rows: opts.rows, head: Object.assign({}, opts.head, { hidden: opts.hidden(i, next) }) });
      addon.lmHeadStep(this._handle(), r.desc, hd, st);
    }
    return this._stepResults(opts, r.packed, k);
  }

  /** decodeStepsWithHead with each launch and wait on a worker thread; opts.hidden may return a promise. */
  decodeStepsWithHeadAsync(opts) {
    const self = this;
    return this._enqueue(function () {
      const k = Math.floor(opts.k);
      if (!(k >= 1)) throw new RangeError('k must be >= 1');
      if (typeof opts.hidden !== 'function') throw new TypeError('hidden must be a function (step, nextTokens)');
      const r = self._describe(opts, true);
      const st = self._stepState(opts, r.packed, k);
      const next = self._scratch.stNext;
      let chain = Promise.resolve();
      for (let i = 0; i < k; i++) {
        chain = chain.then(function () { return opts.hidden(i, next); }).then(function (h) {
          const hd = self._describeHead({ rows: opts.rows, head: Object.assign({}, opts.head, { hidden: h }) });
          return self._worker(addon.lmHeadStepAsync(self._handle(), r.desc, hd, st));
        });
      }
      return chain.then(function () { return self._stepResults(opts, r.packed, k); });
    });
  }

  /**
   * The reference's sample(cands, opts) signature (tokenizer.js:151): a
   * candidate list [id, value] interleaved in ids/vals, presence penalty
   * over opts.recentIds.  Runs on the GPU over a row that holds the
   * candidates' values (every other id excluded).  opts.uniform replaces
   * Math.random() when given.
   */
  sample(cands, opts) {
    this._idle('sample');
    opts = opts || {};
    const n = cands.ids.length >> 1;
    let vocab = 1;
    for (let i = 0; i < n; i++) vocab = Math.max(vocab, (cands.ids[i * 2] >>> 0) + 1);
    const row = new Float32Array(vocab).fill(NaN);
    const words = new Uint32Array(Math.ceil(vocab / 32));
    for (let i = 0; i < n; i++) {
      const id = cands.ids[i * 2] >>> 0;
      row[id] = cands.vals[i * 2 + 1];
      words[id >> 5] |= (1 << (id & 31)) >>> 0;
    }
    const params = {
      temperature: orDefault(opts.temperature, 0.6),
      topK: orDefault(opts.topK, 20),
      topP: orDefault(opts.topP, 0.95),
      presencePenalty: orDefault(opts.presencePenalty, 0),
    };
    const u = new Float64Array([opts.uniform !== undefined ? opts.uniform : Math.random()]);
    const out = this.sampleRows({
      logits: row, rows: 1, vocab: vocab, mask: words, params: params,
      history: opts.recentIds ? [opts.recentIds] : null, uniforms: u,
    });
    return out.ids[0];
  }

  /**
   * Speculative verify.  opts: {target, draft (DeviceBuffer | Float32Array),
   * vocab, seqs, draftLen, draftIds (Uint32Array), uniforms (Float64Array
   * [seqs][draftLen+1][2]), temperature, mask? (Uint32Array words)}.
   * Returns {tokens: Uint32Array[seqs*(draftLen+1)], accepted: Int32Array}.
   */
  verify(opts) {
    this._idle('verify');
    const d = this._describeVerify(opts);
    addon.verify(this._handle(), d);
    return this._collectVerify(opts);
  }

  verifyAsync(opts) {
    const self = this;
    return this._enqueue(function () {
      const d = self._describeVerify(opts);
      return self._worker(addon.verifyAsync(self._handle(), d)).then(function () { return self._collectVerify(opts); });
    });
  }

  /**
   * The reference's exact-match speculative round (specChain's acceptSpec,
   * kernels.js:211-401) for opts.seqs sequences: drafts are the argmax of
   * opts.draft (the draft head's rows [seqs*draftLen][stride]) or given in
   * opts.draftIds; verify row j of a sequence (opts.target
   * [seqs*(draftLen+1)][stride]) is sampled with the sequence's params
   * (opts.params, one or one per sequence, with seed and stop ids), its
   * history (opts.windows or opts.history, as of the round's start) and the
   * draw of (seed, opts.round, j); a draft is accepted iff the verify row
   * before it drew exactly it and it is not a stop id.  Returns per sequence
   * {a, next, picks, drafts, d0, d1, stopped, stopId, eos}; each window
   * receives the committed picks that are not stop ids (model.js:994-996).
   */
  specExact(opts) {
    this._idle('specExact');
    const r = this._describeSpec(opts);
    addon.specExact(this._handle(), r.desc);
    return this._collectSpec(opts, r.packed);
  }

  specExactAsync(opts) {
    const self = this;
    return this._enqueue(function () {
      const r = self._describeSpec(opts);
      return self._worker(addon.specExactAsync(self._handle(), r.desc))
        .then(function () { return self._collectSpec(opts, r.packed); });
    });
  }

  // The device state of a chain of speculative rounds (acceptSpec's ctl,
  // posBuf and ring, kernels.js:211-367): {frozen, round, pos, accepted} per
  // sequence (round opts.round, pos opts.positions or 0), the rings seeded
  // from opts.windows, the round log and the next input tokens
  // (opts.firstTokens).
  _specState(opts, rounds) {
    const seqs = opts.seqs;
    const L = opts.draftLen;
    const W = Math.floor(orDefault(opts.windowSize, opts.windows && opts.windows.length ? opts.windows[0].size : 512));
    if (!(W >= 1 && W <= addon.MAX_HISTORY)) throw new RangeError('windowSize must be in [1, ' + addon.MAX_HISTORY + ']');
    const state = new Uint32Array(seqs * 4);
    const pos = opts.positions ? toU32(opts.positions) : null;
    if (pos && pos.length !== seqs) throw new RangeError('positions must have one entry per sequence');
    for (let q = 0; q < seqs; q++) {
      state[q * 4 + 1] = (orDefault(opts.round, 0)) >>> 0;
      state[q * 4 + 2] = pos ? pos[q] : 0;
    }
    const ring = new Uint32Array(seqs * (1 + W));
    if (opts.windows) {
      if (opts.windows.length !== seqs) throw new RangeError('windows must have one PenaltyWindow per sequence');
      for (let q = 0; q < seqs; q++) {
        const g = opts.windows[q].genIds;
        const n = g.length;
        const base = q * (1 + W);
        ring[base] = n;
        for (let i = Math.max(0, n - W); i < n; i++) ring[base + 1 + (i % W)] = g[i];
      }
    }
    const next = new Uint32Array(seqs);
    if (opts.firstTokens) {
      const f = toU32(opts.firstTokens);
      if (f.length !== seqs) throw new RangeError('firstTokens must have one id per sequence');
      next.set(f);
    }
    return {
      state: this._buf('spState', state.byteLength).upload(state).ptr,
      ring: this._buf('spRing', ring.byteLength).upload(ring).ptr, ringLen: W,
      log: this._buf('spLog', seqs * rounds * (L + 2) * 4).ptr, maxRounds: rounds,
      nextTokens: this._buf('spNext', seqs * 4).upload(next).ptr,
    };
  }

  // Round r's logits from the caller's producer: {target, draft?, draftIds?}.
  _specRound(d, lg, opts) {
    const self = this;
    const dev = function (name, x) {
      if (x instanceof DeviceBuffer) return x.ptr;
      if (x instanceof Float32Array) return self._buf(name, x.byteLength).upload(x).ptr;
      throw new TypeError('round logits must be DeviceBuffers or Float32Arrays');
    };
    if (!lg || !lg.target) throw new TypeError('the logits producer must return {target, draft?, draftIds?}');
    d.targetLogits = dev('sTarget', lg.target);
    if (lg.draft) {
      d.draftLogits = dev('sDraft', lg.draft);
      d.draftIds = this._buf('sIds', opts.seqs * opts.draftLen * 4).ptr;
    } else {
      const ids = toU32(lg.draftIds);
      if (ids.length !== opts.seqs * opts.draftLen) throw new RangeError('draftIds must hold seqs * draftLen ids');
      d.draftLogits = null;
      d.draftIds = this._buf('sIds', ids.byteLength).upload(ids).ptr;
    }
  }

  // The chain's outcome: each round's log entry per sequence, the state,
  // and the windows mirroring the device rings (the committed tokens that
  // are not stop ids, kernels.js:341-357).
  _specChainResults(opts, packed, rounds) {
    const seqs = opts.seqs;
    const L = opts.draftLen;
    const log = this._scratch.spLog.download(new Uint32Array(seqs * rounds * (L + 2)));
    const state = this._scratch.spState.download(new Uint32Array(seqs * 4));
    const out = [];
    for (let r = 0; r < rounds; r++) {
      const row = [];
      for (let q = 0; q < seqs; q++) {
        const e = log.subarray((q * rounds + r) * (L + 2), (q * rounds + r + 1) * (L + 2));
        const a = e[0];
        const drafts = Array.from(e.subarray(2, 2 + L));
        row.push({ a: a, next: e[1], drafts: drafts, frozen: a === 0 });
        if (opts.windows && a > 0) {
          const pk = packed[packed.length > 1 ? q : 0];
          const committed = drafts.slice(0, a - 1).concat([e[1]]);
          for (let i = 0; i < committed.length; i++) if (!pk.stopSet.has(committed[i])) opts.windows[q].note(committed[i]);
        }
      }
      out.push(row);
    }
    const pos = [];
    const stopped = [];
    for (let q = 0; q < seqs; q++) {
      stopped.push(state[q * 4] !== 0);
      pos.push(state[q * 4 + 2]);
    }
    return { rounds: out, pos: pos, stopped: stopped };
  }

  /**
   * specChain's rounds (model.js:867-1008) with acceptSpec's commit on the
   * device (kernels.js:340-367), so that no host work runs between rounds.
   * Round r is specExact's round over opts.logits(r, nextTokens) ->
   * {target, draft?, draftIds?}: the verify rows [seqs*(draftLen+1)][stride]
   * and the draft head's rows [seqs*draftLen][stride] (or the drafts), each
   * a DeviceBuffer or a Float32Array, that the caller's models computed from
   * the tokens in nextTokens (a DeviceBuffer of seqs uint32: opts.firstTokens,
   * then each round's next token).  A sequence's history is its device ring
   * (the last windowSize tokens, seeded from opts.windows); one whose next
   * token is one of its stop ids freezes and reads no logits from then on.
   * opts as specExact otherwise, with opts.rounds (>= 1), opts.round the
   * chain's first round (posBuf[4]; default 0) and opts.positions the
   * sequences' positions.  Returns {rounds: [[{a, next, drafts, frozen}]
   * per sequence] per round, pos, stopped}; each window receives the
   * committed tokens that are not stop ids.
   */
  specSteps(opts) {
    this._idle('specSteps');
    const R = Math.floor(opts.rounds);
    if (!(R >= 1)) throw new RangeError('rounds must be >= 1');
    if (typeof opts.logits !== 'function') throw new TypeError('logits must be a function (round, nextTokens)');
    const st = this._specState(opts, R);
    const next = this._scratch.spNext;
    let r0 = null;
    for (let i = 0; i < R; i++) {
      const lg = opts.logits(i, next);
      if (!r0) r0 = this._describeSpec(this._chainOpts(opts, lg));
      this._specRound(r0.desc, lg, opts);
      addon.specStep(this._handle(), r0.desc, st);
    }
    return this._specChainResults(opts, r0.packed, R);
  }

  /** specSteps with each launch and wait on a worker thread; opts.logits may return a promise. */
  specStepsAsync(opts) {
    const self = this;
    return this._enqueue(function () {
      const R = Math.floor(opts.rounds);
      if (!(R >= 1)) throw new RangeError('rounds must be >= 1');
      if (typeof opts.logits !== 'function') throw new TypeError('logits must be a function (round, nextTokens)');
      const st = self._specState(opts, R);
      const next = self._scratch.spNext;
      let r0 = null;
      let chain = Promise.resolve();
      for (let i = 0; i < R; i++) {
        chain = chain.then(function () { return opts.logits(i, next); }).then(function (lg) {
          if (!r0) r0 = self._describeSpec(self._chainOpts(opts, lg));
          self._specRound(r0.desc, lg, opts);
          return self._worker(addon.specStepAsync(self._handle(), r0.desc, st));
        });
      }
      return chain.then(function () { return self._specChainResults(opts, r0.packed, R); });
    });
  }

  // specExact's options for a chain's descriptor: the first round's
  // logits, no host history (the rings are the history).
  _chainOpts(opts, lg) {
    const o = Object.assign({}, opts, { target: lg.target, draft: lg.draft, draftIds: lg.draftIds });
    delete o.windows;
    delete o.history;
    return o;
  }

  _describeSpec(opts) {
    const self = this;
    const dev = function (name, x) {
      if (x instanceof DeviceBuffer) return x.ptr;
      return self._buf(name, x.byteLength).upload(x).ptr;
    };
    const seqs = opts.seqs;
    const L = opts.draftLen;
    const vocab = opts.vocab;
    const nwords = Math.ceil(vocab / 32);
    const ps = Array.isArray(opts.params) ? opts.params : null;
    if (ps && ps.length !== seqs) throw new RangeError('params must have one entry per sequence');
    const packed = ps ? ps.map(function (p) { return packSamplerParams(p, opts.defaults); })
      : [packSamplerParams(opts.params, opts.defaults)];
    const pk = function (q) { return packed[ps ? q : 0]; };
    const d = {
      targetLogits: dev('sTarget', opts.target), logitsStride: orDefault(opts.stride, vocab), vocab: vocab,
      seqs: seqs, draftLen: L, round: (orDefault(opts.round, 0)) >>> 0, params: packed[0].params,
      outPicks: this._buf('sPicks', seqs * (L + 1) * 4).ptr, outAccepted: this._buf('sAcc', seqs * 4).ptr,
      outNext: this._buf('sNext', seqs * 4).ptr,
    };
    if (opts.draft) {
      d.draftLogits = dev('sDraft', opts.draft);
      d.draftIds = this._buf('sIds', seqs * L * 4).ptr;
    } else {
      const ids = toU32(opts.draftIds);
      if (ids.length !== seqs * L) throw new RangeError('draftIds must hold seqs * draftLen ids');
      d.draftIds = this._buf('sIds', ids.byteLength).upload(ids).ptr;
    }
    if (opts.mask) {
      d.mask = dev('sMask', opts.mask);
      d.maskStride = opts.mask.length === nwords ? 0 : orDefault(opts.maskStride, nwords);
    }
    let hist = opts.history;
    if (!hist && opts.windows) {
      if (opts.windows.length !== seqs) throw new RangeError('windows must have one PenaltyWindow per sequence');
      hist = opts.windows.map(function (w) { return w.recent(); });
    }
    if (hist) this._history(d, hist, seqs, 'sequence');
    if (ps) {
      const ab = new ArrayBuffer(seqs * PARAMS_BYTES);
      const view = new DataView(ab);
      for (let q = 0; q < seqs; q++) writeParams(view, q * PARAMS_BYTES, packed[q].params);
      d.seqParams = this._buf('sParams', ab.byteLength).upload(new Uint8Array(ab)).ptr;
      d.rowHints = packed.every(function (p) { return !(p.params.softcap > 0); }) ? addon.HINT_NO_SOFTCAP : 0;
    }
    const seeds = new Uint32Array(seqs);
    const stops = new Uint32Array(seqs * 4);
    for (let q = 0; q < seqs; q++) {
      seeds[q] = pk(q).seed;
      stops.set(pk(q).paddedStopIds, q * 4);
    }
    d.seeds = this._buf('sSeeds', seeds.byteLength).upload(seeds).ptr;
    d.stopIds = this._buf('sStops', stops.byteLength).upload(stops).ptr;
    return { desc: d, packed: packed };
  }

  _collectSpec(opts, packed) {
    const seqs = opts.seqs;
    const L = opts.draftLen;
    const picks = this._scratch.sPicks.download(new Uint32Array(seqs * (L + 1)));
    const acc = this._scratch.sAcc.download(new Int32Array(seqs));
    const drafts = this._scratch.sIds.download(new Uint32Array(seqs * L));
    const res = [];
    for (let q = 0; q < seqs; q++) {
      const pk = packed[packed.length > 1 ? q : 0];
      const a = acc[q];
      const pq = Array.from(picks.subarray(q * (L + 1), (q + 1) * (L + 1)));
      const dq = Array.from(drafts.subarray(q * L, (q + 1) * L));
      const next = pq[a - 1];
      const stopped = pk.stopSet.has(next);
      if (opts.windows) {
        for (let i = 0; i < a; i++) if (!pk.stopSet.has(pq[i])) opts.windows[q].note(pq[i]);
      }
      res.push({ a: a, next: next, picks: pq, drafts: dq, d0: dq[0], d1: dq[1], stopped: stopped,
        stopId: stopped ? next : null, eos: stopped && pk.eosId !== null && next === pk.eosId });
    }
    return res;
  }

  _describeVerify(opts) {
    const self = this;
    const dev = function (name, x) {
      if (x instanceof DeviceBuffer) return x.ptr;
      return self._buf(name, x.byteLength).upload(x).ptr;
    };
    const seqs = opts.seqs;
    const L = opts.draftLen;
    const nwords = Math.ceil(opts.vocab / 32);
    const d = {
      targetLogits: dev('vTarget', opts.target), draftLogits: dev('vDraft', opts.draft),
      logitsStride: orDefault(opts.stride, opts.vocab), vocab: opts.vocab, seqs: seqs, draftLen: L,
      draftIds: dev('vIds', toU32(opts.draftIds)), uniforms: dev('vU', opts.uniforms),
      temperature: orDefault(opts.temperature, 1.0),
      outTokens: this._buf('vTokens', seqs * (L + 1) * 4).ptr, outAccepted: this._buf('vAcc', seqs * 4).ptr,
    };
    if (opts.mask) {
      d.mask = dev('vMask', opts.mask);
      d.maskStride = opts.mask.length === nwords ? 0 : orDefault(opts.maskStride, nwords);
    }
    return d;
  }

  _collectVerify(opts) {
    const n = opts.seqs * (opts.draftLen + 1);
    return {
      tokens: this._scratch.vTokens.download(new Uint32Array(n)),
      accepted: this._scratch.vAcc.download(new Int32Array(opts.seqs)),
    };
  }
}

module.exports = {
  Sampler: Sampler,
  DeviceBuffer: DeviceBuffer,
  PenaltyWindow: PenaltyWindow,
  MaskBuilder: MaskBuilder,
  packedToolMask: packedToolMask,
  updateTokenMaskState: updateTokenMaskState,
  packSamplerParams: packSamplerParams,
  requestSamplingParams: requestSamplingParams,
  allowedLists: allowedLists,
  PACKER_DEFAULTS: PACKER_DEFAULTS,
  maskFromIds: addon.maskFromIds,
  pcgUniform: addon.pcgUniform,
  clampParams: addon.clampParams,
  version: addon.version,
  MAX_TOP_K: addon.MAX_TOP_K,
  MAX_DRAFT: addon.MAX_DRAFT,
  NO_TOKEN: addon.NO_TOKEN,
  FLAG_EMPTY_ROW: addon.FLAG_EMPTY_ROW,
  FLAG_TOPP_EDGE: addon.FLAG_TOPP_EDGE,
  FLAG_DRAW_EDGE: addon.FLAG_DRAW_EDGE,
  STOP_PAD: STOP_PAD,
  LMH_MAX_ROWS: addon.LMH_MAX_ROWS,
  LMH_MAX_LDS_FLOATS: addon.LMH_MAX_LDS_FLOATS,
  LMH_MAX_VOCAB: addon.LMH_MAX_VOCAB,
};
