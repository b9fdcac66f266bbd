// Types of the Node host API (index.js).  The mask and parameter shapes are
// the reference's: TokenMask (lib/webgpu-llm/tool-constraint.ts:39-42) and
// SampleParams (lib/webgpu-llm/model.d.ts:4-16), with the build's
// additional penalties.

export type TokenMask =
  | { kind: "all" }
  | { kind: "allow"; tokenIds: Uint32Array }
  | { kind: "deny"; tokenIds: Uint32Array }
  /** This build's extension: packed words (ceil(vocab / 32), bit id & 31 of word id >> 5 = allowed). */
  | { kind: "words"; words: Uint32Array };

/** Packed-bitmask producer for grammar code; results are immutable words arrays. */
export declare class MaskBuilder {
  constructor(vocab: number, cacheSize?: number);
  readonly vocab: number;
  readonly nwords: number;
  hits: number;
  misses: number;
  all(): Uint32Array;
  none(): Uint32Array;
  allow(ids: Uint32Array | number[] | Set<number>): Uint32Array;
  deny(ids: Uint32Array | number[] | Set<number>): Uint32Array;
  fromTokenMask(mask: TokenMask): Uint32Array;
  or(a: Uint32Array, b: Uint32Array): Uint32Array;
  and(a: Uint32Array, b: Uint32Array): Uint32Array;
  andNot(a: Uint32Array, b: Uint32Array): Uint32Array;
  count(words: Uint32Array): number;
}

/** A ToolConstraint's TokenMask (tool-constraint.ts:653-661) as packed words. */
export declare function packedToolMask(
  constraint: { mask(raw: string, parseArguments: unknown): TokenMask },
  raw: string,
  parseArguments: unknown,
  builder: MaskBuilder
): { kind: "words"; words: Uint32Array };

export interface SampleParams {
  temperature?: number;
  topP?: number;
  topK?: number;
  presencePenalty?: number;
  repetitionPenalty?: number;
  frequencyPenalty?: number;
  /** Gemma final-logit softcap (30); 0 = off. */
  softcap?: number;
  eosId?: number;
  stopIds?: number[];
  seed?: number;
  /** Whitelist (model.d.ts:15): the draw is restricted to these ids. */
  allowedTokenIds?: Uint32Array;
}

export interface PackerDefaults {
  temperature?: number;
  topP?: number;
  topK?: number;
  seed?: number | null;
  eosFromStops?: boolean;
}

export interface ClampedParams {
  temperature: number;
  topP: number;
  topK: number;
  repetitionPenalty: number;
  presencePenalty: number;
  frequencyPenalty: number;
  softcap: number;
}

export interface PackedParams {
  params: ClampedParams;
  seed: number;
  stopIds: number[];
  paddedStopIds: number[];
  stopSet: Set<number>;
  eosId: number | null;
  allowedTokenIds: Uint32Array | null;
}

/** The generated-token window of one sequence (model.js:386-389). */
export declare class PenaltyWindow {
  constructor(size?: number);
  readonly size: number;
  genIds: number[];
  reset(): void;
  note(id: number): void;
  recent(): Uint32Array;
  recentSet(): Set<number>;
  rewind(sampledCount: number): void;
}

/** decodeBatch's result (model.d.ts:23-29). */
export interface DecodeBatchResult {
  ids: number[];
  fed: number;
  eos: boolean;
  stopped: boolean;
  stopId: number | null;
}

export interface TokenMaskState {
  cfg: { text: { vocab: number } };
  allowedCount: number;
  allowedTokens: number;
  tokenMaskKind: "all" | "allow" | "deny";
  tokenMaskIds: Uint32Array | null;
  words: DeviceBuffer;
  uploads: number;
  upload(words: Uint32Array): void;
}

export declare class DeviceBuffer {
  readonly ptr: bigint;
  readonly bytes: number;
  upload(data: ArrayBufferView): this;
  download<T extends ArrayBufferView>(into: T): T;
  free(): void;
}

export interface SampleRowsOptions {
  logits: DeviceBuffer | Float32Array;
  rows: number;
  vocab: number;
  stride?: number;
  mask?: TokenMaskState | TokenMask | Uint32Array | DeviceBuffer;
  maskStride?: number;
  params?: SampleParams | SampleParams[];
  defaults?: PackerDefaults;
  history?: Array<number[] | Uint32Array | Set<number>>;
  windows?: PenaltyWindow[];
  recentIds?: Set<number> | number[];
  uniforms?: Float64Array;
  iteration?: number;
  full?: boolean;
}

/** The LM head of lmHeadSample: logits[row][id] = sum over k of
 * weight[id][k] * hidden[row][k]: a bf16 head widened to f32, or a GGUF
 * head (Q8_0 / Q4_0 / Q6_K blocks) against the Q8_1-quantized hidden
 * state, summed in the library's fixed order. */
export type LmHeadFormat = 'bf16' | 'q8_0' | 'q4_0' | 'q6_k';

export interface LmHead {
  /** [rows][hiddenStride] f32 final-normed hidden states. */
  hidden: DeviceBuffer | Float32Array;
  /** [vocab] rows, device-resident: bf16 bits, or GGUF blocks. */
  weight: DeviceBuffer;
  /** Default 'bf16'. */
  format?: LmHeadFormat;
  /** A multiple of 256; rows * dim <= LMH_MAX_LDS_FLOATS. */
  dim: number;
  hiddenStride?: number;
  /** Between rows: elements (bf16, default dim) or bytes (GGUF, default the row's bytes). */
  weightStride?: number;
  /** Also write the logits [rows][vocab] f32 here. */
  outLogits?: DeviceBuffer;
}

export interface LmHeadSampleOptions extends Omit<SampleRowsOptions, 'logits' | 'stride'> {
  head: LmHead;
}

export interface DecodeStepsOptions {
  /** Step i's logits [rows][stride], computed from the tokens in nextTokens. */
  logits(i: number, nextTokens: DeviceBuffer): DeviceBuffer | Float32Array | Promise<DeviceBuffer | Float32Array>;
  rows: number;
  vocab: number;
  k: number;
  stride?: number;
  mask?: TokenMaskState | TokenMask | Uint32Array | DeviceBuffer;
  maskStride?: number;
  params?: SampleParams | SampleParams[];
  defaults?: PackerDefaults;
  /** The tokens fed at step 0 (decodeBatch's firstTok per row). */
  firstTokens?: Uint32Array | number[];
  windows?: PenaltyWindow[];
  windowSize?: number;
}

export interface SampleRowsResult {
  ids: Uint32Array;
  stopped: boolean[];
  stopId: Array<number | null>;
  probs?: Float64Array;
  candIds?: Uint32Array;
  counts?: Int32Array;
  flags?: Uint32Array;
}

export interface VerifyOptions {
  target: DeviceBuffer | Float32Array;
  draft: DeviceBuffer | Float32Array;
  vocab: number;
  stride?: number;
  seqs: number;
  draftLen: number;
  draftIds: Uint32Array | number[];
  uniforms: DeviceBuffer | Float64Array;
  temperature?: number;
  mask?: DeviceBuffer | Uint32Array;
  maskStride?: number;
}

export interface SpecExactOptions {
  /** Verify rows [seqs * (draftLen + 1)][stride]. */
  target: DeviceBuffer | Float32Array;
  /** The draft head's rows [seqs * draftLen][stride] (drafts = their argmax), or draftIds. */
  draft?: DeviceBuffer | Float32Array;
  draftIds?: Uint32Array | number[];
  vocab: number;
  stride?: number;
  seqs: number;
  draftLen: number;
  params?: SampleParams | SampleParams[];
  defaults?: PackerDefaults;
  round?: number;
  history?: Array<number[] | Uint32Array | Set<number>>;
  windows?: PenaltyWindow[];
  mask?: DeviceBuffer | Uint32Array;
  maskStride?: number;
}

/** decodeSteps with the LM head fused into each step (rows <= LMH_MAX_ROWS). */
export interface DecodeStepsWithHeadOptions extends Omit<DecodeStepsOptions, 'logits' | 'stride'> {
  /** Step i's final-normed hidden states [rows][hiddenStride], computed from the tokens in nextTokens. */
  hidden(i: number, nextTokens: DeviceBuffer): DeviceBuffer | Float32Array | Promise<DeviceBuffer | Float32Array>;
  head: Omit<LmHead, 'hidden' | 'outLogits'>;
}

/** A chain of speculative rounds with acceptSpec's commit on the device. */
export interface SpecStepsOptions extends Omit<SpecExactOptions, 'target' | 'draft' | 'draftIds' | 'history'> {
  rounds: number;
  /** Round r's verify rows and draft head rows (or drafts), computed from the tokens in nextTokens. */
  logits(r: number, nextTokens: DeviceBuffer): SpecRoundLogits | Promise<SpecRoundLogits>;
  /** The tokens fed to round 0, one per sequence. */
  firstTokens?: Uint32Array | number[];
  /** The sequences' positions at the chain's start (posBuf[0]); default 0. */
  positions?: Uint32Array | number[];
  windowSize?: number;
}

export interface SpecRoundLogits {
  target: DeviceBuffer | Float32Array;
  draft?: DeviceBuffer | Float32Array;
  draftIds?: Uint32Array | number[];
}

/** A chain's rounds: the log entry of each sequence in each round, the final positions and stop state. */
export interface SpecStepsResult {
  rounds: Array<Array<{ a: number; next: number; drafts: number[]; frozen: boolean }>>;
  pos: number[];
  stopped: boolean[];
}

/** One sequence's round (the reference's SpecRound, model.d.ts, plus the picks). */
export interface SpecExactResult {
  a: number;
  next: number;
  picks: number[];
  drafts: number[];
  d0?: number;
  d1?: number;
  stopped: boolean;
  stopId: number | null;
  eos: boolean;
}

export interface VerifyResult {
  tokens: Uint32Array;
  accepted: Int32Array;
}

export declare class Sampler {
  constructor(device?: number);
  close(): Promise<void>;
  /** Pre-sizes device scratch so calls of at most these shapes allocate nothing (sas_reserve_for). */
  reserve(rows: number, vocab: number, opts?: { histIds?: number; lmHeadRows?: number; verifySeqs?: number;
    verifyDraftLen?: number }): void;
  alloc(bytes: number): DeviceBuffer;
  synchronize(): void;
  createTokenMaskState(vocab: number): TokenMaskState;
  sampleRows(opts: SampleRowsOptions): SampleRowsResult;
  sampleRowsAsync(opts: SampleRowsOptions): Promise<SampleRowsResult>;
  /** The LM head with the sampling step fused (rows <= LMH_MAX_ROWS). */
  lmHeadSample(opts: LmHeadSampleOptions): SampleRowsResult;
  lmHeadSampleAsync(opts: LmHeadSampleOptions): Promise<SampleRowsResult>;
  decodeRows(opts: SampleRowsOptions): DecodeBatchResult[];
  decodeRowsAsync(opts: SampleRowsOptions): Promise<DecodeBatchResult[]>;
  decodeSteps(opts: DecodeStepsOptions): DecodeBatchResult[];
  decodeStepsAsync(opts: DecodeStepsOptions): Promise<DecodeBatchResult[]>;
  decodeStepsWithHead(opts: DecodeStepsWithHeadOptions): DecodeBatchResult[];
  decodeStepsWithHeadAsync(opts: DecodeStepsWithHeadOptions): Promise<DecodeBatchResult[]>;
  sample(
    cands: { ids: ArrayLike<number>; vals: ArrayLike<number> },
    opts?: {
      temperature?: number;
      topK?: number;
      topP?: number;
      presencePenalty?: number;
      recentIds?: Set<number> | null;
      uniform?: number;
    }
  ): number;
  specExact(opts: SpecExactOptions): SpecExactResult[];
  specExactAsync(opts: SpecExactOptions): Promise<SpecExactResult[]>;
  specSteps(opts: SpecStepsOptions): SpecStepsResult;
  specStepsAsync(opts: SpecStepsOptions): Promise<SpecStepsResult>;
  verify(opts: VerifyOptions): VerifyResult;
  verifyAsync(opts: VerifyOptions): Promise<VerifyResult>;
}

export declare function updateTokenMaskState(
  state: { cfg: { text: { vocab: number } }; tokenMaskKind: string; tokenMaskIds: Uint32Array | null;
           allowedCount: number; upload(words: Uint32Array): void },
  mask: TokenMask | undefined | null
): void;
export declare function packSamplerParams(sp?: SampleParams, defaults?: PackerDefaults): PackedParams;
export declare const PACKER_DEFAULTS: { qwen: PackerDefaults; gemma: PackerDefaults };
/** Request defaults and ranges (completions.ts:268-273, gemma-completions.ts:212-217). */
export declare function requestSamplingParams(
  request?: { temperature?: number; top_p?: number; top_k?: number; presence_penalty?: number },
  grammar?: "qwen" | "gemma"
): { temperature: number; topP: number; topK: number; presencePenalty: number };
export declare function allowedLists(packed: PackedParams[], vocab: number, hasMask: boolean):
  Array<Uint32Array | null>;
export declare function maskFromIds(kind: number, ids: Uint32Array | null, vocab: number):
  { words: Uint32Array; allowed: number };
export declare function pcgUniform(seed: number, it: number, row: number): number;
export declare function clampParams(p: Partial<ClampedParams>): ClampedParams;
export declare function version(): string;
export declare const MAX_TOP_K: number;
export declare const MAX_DRAFT: number;
export declare const NO_TOKEN: number;
export declare const FLAG_EMPTY_ROW: number;
export declare const FLAG_TOPP_EDGE: number;
export declare const FLAG_DRAW_EDGE: number;
export declare const STOP_PAD: number;
export declare const LMH_MAX_ROWS: number;
export declare const LMH_MAX_LDS_FLOATS: number;
export declare const LMH_MAX_VOCAB: number;
