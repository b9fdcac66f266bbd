// Types of the Node host API (index.js).  The mask and parameter shapes are
// the reference's: TokenMask (lib/webgpu-llm/tool-constraint.ts:39-42) and
// SampleParams (lib/webgpu-llm/model.d.ts:4-16), with the build's
// additional penalties.

export type TokenMask =
  | { kind: "all" }
  | { kind: "allow"; tokenIds: Uint32Array }
  | { kind: "deny"; tokenIds: Uint32Array };

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
  defaults?: Partial<SampleParams>;
  history?: Array<number[] | Uint32Array | Set<number>>;
  recentIds?: Set<number> | number[];
  uniforms?: Float64Array;
  iteration?: number;
  full?: boolean;
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

export interface VerifyResult {
  tokens: Uint32Array;
  accepted: Int32Array;
}

export declare class Sampler {
  constructor(device?: number);
  close(): void;
  reserve(rows: number, vocab: number): void;
  alloc(bytes: number): DeviceBuffer;
  synchronize(): void;
  createTokenMaskState(vocab: number): TokenMaskState;
  sampleRows(opts: SampleRowsOptions): SampleRowsResult;
  sampleRowsAsync(opts: SampleRowsOptions): Promise<SampleRowsResult>;
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
  verify(opts: VerifyOptions): VerifyResult;
  verifyAsync(opts: VerifyOptions): Promise<VerifyResult>;
}

export declare function updateTokenMaskState(
  state: { cfg: { text: { vocab: number } }; tokenMaskKind: string; tokenMaskIds: Uint32Array | null;
           allowedCount: number; upload(words: Uint32Array): void },
  mask: TokenMask | undefined | null
): void;
export declare function packSamplerParams(sp?: SampleParams, defaults?: Partial<SampleParams>): PackedParams;
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
