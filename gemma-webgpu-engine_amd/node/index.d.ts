// Type declarations of the gsample Node host (index.js): the reference's
// sampling-stage API (src/runtime/sampling.ts, decoding.ts,
// generation-config.ts, constraints.ts, token-byte-trie.ts) plus the batched
// Engine over the libgsample N-API addon.

export interface DecodingConfig {
  temperature: number;
  topK: number;
  topP: number;
  minP: number;
  typicalP: number;
  repetitionPenalty: number;
  repetitionWindow: number;
  frequencyPenalty: number;
  presencePenalty: number;
  maxNewTokens: number;
  seed: number;
  stopTokenIds: number[];
}

export const DEFAULT_DECODING_CONFIG: DecodingConfig;
export function validateDecodingConfig(input: Partial<DecodingConfig>): { ok: boolean; errors: string[] };

export const VOCAB_SIZE: 262144;
export const DEFAULT_GENERATION_CONFIG: DecodingConfig;
export type GemmaGenerationOptions = Partial<DecodingConfig> & {
  constraint?: GenerationConstraint;
  captureTokenLogProbabilities?: boolean;
  [other: string]: unknown;
};
export function resolveGemmaGenerationConfig(options: GemmaGenerationOptions): DecodingConfig;
export function usesGemmaGpuGreedy(config: DecodingConfig): boolean;

export class SeededRandom {
  constructor(seed: number);
  next(): number;
}
export function sampleToken(
  rawLogits: ArrayLike<number>, history: readonly number[], config: DecodingConfig, random: () => number): number;
export function sampleTokenWithProbability(
  rawLogits: ArrayLike<number>, history: readonly number[], config: DecodingConfig, random: () => number,
): { token: number; probability: number; flags: number };
export function tokenLogProbability(rawLogits: ArrayLike<number>, token: number): number;
export function engineFor(vocabSize: number): Engine;
export function releaseEngines(): void;

export interface TokenByteSource {
  readonly vocabularySize: number;
  tokenBytes(tokenId: number): Uint8Array | null;
}
export class TokenByteTrie implements TokenByteSource {
  constructor(source: TokenByteSource);
  readonly vocabularySize: number;
  readonly tokenCount: number;
  readonly offsets: Int32Array;
  readonly bytes: Uint8Array;
  tokenBytes(tokenId: number): Uint8Array | null;
}

export interface ByteDfaSpec {
  stateCount?: number;
  next: ArrayLike<number>;      // [stateCount * 256], -1 = no edge
  finals: ArrayLike<number | boolean>;
  initial?: number;
}
export type GenerationConstraint =
  | ({ type: "byte-dfa"; validateOutput?: (text: string) => void } & ByteDfaSpec)
  | { type: "regex"; pattern: string }
  | { type: "json" | "json-object"; maxDepth?: number; whitespace?: "none" | "compact" | "any" }
  | { type: "json-schema"; schema: object; maxDepth?: number; whitespace?: "none" | "compact" | "any" };

export class ByteLevelDfa {
  constructor(spec: ByteDfaSpec);
  readonly stateCount: number;
  readonly next: Int32Array;
  readonly finals: Uint8Array;
  readonly initial: number;
}
export class CompiledGenerationConstraint {
  constructor(dfa: ByteLevelDfa | ByteDfaSpec, validateOutput?: (text: string) => void, engine?: Engine);
  state: number;
  readonly accepting: boolean;
  legalTokenIds(trie: TokenByteTrie): readonly number[];
  acceptToken(tokenBytes: ArrayLike<number>): void;
  acceptBytes(bytes: ArrayLike<number>): void;
  validateFinal(text: string): void;
}
export function compileGenerationConstraint(constraint: GenerationConstraint): CompiledGenerationConstraint;
export function maskConstraintLogits(
  rawLogits: ArrayLike<number>, legalTokenIds: readonly number[], terminationTokenIds: readonly number[]): Float32Array;
export const EOS_TOKEN_IDS: readonly number[];
export function selectConstrainedToken(args: {
  logits: Float32Array;
  history: readonly number[];
  config: DecodingConfig;
  random: SeededRandom;
  constraint: CompiledGenerationConstraint;
  trie: TokenByteTrie;
  customStopTokens?: Iterable<number>;
  additionalLegalTokens?: readonly number[];
}): number;

export interface RowOptions extends Partial<DecodingConfig> {
  drawIndex?: number;      // draw number of SeededRandom(seed) (0 = first)
  uniform?: number;        // explicit random() value; overrides seed/drawIndex
  softcap?: number;        // > 0: logit <- softcap * tanh(logit / softcap) first
  maskSlot?: number;       // row of the mask table; -1 / undefined: unconstrained
  accepting?: boolean;     // constraint accepting: termination ids are legal
  forceExact?: boolean;    // resolve on the sequential exact path
}
export interface SampleRequest {
  logits: Float32Array | Uint16Array | DeviceBuffer;
  dtype?: "f32" | "bf16";
  rows?: number;
  rowStride?: number;
  configs: RowOptions[];
  histories?: ArrayLike<number>[] | null;
  forced?: { termination?: number[]; extra?: number[] }[] | null;
  maskTable?: DeviceBuffer | null;
  maskSlots?: number;
}
export interface SampleResult {
  tokens: Int32Array;
  probabilities: Float64Array;
  flags: Uint32Array;
}
export const FLAGS: {
  readonly TOPP_TIE: 1; readonly EXACT_PATH: 2; readonly NEAR_TIE: 4; readonly DEAD_END: 8;
  readonly NONFINITE: 16; readonly EMPTY_CANDIDATES: 32; readonly GREEDY: 64; readonly UNSUPPORTED: 128;
};
export const STAGES: readonly ["lmhead", "scan", "finish", "exact", "deep"];

export class DeviceBuffer {
  readonly bytes: number;
  write(data: ArrayBufferView, byteOffset?: number): this;
  read<T extends ArrayBufferView>(out: T, byteOffset?: number): T;
  free(): void;
}
export class Engine {
  constructor(options: { vocabSize: number; maxRows?: number; device?: number });
  readonly vocabSize: number;
  readonly maxRows: number;
  destroy(): void;
  allocate(bytes: number): DeviceBuffer;
  sampleRows(request: SampleRequest): SampleResult;
  tokenLogProbabilities(logits: Float32Array, rows: number, tokens: ArrayLike<number>): Float64Array;
  maskLogits(raw: Float32Array, legal: ArrayLike<number>, termination: ArrayLike<number>): Float32Array;
  useVocab(trie: TokenByteTrie): void;
  useDfa(dfa: ByteLevelDfa): void;
  buildMasks(states: ArrayLike<number>, table?: DeviceBuffer): DeviceBuffer;
  legalTokenIds(state: number): Int32Array;
  dfaAdvance(states: ArrayLike<number>, tokens: ArrayLike<number>): Int32Array;
  dfaAdvanceBytes(state: number, bytes: Uint8Array): number;
  dfaAccepting(state: number): boolean;
  lmhead(hidden: DeviceBuffer, weight: DeviceBuffer, mRows: number, width: number, softcap: number,
         logits: DeviceBuffer): DeviceBuffer;
  qatLmhead(x: DeviceBuffer, mRows: number, width: number, codes: DeviceBuffer, layout: "row-major" | "block-major",
            rowScales: DeviceBuffer, inputScale: number, outputScale: number, logits: DeviceBuffer): DeviceBuffer;
  qatLmheadSample(x: DeviceBuffer, width: number, codes: DeviceBuffer, layout: "row-major" | "block-major",
                  rowScales: DeviceBuffer, inputScale: number, outputScale: number, scratch: DeviceBuffer,
                  request: SampleRequest): SampleResult;
  lmheadSample(hidden: DeviceBuffer, weight: DeviceBuffer, width: number, softcap: number, scratch: DeviceBuffer,
               request: SampleRequest): SampleResult;
  timingBegin(maxCalls: number): void;
  timingEnd(): Record<"lmhead" | "scan" | "finish" | "exact" | "deep", [number, number]>;
}

export const ADDON_PATH: string;

// token-bytes.js: the Gemma token byte table (gemma-tokenizer.ts:17-19,346-360)
export const GEMMA_START_CHANNEL_TOKEN_ID: number;
export const GEMMA_END_CHANNEL_TOKEN_ID: number;
export function createTokenByteTable(
  vocabulary: Map<string, number> | Record<string, number>, specialIds: Iterable<number>): (Uint8Array | null)[];
export function readTokenizerJson(path: string): { vocabulary: Map<string, number>; specialIds: number[] };
export function loadTokenizerJson(path: string): (Uint8Array | null)[];
export function tokenByteSource(table: (Uint8Array | null)[]): TokenByteSource;
export function writeTokenByteTable(path: string, table: (Uint8Array | null)[]): void;
export function readTokenByteTable(path: string): (Uint8Array | null)[];
