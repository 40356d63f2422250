// Types of the Node host (index.js), matching src/engine/sampler.ts and forward.ts's
// TopKResult so a caller of the reference's sampler can switch without changes.

/** sampler.ts:83-91. topK = 0 samples over the whole vocabulary. */
export interface SamplingParams {
  temperature: number;
  topK: number;
  topP: number;
  seed: number;
}

/** sampler.ts:93-98 */
export declare const DEFAULT_SAMPLING: Readonly<SamplingParams>;

/** forward.ts:93-103 */
export interface TopKResult {
  maxLogit: number;
  sumExp: number;
  ids: number[];
  logits: number[];
}

/** sampler.ts:121-135 */
export interface SampleOutcome {
  id: number;
  probability: number;
  consideredCount: number;
  poolMass: number;
  poolExhausted: boolean;
  /** Present when sampleBatch was asked for top-k lists. */
  top?: TopKResult;
}

/** mulberry32, sampler.ts:105-119 */
export declare class SeededRandom {
  constructor(seed: number);
  next(): number;
}

export declare const F32: 0;
export declare const F16: 1;

/** inference.worker.ts:118-123: the worker's candidate pool (1 at temperature 0). */
export declare function poolSize(sampling: Pick<SamplingParams, 'temperature' | 'topK'>, maxTopK?: number): number;
export declare const MAX_TOP_K: 64;

/** sampler.ts:32-52 */
export interface GenerateOptions {
  maxNewTokens: number;
  stopTokens?: readonly number[];
  /** An AbortSignal, or any object with `aborted` (and optionally `reason`). */
  signal?: { aborted: boolean; reason?: unknown; throwIfAborted?(): void };
  onToken?: (id: number, index: number) => void;
}
export interface GenerateResult {
  tokens: number[];
  stopped: boolean;
  ms: number;
}

/** The decode loop of inference.worker.ts:108-206 over Sampler.generate. */
export interface DecodeLoopOptions {
  promptIds: readonly number[];
  prefill(ids: readonly number[]): Promise<DeviceLogits | Float32Array>;
  decode(id: number): Promise<DeviceLogits | Float32Array>;
  sampling: SamplingParams;
  maxNewTokens: number;
  stopTokens?: Iterable<number>;
  isCancelled?(): boolean;
  onToken?(id: number, index: number): void;
  maxTopK?: number;
}
export interface DecodeLoopResult {
  tokens: number[];
  stopped: boolean;
  cancelled: boolean;
  poolExhausted: boolean;
  readbackPerToken: number;
  totalReadback: number;
  ttftMs: number;
  decodeMs: number;
}

export declare class DeviceLogits {
  readonly device: number;
  readonly rows: number;
  readonly vocab: number;
  readonly dtype: 0 | 1;
  static fromDevicePointer(address: bigint, rows: number, vocab: number, dtype?: 0 | 1,
                           device?: number): DeviceLogits;
  upload(data: Float32Array | Uint16Array): this;
  download(): Float32Array | Uint16Array;
  free(): void;
}

export type UniformSource = SeededRandom | number | ArrayLike<number>;

export declare class Sampler {
  constructor(opts: { vocabMax: number; rowsMax?: number; kMax?: number; device?: number });
  upload(data: Float32Array | Uint16Array, rows: number, vocab: number): DeviceLogits;
  sampleBatch(logits: DeviceLogits, params: SamplingParams | SamplingParams[],
              rng: UniformSource, opts?: { topK?: number }): SampleOutcome[];
  sample(logits: DeviceLogits | Float32Array | Uint16Array,
         params: Pick<SamplingParams, 'temperature' | 'topK' | 'topP'>,
         rng: UniformSource): SampleOutcome;
  /** Greedy ids on the GPU, one per row (sampler.ts:13-23). */
  argmax(logits: DeviceLogits | Float32Array | Uint16Array): Int32Array;
  generate(opts: DecodeLoopOptions): Promise<DecodeLoopResult>;
  softmaxRowsDevice(x: DeviceLogits, out: DeviceLogits, nRows: number, rowLen: number,
                    causalPeriod?: number, causalOffset?: number): DeviceLogits;
  destroy(): void;
}

/** sampler.ts:13-23, on the GPU. */
export declare function argmax(logits: Float32Array | Uint16Array | DeviceLogits): number;

/** sampler.ts:54-76, the argmax on the GPU. */
export declare function generateGreedy(promptIds: readonly number[],
                                       forward: (ids: readonly number[]) => Promise<Float32Array | DeviceLogits>,
                                       options: GenerateOptions, sampler?: Sampler): Promise<GenerateResult>;

/** cpu.ts:238-264 (softmax_rows.wgsl's contract), computed on the GPU, bit for bit. */
export declare function softmaxRows(x: Float32Array, nRows: number, rowLen: number,
                                    causalPeriod?: number, causalOffset?: number): Float32Array;

export declare function version(): string;

/** A TopKResult as the sample block of forward.ts:127-157: f32 words [maxLogit, sumExp,
 *  (value, index) * k], each index a u32 in its word. k defaults to all candidates. */
export declare function encodeSampleBlock(top: TopKResult, k?: number): ArrayBuffer;

/** forward.ts:142-157: the first k candidates of a sample block. */
export declare function decodeSampleBlock(raw: ArrayBuffer, k: number): TopKResult;
