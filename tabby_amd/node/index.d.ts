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

export declare class DeviceLogits {
  readonly device: number;
  readonly rows: number;
  readonly vocab: number;
  readonly dtype: 0 | 1;
  static fromDevicePointer(address: bigint, rows: number, vocab: number, dtype?: 0 | 1,
                           device?: number): DeviceLogits;
  upload(data: Float32Array | Uint16Array): this;
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
  destroy(): void;
}

export declare function version(): string;

/** A TopKResult as the sample block of forward.ts:127-157: f32 words [maxLogit, sumExp,
 *  (value, index) * k], each index a u32 in its word. k defaults to all candidates. */
export declare function encodeSampleBlock(top: TopKResult, k?: number): ArrayBuffer;

/** forward.ts:142-157: the first k candidates of a sample block. */
export declare function decodeSampleBlock(raw: ArrayBuffer, k: number): TopKResult;
