'use strict';
/*
 * Node host of the MI355X sampler: the reference's sampling surface
 * (src/engine/sampler.ts) over libtabby_sampler.so, through the N-API addon in
 * build/tabby_sampler.node. Written for Node 12 (CommonJS; no `?.` or `??`).
 *
 *   SeededRandom       mulberry32, sampler.ts:105-119 (produces each row's uniform)
 *   DEFAULT_SAMPLING   sampler.ts:93-98
 *   SampleOutcome      sampler.ts:121-135 ({id, probability, consideredCount, poolMass,
 *                      poolExhausted})
 *   TopKResult         forward.ts:93-103 ({maxLogit, sumExp, ids, logits})
 *   Sampler            ForwardPass's sampling scratch + encodeSampling + readback +
 *                      sampleFromTopK (forward.ts:243-248, 442-451, 522-601;
 *                      sampler.ts:147-212), one launch for a batch of rows
 *   sample(logits, params, rng)   the one-row call of inference.worker.ts:162-168
 *   encodeSampleBlock / decodeSampleBlock   the sample block a decode step reads back
 *                      (forward.ts:127-157): [maxLogit, sumExp, (value, index) * k] as
 *                      f32 words, each index a u32 in its word's bytes
 *
 * Every sampling computation runs on the GPU. There is no JavaScript fallback: if the
 * addon or the library is missing, require() throws.
 */
const native = require('./build/tabby_sampler.node');

const F32 = 0;
const F16 = 1;
const PARAMS_BYTES = 32;  // tabby_row_params
const RESULT_BYTES = 48;  // tabby_row_result

class SeededRandom {
  constructor(seed) {
    this.state = seed >>> 0;
  }

  next() {
    const s = (this.state + 0x6d2b79f5) >>> 0;
    this.state = s;
    let t = Math.imul(s ^ (s >>> 15), s | 1);
    t = (t ^ (t + Math.imul(t ^ (t >>> 7), t | 61))) | 0;
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  }
}

const DEFAULT_SAMPLING = Object.freeze({ temperature: 0.7, topK: 40, topP: 0.9, seed: 0 });

/** Logits resident on the GPU: [rows, vocab] of f32, or of f16 given as Uint16Array bits. */
class DeviceLogits {
  constructor(device, rows, vocab, dtype, address) {
    this.device = device;
    this.rows = rows;
    this.vocab = vocab;
    this.dtype = dtype;
    const bytes = rows * vocab * (dtype === F16 ? 2 : 4);
    this.buffer = address === undefined
      ? native.deviceAlloc(device, bytes)
      : native.wrapDevicePointer(device, BigInt(address), bytes);
  }

  /**
   * Logits that a HIP producer in this process already wrote (the decode loop's lm_head):
   * `address` is the device pointer as a BigInt. The memory stays the caller's.
   */
  static fromDevicePointer(address, rows, vocab, dtype, device) {
    return new DeviceLogits(device || 0, rows, vocab, dtype === undefined ? F32 : dtype, address);
  }

  upload(data) {
    const want = this.rows * this.vocab;
    if (data.length !== want) throw new Error(`expected ${want} logits, got ${data.length}`);
    if ((this.dtype === F32) !== (data instanceof Float32Array)) {
      throw new Error('f32 logits come as a Float32Array, f16 logits as a Uint16Array of bits');
    }
    native.upload(this.buffer, data);
    return this;
  }

  free() {
    native.deviceFree(this.buffer);
  }
}

function dtypeOf(data) {
  if (data instanceof Float32Array) return F32;
  if (data instanceof Uint16Array) return F16;
  throw new Error('logits must be a Float32Array or a Uint16Array of f16 bits');
}

// Each row's uniform: a SeededRandom advanced once per row with temperature > 0, in row
// order (sampler.ts:159-167, 194), or caller-supplied numbers.
function uniformsFor(params, rng) {
  const u = new Float64Array(params.length);
  for (let r = 0; r < params.length; r++) {
    if (typeof rng === 'number') u[r] = rng;
    else if (Array.isArray(rng) || ArrayBuffer.isView(rng)) u[r] = rng[r];
    else if (rng && typeof rng.next === 'function') u[r] = params[r].temperature > 0 ? rng.next() : 0;
    else throw new Error('rng must be a SeededRandom, a uniform in [0,1), or one per row');
  }
  return u;
}

function packParams(params, uniforms) {
  const buf = new ArrayBuffer(params.length * PARAMS_BYTES);
  const view = new DataView(buf);
  for (let r = 0; r < params.length; r++) {
    const p = params[r];
    const o = r * PARAMS_BYTES;
    view.setFloat64(o, p.temperature, true);
    view.setFloat64(o + 8, p.topP, true);
    view.setFloat64(o + 16, uniforms[r], true);
    view.setInt32(o + 24, p.topK, true);
    view.setInt32(o + 28, 0, true);
  }
  return buf;
}

function readOutcome(view, r) {
  const o = r * RESULT_BYTES;
  return {
    id: view.getInt32(o, true),
    probability: view.getFloat64(o + 8, true),
    consideredCount: view.getUint32(o + 4, true),
    poolMass: view.getFloat64(o + 16, true),
    poolExhausted: view.getInt32(o + 28, true) !== 0,
  };
}

class Sampler {
  /**
   * @param {{vocabMax: number, rowsMax?: number, kMax?: number, device?: number}} opts
   * kMax bounds topK (the reference allows 0..64, forward.ts:348-351); up to 1024 here.
   */
  constructor(opts) {
    const o = opts || {};
    this.device = o.device || 0;
    this.vocabMax = o.vocabMax;
    this.rowsMax = o.rowsMax || 1;
    this.kMax = o.kMax === undefined ? 64 : o.kMax;
    this.handle = native.create(this.device, this.vocabMax, this.rowsMax, this.kMax);
    this.staging = null;
  }

  /** Uploads host logits ([rows * vocab]) to a new DeviceLogits. */
  upload(data, rows, vocab) {
    return new DeviceLogits(this.device, rows, vocab, dtypeOf(data)).upload(data);
  }

  /**
   * Samples every row of `logits` (a DeviceLogits) in one launch. `params` is one
   * SamplingParams for all rows or one per row. With opts.topK > 0 each outcome also
   * carries `top` (TopKResult: the first opts.topK candidates, highest first).
   * @returns {Array<object>} SampleOutcome per row
   */
  sampleBatch(logits, params, rng, opts) {
    if (!(logits instanceof DeviceLogits)) throw new Error('sampleBatch needs DeviceLogits');
    const rows = logits.rows;
    const list = Array.isArray(params) ? params : new Array(rows).fill(params);
    if (list.length !== rows) throw new Error(`expected ${rows} SamplingParams, got ${list.length}`);
    for (const p of list) {
      if (!Number.isInteger(p.topK) || p.topK < 0 || p.topK > this.kMax) {
        // forward.ts:348-351 rejects before any GPU work
        throw new Error(`topK must be between 0 and ${this.kMax}, got ${p.topK}`);
      }
    }
    const cap = opts && opts.topK ? opts.topK : 0;
    const packed = packParams(list, uniformsFor(list, rng));
    const out = native.sample(this.handle, logits.buffer, logits.dtype, rows, logits.vocab, packed, cap);
    const view = new DataView(out.results);
    const outcomes = [];
    for (let r = 0; r < rows; r++) {
      const outcome = readOutcome(view, r);
      if (cap > 0) {
        const n = view.getInt32(r * RESULT_BYTES + 44, true);
        outcome.top = {
          maxLogit: view.getFloat32(r * RESULT_BYTES + 24, true),
          sumExp: view.getFloat64(r * RESULT_BYTES + 32, true),
          ids: Array.from(out.topkIds.subarray(r * cap, r * cap + n)),
          logits: Array.from(out.topkLogits.subarray(r * cap, r * cap + n)),
        };
      }
      outcomes.push(outcome);
    }
    return outcomes;
  }

  /**
   * sample(logits, {temperature, topK, topP}, rng) for one row, the reference's call shape.
   * `logits` is a DeviceLogits with one row, or a Float32Array / Uint16Array (f16 bits),
   * which is uploaded to a staging buffer kept by this Sampler.
   */
  sample(logits, params, rng) {
    let dev = logits;
    if (!(logits instanceof DeviceLogits)) {
      const dtype = dtypeOf(logits);
      const s = this.staging;
      if (!s || s.vocab !== logits.length || s.dtype !== dtype) {
        if (s) s.free();
        this.staging = new DeviceLogits(this.device, 1, logits.length, dtype);
      }
      dev = this.staging.upload(logits);
    }
    if (dev.rows !== 1) throw new Error('sample() takes one row; use sampleBatch() for more');
    return this.sampleBatch(dev, [params], rng)[0];
  }

  destroy() {
    if (this.staging) this.staging.free();
    this.staging = null;
    native.destroy(this.handle);
  }
}

// The reference's sample block (forward.ts:127-129, 142-157): f32 words [maxLogit, sumExp,
// then (value, index) per candidate], the index written as a u32 into its word.
const SAMPLE_HEADER_FLOATS = 2;

/** A TopKResult as a sample block of k slots (default: all of its candidates). */
function encodeSampleBlock(top, k) {
  const n = k === undefined ? top.ids.length : k;
  if (!(n >= 0) || n > top.ids.length || top.logits.length !== top.ids.length) {
    throw new Error('encodeSampleBlock: k must be within the result\'s ' + top.ids.length + ' candidates');
  }
  const raw = new ArrayBuffer((SAMPLE_HEADER_FLOATS + 2 * n) * 4);
  const asFloat = new Float32Array(raw);
  const asUint = new Uint32Array(raw);
  asFloat[0] = top.maxLogit;
  asFloat[1] = top.sumExp;
  for (let i = 0; i < n; i++) {
    const slot = SAMPLE_HEADER_FLOATS + i * 2;
    asFloat[slot] = top.logits[i];
    asUint[slot + 1] = top.ids[i] >>> 0;
  }
  return raw;
}

/** The first k candidates of a sample block, as a TopKResult. */
function decodeSampleBlock(raw, k) {
  const asFloat = new Float32Array(raw);
  const asUint = new Uint32Array(raw);
  if (SAMPLE_HEADER_FLOATS + 2 * k > asFloat.length) {
    throw new Error('decodeSampleBlock: the block holds ' + ((asFloat.length - SAMPLE_HEADER_FLOATS) >> 1) +
                    ' candidates, asked for ' + k);
  }
  const ids = [];
  const logits = [];
  for (let i = 0; i < k; i++) {
    const slot = SAMPLE_HEADER_FLOATS + i * 2;
    ids.push(asUint[slot + 1]);
    logits.push(asFloat[slot]);
  }
  return { maxLogit: asFloat[0], sumExp: asFloat[1], ids, logits };
}

module.exports = {
  Sampler,
  encodeSampleBlock,
  decodeSampleBlock,
  DeviceLogits,
  SeededRandom,
  DEFAULT_SAMPLING,
  F32,
  F16,
  version: native.version,
};
