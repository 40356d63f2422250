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
 *   poolSize           the worker's candidate-pool rule (inference.worker.ts:118-123)
 *   Sampler.generate   the worker's decode loop (inference.worker.ts:108-206): one launch and
 *                      one 48-byte readback per token, stop tokens, cancellation re-checked
 *                      after every await
 *   argmax / Sampler.argmax / generateGreedy   greedy decoding (sampler.ts:13-23, 54-76) on
 *                      the GPU's argmax, no pool and no uniform
 *   softmaxRows / Sampler.softmaxRows   the attention row softmax (cpu.ts:238-264,
 *                      softmax_rows.wgsl), bit for bit the CPU reference's
 *
 * Every sampling computation runs on the GPU. There is no JavaScript fallback: if the
 * addon or the library is missing, require() throws.
 */
const native = require('./build/tabby_sampler.node');
const { performance } = require('perf_hooks');

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

/** The reference's largest pool (MAX_TOP_K, the topK bound of forward.ts:348-351). */
const MAX_TOP_K = 64;

/**
 * The candidate pool the worker asks the GPU for (inference.worker.ts:118-123): temperature 0
 * needs only the argmax; otherwise top-p may look past top-k, so the pool is the larger of the
 * two intents, topK = 0 meaning the largest pool.
 */
function poolSize(sampling, maxTopK) {
  const cap = maxTopK === undefined ? MAX_TOP_K : maxTopK;
  return sampling.temperature <= 0 ? 1 : Math.min(cap, Math.max(1, sampling.topK || cap));
}

/** AbortSignal.throwIfAborted for signals with or without that method (Node 12 has none). */
function throwIfAborted(signal) {
  if (!signal) return;
  if (typeof signal.throwIfAborted === 'function') {
    signal.throwIfAborted();
    return;
  }
  if (signal.aborted) {
    if (signal.reason !== undefined) throw signal.reason;
    const e = new Error('This operation was aborted');
    e.name = 'AbortError';
    throw e;
  }
}

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

  /** Copies the buffer back into a new Float32Array (f32) or Uint16Array (f16 bits). */
  download() {
    const n = this.rows * this.vocab;
    const out = this.dtype === F16 ? new Uint16Array(n) : new Float32Array(n);
    native.download(this.buffer, out);
    return out;
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
      // A NaN or +Infinity temperature is refused on every path (sampler.ts would sample
      // NaN weights), before any uniform is drawn.
      if (!(p.temperature < Infinity)) {
        throw new Error(`temperature must not be NaN or +Infinity, got ${p.temperature}`);
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
    const dev = logits instanceof DeviceLogits ? logits : this.stage(logits);
    if (dev.rows !== 1) throw new Error('sample() takes one row; use sampleBatch() for more');
    return this.sampleBatch(dev, [params], rng)[0];
  }

  /**
   * Greedy ids on the GPU (sampler.ts:13-23 per row): one launch over `logits` (a
   * DeviceLogits, or a Float32Array / Uint16Array row uploaded to the staging buffer), one
   * 4-byte-per-row readback. Returns an Int32Array, one id per row.
   */
  argmax(logits) {
    const dev = logits instanceof DeviceLogits ? logits : this.stage(logits);
    return native.argmax(this.handle, dev.buffer, dev.dtype, dev.rows, dev.vocab);
  }

  /** Uploads one host row into this Sampler's staging buffer (reused while it fits). */
  stage(row) {
    const dtype = dtypeOf(row);
    const s = this.staging;
    if (!s || s.vocab !== row.length || s.dtype !== dtype) {
      if (s) s.free();
      this.staging = new DeviceLogits(this.device, 1, row.length, dtype);
    }
    return this.staging.upload(row);
  }

  /**
   * The worker's decode loop (handleGenerate, inference.worker.ts:108-206) with this sampler
   * in place of encodeSampling + readback + sampleFromTopK: per token one launch on the
   * step's logits and one 48-byte result read back.
   *   opts.promptIds           the prompt's ids
   *   opts.prefill(ids)        -> Promise<DeviceLogits | Float32Array>: the last position's logits
   *   opts.decode(id)          -> Promise<DeviceLogits | Float32Array>: logits after `id`
   *   opts.sampling            {temperature, topK, topP, seed}: a SeededRandom(seed) per request
   *   opts.maxNewTokens, opts.stopTokens (ids), opts.isCancelled() (checked before every
   *   decode and again after its await), opts.onToken(id, index), opts.maxTopK (default 64:
   *   the worker's pool bound; the pool is poolSize(sampling, maxTopK))
   * Resolves to {tokens, stopped, cancelled, poolExhausted, readbackPerToken, totalReadback,
   * ttftMs, decodeMs}.
   */
  async generate(opts) {
    const sampling = opts.sampling;
    const stopTokens = new Set(opts.stopTokens || []);
    const isCancelled = opts.isCancelled || (() => false);
    const pool = poolSize(sampling, opts.maxTopK);
    const params = { temperature: sampling.temperature, topK: pool, topP: sampling.topP, seed: sampling.seed };
    const random = new SeededRandom(sampling.seed);
    const started = performance.now();
    const tokens = [];
    let stopped = false;
    let poolExhausted = false;
    let totalReadback = 0;
    let readbackPerToken = 0;

    const choose = (logits) => {
      const dev = logits instanceof DeviceLogits ? logits : this.stage(logits);
      const outcome = this.sampleBatch(dev, [params], random)[0];
      readbackPerToken = RESULT_BYTES;
      totalReadback += RESULT_BYTES;
      if (outcome.poolExhausted) poolExhausted = true;
      return outcome.id;
    };
    const emit = (id) => {
      tokens.push(id);
      if (opts.onToken) opts.onToken(id, tokens.length - 1);
    };
    const finish = (cancelled, ttftMs, decodeMs) => ({
      tokens, stopped, cancelled, poolExhausted, readbackPerToken, totalReadback, ttftMs, decodeMs,
    });

    let next = choose(await opts.prefill(opts.promptIds));
    const ttftMs = performance.now() - started;
    if (isCancelled()) return finish(true, ttftMs, 0);
    emit(next);
    if (stopTokens.has(next)) stopped = true;

    const decodeStart = performance.now();
    while (!stopped && tokens.length < opts.maxNewTokens) {
      if (isCancelled()) break;
      const logits = await opts.decode(next);
      // A cancel may land while the forward pass is busy: nothing is emitted after it.
      if (isCancelled()) break;
      next = choose(logits);
      emit(next);
      if (stopTokens.has(next)) stopped = true;
    }
    return finish(isCancelled(), ttftMs, performance.now() - decodeStart);
  }

  /**
   * Row softmax on the device (softmax_rows.wgsl's contract; bit for bit cpu.ts:238-264):
   * `x` and `out` are DeviceLogits-shaped f32 buffers of nRows x rowLen (`out` may be `x`).
   */
  softmaxRowsDevice(x, out, nRows, rowLen, causalPeriod, causalOffset) {
    native.softmaxRows(x.buffer, out.buffer, nRows, rowLen, causalPeriod || 0, causalOffset || 0);
    return out;
  }

  destroy() {
    if (this.staging) this.staging.free();
    this.staging = null;
    native.destroy(this.handle);
  }
}

// A Sampler grown to fit, for the module-level functions that mirror the reference's free
// functions (argmax, generateGreedy, softmaxRows).
let defaultSampler = null;
function samplerFor(vocab, rows) {
  const s = defaultSampler;
  if (!s || s.vocabMax < vocab || s.rowsMax < rows) {
    if (s) s.destroy();
    defaultSampler = new Sampler({ vocabMax: vocab, rowsMax: rows, kMax: MAX_TOP_K });
  }
  return defaultSampler;
}

/** sampler.ts:13-23 on the GPU: the id of the first maximum of one row (Float32Array,
 *  Uint16Array of f16 bits, or a one-row DeviceLogits). */
function argmax(logits) {
  const vocab = logits instanceof DeviceLogits ? logits.vocab : logits.length;
  return samplerFor(vocab, 1).argmax(logits)[0];
}

/**
 * generateGreedy (sampler.ts:54-76): greedy decoding against any function mapping the full
 * token sequence to next-token logits (a Float32Array or a one-row DeviceLogits), the argmax
 * taken on the GPU. options: {maxNewTokens, stopTokens, signal, onToken(id, index)}; an
 * optional Sampler to use. Resolves to {tokens, stopped, ms}.
 */
async function generateGreedy(promptIds, forward, options, sampler) {
  const stopTokens = new Set(options.stopTokens || []);
  const sequence = promptIds.slice();
  const tokens = [];
  const started = performance.now();
  for (let step = 0; step < options.maxNewTokens; step++) {
    throwIfAborted(options.signal);
    const logits = await forward(sequence);
    const vocab = logits instanceof DeviceLogits ? logits.vocab : logits.length;
    const next = (sampler || samplerFor(vocab, 1)).argmax(logits)[0];
    tokens.push(next);
    sequence.push(next);
    if (options.onToken) options.onToken(next, step);
    if (stopTokens.has(next)) return { tokens, stopped: true, ms: performance.now() - started };
  }
  return { tokens, stopped: false, ms: performance.now() - started };
}

/** softmaxRows (cpu.ts:238-264) computed on the GPU: a new Float32Array, bit for bit the
 *  CPU reference's. */
function softmaxRows(x, nRows, rowLen, causalPeriod, causalOffset) {
  if (!(x instanceof Float32Array) || x.length !== nRows * rowLen) {
    throw new Error(`softmaxRows: expected a Float32Array of ${nRows} x ${rowLen}`);
  }
  const s = samplerFor(1, 1);
  const dev = new DeviceLogits(s.device, nRows, rowLen, F32).upload(x);
  try {
    s.softmaxRowsDevice(dev, dev, nRows, rowLen, causalPeriod, causalOffset);
    return dev.download();
  } finally {
    dev.free();
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
  poolSize,
  MAX_TOP_K,
  argmax,
  generateGreedy,
  softmaxRows,
  encodeSampleBlock,
  decodeSampleBlock,
  DeviceLogits,
  SeededRandom,
  DEFAULT_SAMPLING,
  F32,
  F16,
  version: native.version,
};
