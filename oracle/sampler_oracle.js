'use strict';
/*
 * Node restatement of the reference CPU sampler -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/ and bench.py's cpu_baseline leg run this file. It is written for Node 12
 * (CommonJS, no `?.`/`??`), the Node in this image, and it calls V8's own Math.exp, the
 * exp the reference's sampler runs on. Semantics follow:
 *   SeededRandom     src/engine/sampler.ts:105-119
 *   argmax           src/engine/sampler.ts:13-23
 *   topK             src/engine/sampler.ts:25-30
 *   sampleFromTopK   src/engine/sampler.ts:147-212
 *   sumExp           tests/sampling.test.ts:73-77
 *   sampleRow        encodeSampling (src/engine/forward.ts:522-601) + sampleFromTopK, with
 *                    topK = 0 meaning the whole vocabulary
 *   softmaxRows      src/reference/cpu.ts:238-264 (f32 = Math.fround)
 *   matmulQuantized  src/reference/cpu.ts:352-393 (f32 = Math.fround)
 */

class SeededRandom {
  constructor(seed) {
    this.state = seed >>> 0;
  }

  next() {
    // u32 add, then two multiply-xorshift rounds; the result has 32 significant bits.
    const s = (this.state + 0x6d2b79f5) >>> 0;
    this.state = s;
    let t = Math.imul(s ^ (s >>> 15), s | 1);
    t = (t ^ (t + Math.imul(t ^ (t >>> 7), t | 61))) | 0;
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  }
}

function argmax(row) {
  let best = 0;
  for (let i = 1; i < row.length; i++) if (row[i] > row[best]) best = i;
  return best;
}

// Value descending, then id ascending. A difference that is NaN (inf - inf) counts as a tie.
function byValueThenId(a, b) {
  const d = b.value - a.value;
  if (d > 0 || d < 0) return d;
  return a.id - b.id;
}

function topK(row, k) {
  const all = new Array(row.length);
  for (let i = 0; i < row.length; i++) all[i] = { id: i, value: row[i] };
  all.sort(byValueThenId);
  return all.slice(0, k);
}

function sumExp(row, maxLogit) {
  let sum = 0;
  for (let i = 0; i < row.length; i++) sum += Math.exp(row[i] - maxLogit);
  return sum;
}

function sampleFromTopK(top, params, uniformSource) {
  const ids = top.ids;
  const logits = top.logits;
  const n = ids.length;
  if (n === 0) throw new Error('sampleFromTopK: empty candidate set');

  const exact = new Float64Array(n);
  for (let i = 0; i < n; i++) exact[i] = Math.exp(logits[i] - top.maxLogit) / top.sumExp;
  let poolMass = 0;
  for (let i = 0; i < n; i++) poolMass += exact[i];

  if (params.temperature <= 0) {
    return { id: ids[0], probability: exact[0], consideredCount: 1, poolMass, poolExhausted: false };
  }

  const w = new Float64Array(n);
  for (let i = 0; i < n; i++) w[i] = Math.exp((logits[i] - top.maxLogit) / params.temperature);
  let scaledTotal = 0;
  for (let i = 0; i < n; i++) scaledTotal += w[i];
  for (let i = 0; i < n; i++) w[i] = w[i] / scaledTotal;

  let cut = n;
  let poolExhausted = false;
  if (params.topP < 1) {
    let cumulative = 0;
    for (let i = 0; i < n; i++) {
      cumulative += w[i];
      if (cumulative >= params.topP) {
        cut = i + 1;
        break;
      }
    }
    poolExhausted = poolMass < params.topP;
  }

  let total = 0;
  for (let i = 0; i < cut; i++) total += w[i];
  const u = typeof uniformSource === 'number' ? uniformSource : uniformSource.next();
  const target = u * total;
  let running = 0;
  let chosen = cut - 1;
  for (let i = 0; i < cut; i++) {
    running += w[i];
    if (target < running) {
      chosen = i;
      break;
    }
  }
  return {
    id: ids[chosen],
    probability: exact[chosen],
    consideredCount: cut,
    poolMass,
    poolExhausted,
  };
}

// One row end to end. `row` is a Float32Array; `uniform` a number in [0,1). With
// topkCap > 0 the outcome also carries the first topkCap ids of the sorted pool.
function sampleRow(row, params, uniform, topkCap) {
  const k = params.topK <= 0 || params.topK >= row.length ? row.length : params.topK;
  const cands = topK(row, k);
  const maxLogit = cands[0].value;
  const top = {
    maxLogit,
    sumExp: sumExp(row, maxLogit),
    ids: cands.map((c) => c.id),
    logits: cands.map((c) => c.value),
  };
  const outcome = sampleFromTopK(top, params, uniform);
  outcome.maxLogit = maxLogit;
  outcome.sumExp = top.sumExp;
  if (topkCap > 0) outcome.topIds = top.ids.slice(0, topkCap);
  return outcome;
}

// Row softmax with a causal prefix: each row's first `valid` entries are normalised in f32
// steps, the rest set to 0. Returns a new Float32Array.
function softmaxRows(x, nRows, rowLen, causalPeriod, causalOffset) {
  const f32 = Math.fround;
  const period = causalPeriod || 0;
  const offset = causalOffset || 0;
  const out = Float32Array.from(x);
  for (let row = 0; row < nRows; row++) {
    const valid = period !== 0 ? offset + (row % period) + 1 : rowLen;
    const base = row * rowLen;
    let maxV = out[base];
    for (let i = 1; i < valid; i++) maxV = Math.max(maxV, out[base + i]);
    let sum = 0;
    for (let i = 0; i < valid; i++) {
      const e = f32(Math.exp(f32(out[base + i] - maxV)));
      out[base + i] = e;
      sum = f32(sum + e);
    }
    const inv = f32(1 / sum);
    for (let i = 0; i < valid; i++) out[base + i] = f32(out[base + i] * inv);
    for (let i = valid; i < rowLen; i++) out[base + i] = 0;
  }
  return out;
}

// y[t, m] = sum_k dequant(w[m, k]) * x[t, k] + bias[m]: per word, an f32 partial sum of its
// values, scaled by the block's scale and added to the row's f32 accumulator.
function matmulQuantized(words, scales, x, nTokens, outDim, inDim, bits, blockSize, bias) {
  const f32 = Math.fround;
  const perWord = bits === 4 ? 8 : 4;
  const shift = 32 / perWord;
  const mask = (1 << shift) - 1;
  const wordsPerRow = inDim / perWord;
  const wordsPerBlock = blockSize / perWord;
  const blocksPerRow = inDim / blockSize;
  const y = new Float32Array(nTokens * outDim);
  for (let t = 0; t < nTokens; t++) {
    const xBase = t * inDim;
    for (let m = 0; m < outDim; m++) {
      const wBase = m * wordsPerRow;
      const sBase = m * blocksPerRow;
      let acc = 0;
      for (let w = 0; w < wordsPerRow; w++) {
        const word = words[wBase + w];
        const scale = scales[sBase + Math.floor(w / wordsPerBlock)];
        const k0 = w * perWord;
        let partial = 0;
        for (let j = 0; j < perWord; j++) {
          const raw = (word >>> (j * shift)) & mask;
          const centred = bits === 4 ? raw - 8 : raw > 127 ? raw - 256 : raw;
          partial = f32(partial + f32(centred * x[xBase + k0 + j]));
        }
        acc = f32(acc + f32(partial * scale));
      }
      if (bias) acc = f32(acc + bias[m]);
      y[t * outDim + m] = acc;
    }
  }
  return y;
}

module.exports = { SeededRandom, argmax, topK, sumExp, sampleFromTopK, sampleRow, softmaxRows, matmulQuantized };
