'use strict';
/*
 * Drives the Node host (tabby_amd/node/index.js) for tests/test_node_host.py.
 *   node node_host.js load                 -> prints the library version (no GPU needed)
 *   node node_host.js sample SPEC.json     -> writes SPEC.out: one outcome per row, sampled
 *                                             through Sampler.sampleBatch in one launch
 *   node node_host.js api                  -> exercises sample()/SeededRandom/errors, prints JSON
 *   node node_host.js wire JSON            -> {top, k, block64}: the encoded block of `top` (base64)
 *                                             and the decoding of block64 with k candidates
 *   node node_host.js decode VOCAB         -> the decode loop (Sampler.generate) on a synthetic
 *                                             model, against the CPU restatement's replay
 *   node node_host.js greedy VOCAB         -> generateGreedy / argmax against the CPU argmax
 *   node node_host.js softmax SPEC.json    -> softmaxRows on the GPU ({x, nRows, rowLen,
 *                                             period, offset, out})
 * SPEC.json: {logits: path, dtype: "f32"|"f16", rows, vocab, topK[], temperature[], topP[],
 *             uniform[], topkCap, kMax, out}
 */
const fs = require('fs');
const path = require('path');
const tabby = require(path.join(__dirname, '..', 'tabby_amd', 'node', 'index.js'));
const cpu = require(path.join(__dirname, '..', 'oracle', 'sampler_oracle.js'));

// A deterministic stand-in for the forward pass: the next position's logits as a function of
// the whole sequence (mulberry32 seeded by an FNV-1a hash of the ids), spread over [-6, 6)
// with a few peaks, so that sampling at T = 0.9 has real choices to make.
function fakeLogits(seq, vocab) {
  let h = 0x811c9dc5;
  for (const id of seq) {
    h ^= id;
    h = Math.imul(h, 0x01000193) >>> 0;
  }
  const rng = new cpu.SeededRandom(h);
  const row = new Float32Array(vocab);
  for (let i = 0; i < vocab; i++) row[i] = (rng.next() - 0.5) * 12;
  for (let j = 0; j < 6; j++) row[Math.floor(rng.next() * vocab)] = 7 + rng.next() * 3;
  return row;
}

// The worker's loop replayed on the CPU restatement (inference.worker.ts:108-206 with
// sampleFromTopK over a poolSize pool): the ids the GPU loop must reproduce.
function replayOnCpu(prompt, sampling, maxNewTokens, stopTokens, vocab) {
  const random = new cpu.SeededRandom(sampling.seed);
  const pool = tabby.poolSize(sampling);
  const seq = prompt.slice();
  const tokens = [];
  const stop = new Set(stopTokens || []);
  const choose = () => {
    const u = sampling.temperature > 0 ? random.next() : 0;
    const o = cpu.sampleRow(fakeLogits(seq, vocab), { temperature: sampling.temperature, topK: pool,
                                                       topP: sampling.topP }, u, 0);
    return o.id;
  };
  let next = choose();
  tokens.push(next);
  let stopped = stop.has(next);
  while (!stopped && tokens.length < maxNewTokens) {
    seq.push(next);
    next = choose();
    tokens.push(next);
    if (stop.has(next)) stopped = true;
  }
  return { tokens, stopped };
}

async function runLoop(s, vocab, sampling, maxNewTokens, extra) {
  const seq = [11, 22, 33, 44];
  const dev = new tabby.DeviceLogits(0, 1, vocab, tabby.F32);
  const x = extra || {};
  let decodes = 0;
  const out = await s.generate({
    promptIds: seq.slice(),
    prefill: async (ids) => dev.upload(fakeLogits(ids, vocab)),
    decode: async (id) => {
      seq.push(id);
      decodes++;
      if (x.cancelOnDecode && decodes === x.cancelOnDecode) x.cancelled = true;
      return dev.upload(fakeLogits(seq, vocab));
    },
    sampling,
    maxNewTokens,
    stopTokens: x.stopTokens,
    isCancelled: () => !!x.cancelled,
    onToken: (id, index) => { if (x.seen) x.seen.push([id, index]); },
  });
  dev.free();
  out.decodes = decodes;
  return out;
}

async function decodeReport(vocab) {
  const s = new tabby.Sampler({ vocabMax: vocab, rowsMax: 1, kMax: 64 });
  const warm = (seed) => ({ temperature: 0.9, topK: 40, topP: 0.95, seed });
  const cold = (seed) => ({ temperature: 0, topK: 1, topP: 1, seed });
  const report = {};
  // sampling.test.ts:151-204: seed 42 twice, seed 43, and temperature 0 under two seeds.
  report.seed42 = await runLoop(s, vocab, warm(42), 24);
  report.seed42again = await runLoop(s, vocab, warm(42), 24);
  report.seed43 = await runLoop(s, vocab, warm(43), 24);
  report.greedy1 = await runLoop(s, vocab, cold(1), 10);
  report.greedy999 = await runLoop(s, vocab, cold(999), 10);
  report.cpu = {
    seed42: replayOnCpu([11, 22, 33, 44], warm(42), 24, [], vocab),
    seed43: replayOnCpu([11, 22, 33, 44], warm(43), 24, [], vocab),
    greedy1: replayOnCpu([11, 22, 33, 44], cold(1), 10, [], vocab),
  };
  // A whole-vocabulary intent (topK 0) runs at the worker's pool, 64.
  report.topK0 = await runLoop(s, vocab, { temperature: 1.1, topK: 0, topP: 0.9, seed: 5 }, 12);
  report.cpu.topK0 = replayOnCpu([11, 22, 33, 44], { temperature: 1.1, topK: 0, topP: 0.9, seed: 5 }, 12, [], vocab);
  // A stop token: the 7th id of the seed-42 run ends the loop at its first occurrence.
  const stopId = report.seed42.tokens[6];
  const seen = [];
  report.stop = await runLoop(s, vocab, warm(42), 24, { stopTokens: [stopId], seen });
  report.stop.seen = seen;
  report.stopId = stopId;
  report.cpu.stop = replayOnCpu([11, 22, 33, 44], warm(42), 24, [stopId], vocab);
  // A cancel that lands while the third decode is in flight: nothing after it is emitted.
  report.cancelInFlight = await runLoop(s, vocab, warm(42), 24, { cancelOnDecode: 3 });
  // A cancel before the first token: the prefill's id is not emitted.
  report.cancelFirst = await runLoop(s, vocab, warm(42), 24, { cancelled: true });
  s.destroy();
  return report;
}

async function greedyReport(vocab) {
  const forward = async (ids) => fakeLogits(ids, vocab);
  const report = {};
  const seen = [];
  report.plain = await tabby.generateGreedy([5, 6, 7], forward, { maxNewTokens: 12, onToken: (id, i) => seen.push([id, i]) });
  report.seen = seen;
  const cpuTokens = [];
  const seq = [5, 6, 7];
  for (let i = 0; i < 12; i++) {
    const id = cpu.argmax(fakeLogits(seq, vocab));
    cpuTokens.push(id);
    seq.push(id);
  }
  report.cpuTokens = cpuTokens;
  report.stopped = await tabby.generateGreedy([5, 6, 7], forward, { maxNewTokens: 12, stopTokens: [cpuTokens[4]] });
  const signal = { aborted: false };
  const aborted = [];
  try {
    await tabby.generateGreedy([5, 6, 7], forward, {
      maxNewTokens: 12, signal, onToken: (id, i) => { aborted.push(id); if (i === 3) signal.aborted = true; },
    });
    report.abortError = null;
  } catch (e) {
    report.abortError = e.name;
  }
  report.abortedTokens = aborted;
  // argmax on special rows, through the module-level function (sampler.ts:13-23).
  const rows = [];
  const r1 = new Float32Array(vocab).fill(-Infinity); rows.push(r1);
  const r2 = new Float32Array(vocab).fill(2); r2[0] = NaN; rows.push(r2);
  const r3 = new Float32Array(vocab).fill(-1); r3[vocab - 1] = 4; r3[vocab - 2] = 4; rows.push(r3);
  const r4 = new Float32Array(vocab).fill(0); r4[3] = -0; r4[9] = NaN; rows.push(r4);
  report.special = rows.map((r) => [tabby.argmax(r), cpu.argmax(r)]);
  return report;
}

function main() {
  const cmd = process.argv[2];
  if (cmd === 'load') {
    console.log(JSON.stringify({ version: tabby.version() }));
  } else if (cmd === 'wire') {
    const spec = JSON.parse(process.argv[3]);
    const enc = Buffer.from(tabby.encodeSampleBlock(spec.top, spec.k)).toString('base64');
    const b = Buffer.from(spec.block64, 'base64');
    const raw = b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength);
    console.log(JSON.stringify({ encoded: enc, decoded: tabby.decodeSampleBlock(raw, spec.k) }));
  } else if (cmd === 'sample') {
    const spec = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
    const buf = fs.readFileSync(spec.logits);
    const data = spec.dtype === 'f16'
      ? new Uint16Array(buf.buffer, buf.byteOffset, buf.byteLength / 2)
      : new Float32Array(buf.buffer, buf.byteOffset, buf.byteLength / 4);
    const s = new tabby.Sampler({ vocabMax: spec.vocab, rowsMax: spec.rows, kMax: spec.kMax });
    const dev = s.upload(data, spec.rows, spec.vocab);
    const params = [];
    for (let r = 0; r < spec.rows; r++) {
      params.push({ temperature: spec.temperature[r], topK: spec.topK[r], topP: spec.topP[r], seed: 0 });
    }
    const out = s.sampleBatch(dev, params, spec.uniform, { topK: spec.topkCap });
    dev.free();
    s.destroy();
    fs.writeFileSync(spec.out, JSON.stringify(out));
  } else if (cmd === 'decode' || cmd === 'greedy') {
    const vocab = Number(process.argv[3]);
    const run = cmd === 'decode' ? decodeReport(vocab) : greedyReport(vocab);
    run.then((r) => console.log(JSON.stringify(r)), (e) => { console.error(e); process.exit(1); });
  } else if (cmd === 'softmax') {
    const spec = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
    const buf = fs.readFileSync(spec.x);
    const x = new Float32Array(buf.buffer.slice(buf.byteOffset, buf.byteOffset + buf.byteLength));
    const y = tabby.softmaxRows(x, spec.nRows, spec.rowLen, spec.period, spec.offset);
    fs.writeFileSync(spec.out, Buffer.from(y.buffer, y.byteOffset, y.byteLength));
  } else if (cmd === 'api') {
    const vocab = 5000;
    const row = new Float32Array(vocab);
    const rng0 = new tabby.SeededRandom(7);
    for (let i = 0; i < vocab; i++) row[i] = (rng0.next() - 0.5) * 8;
    const s = new tabby.Sampler({ vocabMax: vocab, rowsMax: 1, kMax: 64 });
    const report = {};
    // sample(): greedy consumes no uniform; a non-greedy call consumes exactly one.
    const rng = new tabby.SeededRandom(42);
    report.greedy = s.sample(row, { temperature: 0, topK: 40, topP: 0.9 }, rng);
    report.stateAfterGreedy = rng.state;
    report.sampled = s.sample(row, tabby.DEFAULT_SAMPLING, rng);
    report.stateAfterSample = rng.state;
    report.row = Array.from(row);
    try {
      s.sample(row, { temperature: 0.7, topK: 65, topP: 0.9 }, rng);
      report.topKError = null;
    } catch (e) {
      report.topKError = e.message;
    }
    report.stateAfterError = rng.state;
    // A NaN or +Infinity temperature is refused before a uniform is drawn; -0 is greedy.
    report.temperatureErrors = [NaN, Infinity].map((t) => {
      try {
        s.sample(row, { temperature: t, topK: 40, topP: 0.9 }, rng);
        return null;
      } catch (e) {
        return e.message;
      }
    });
    report.stateAfterTemperatureErrors = rng.state;
    report.negZero = s.sample(row, { temperature: -0, topK: 40, topP: 0.9 }, rng);
    report.stateAfterNegZero = rng.state;
    s.destroy();
    console.log(JSON.stringify(report));
  } else {
    throw new Error(`unknown command ${cmd}`);
  }
}

main();
