'use strict';
/*
 * Drives the Node host (tabby_amd/node/index.js) for tests/test_node_host.py.
 *   node node_host.js load                 -> prints the library version (no GPU needed)
 *   node node_host.js sample SPEC.json     -> writes SPEC.out: one outcome per row, sampled
 *                                             through Sampler.sampleBatch in one launch
 *   node node_host.js api                  -> exercises sample()/SeededRandom/errors, prints JSON
 *   node node_host.js wire JSON            -> {top, k, block64}: the encoded block of `top` (base64)
 *                                             and the decoding of block64 with k candidates
 * SPEC.json: {logits: path, dtype: "f32"|"f16", rows, vocab, topK[], temperature[], topP[],
 *             uniform[], topkCap, kMax, out}
 */
const fs = require('fs');
const path = require('path');
const tabby = require(path.join(__dirname, '..', 'tabby_amd', 'node', 'index.js'));

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
    s.destroy();
    console.log(JSON.stringify(report));
  } else {
    throw new Error(`unknown command ${cmd}`);
  }
}

main();
