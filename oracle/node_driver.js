'use strict';
/*
 * Command-line driver for the Node restatement -- TEST INFRASTRUCTURE ONLY.
 *
 *   node node_driver.js exp IN.f64 OUT.f64          Math.exp over a file of f64
 *   node node_driver.js mulberry SEED N OUT.f64     N draws of SeededRandom(SEED)
 *   node node_driver.js sample SPEC.json            rows of an f32 file through sampleRow
 *   node node_driver.js bench SPEC.json             time sampleRow (single thread, or
 *                                                   worker_threads when spec.threads > 1)
 *   node node_driver.js softmax SPEC.json           softmaxRows over an f32 file
 *                                                   ({x, nRows, rowLen, period, offset, out})
 *   node node_driver.js argmax SPEC.json            argmax of each row of an f32 file
 *                                                   ({logits, rows, vocab, out: JSON ids})
 *   node node_driver.js matmulq SPEC.json           matmulQuantized ({words: u32 file, scales:
 *                                                   f32 file, x: f32 file, bias: f32 file or
 *                                                   null, nTokens, outDim, inDim, bits,
 *                                                   blockSize, out: f32 file})
 *
 * SPEC.json: {logits: path (f32, row-major), rows, vocab, topK[], temperature[], topP[],
 *             uniform[], out: path (JSON outcomes), topkCap, threads, seconds}
 */
const fs = require('fs');
const os = require('os');
const path = require('path');
const oracle = require('./sampler_oracle.js');

function readF64(file) {
  const buf = fs.readFileSync(file);
  return new Float64Array(buf.buffer, buf.byteOffset, buf.byteLength / 8);
}

function writeF64(file, arr) {
  fs.writeFileSync(file, Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));
}

function readRows(spec) {
  const buf = fs.readFileSync(spec.logits);
  const all = new Float32Array(buf.buffer, buf.byteOffset, buf.byteLength / 4);
  const rows = [];
  for (let r = 0; r < spec.rows; r++) rows.push(all.subarray(r * spec.vocab, (r + 1) * spec.vocab));
  return rows;
}

function paramsOf(spec, r) {
  return { temperature: spec.temperature[r], topK: spec.topK[r], topP: spec.topP[r], seed: 0 };
}

function runRows(spec, rows, first, count) {
  const out = [];
  for (let i = 0; i < count; i++) {
    const r = (first + i) % spec.rows;
    out.push(oracle.sampleRow(rows[r], paramsOf(spec, r), spec.uniform[r], spec.topkCap || 0));
  }
  return out;
}

function benchSingle(spec, rows) {
  // Rows are cycled until the time budget is spent; inputs were generated outside.
  const budgetMs = 1000 * (spec.seconds || 10);
  const started = process.hrtime.bigint();
  let done = 0;
  for (;;) {
    runRows(spec, rows, done, 1);
    done++;
    const elapsedMs = Number(process.hrtime.bigint() - started) / 1e6;
    if (elapsedMs >= budgetMs || (spec.maxRows && done >= spec.maxRows)) {
      return { rows: done, seconds: elapsedMs / 1000 };
    }
  }
}

function main() {
  const cmd = process.argv[2];
  if (cmd === 'exp') {
    const x = readF64(process.argv[3]);
    const y = new Float64Array(x.length);
    for (let i = 0; i < x.length; i++) y[i] = Math.exp(x[i]);
    writeF64(process.argv[4], y);
  } else if (cmd === 'mulberry') {
    const rng = new oracle.SeededRandom(Number(process.argv[3]));
    const n = Number(process.argv[4]);
    const y = new Float64Array(n);
    for (let i = 0; i < n; i++) y[i] = rng.next();
    writeF64(process.argv[5], y);
  } else if (cmd === 'sample') {
    const spec = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
    const rows = readRows(spec);
    fs.writeFileSync(spec.out, JSON.stringify(runRows(spec, rows, 0, spec.rows)));
  } else if (cmd === 'bench') {
    const spec = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
    const threads = spec.threads || 1;
    if (threads <= 1) {
      const rows = readRows(spec);
      const r = benchSingle(spec, rows);
      process.stdout.write(JSON.stringify({
        rows: r.rows, seconds: r.seconds, rowsPerSec: r.rows / r.seconds, threads: 1,
        node: process.version, cpu: os.cpus()[0].model,
      }) + '\n');
      return;
    }
    const { Worker } = require('worker_threads');
    const results = [];
    let pending = threads;
    const started = process.hrtime.bigint();
    for (let t = 0; t < threads; t++) {
      const w = new Worker(path.join(__dirname, 'node_driver.js'), {
        argv: ['worker'], workerData: spec,
      });
      w.on('message', (m) => {
        results.push(m);
        if (--pending === 0) {
          const wall = Number(process.hrtime.bigint() - started) / 1e9;
          const rows = results.reduce((a, b) => a + b.rows, 0);
          process.stdout.write(JSON.stringify({
            rows, seconds: wall, rowsPerSec: results.reduce((a, b) => a + b.rows / b.seconds, 0),
            threads, node: process.version, cpu: os.cpus()[0].model,
          }) + '\n');
        }
      });
      w.on('error', (e) => { process.stderr.write(String(e) + '\n'); process.exit(1); });
    }
  } else if (cmd === 'softmax') {
    const spec = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
    const buf = fs.readFileSync(spec.x);
    const x = new Float32Array(buf.buffer, buf.byteOffset, buf.byteLength / 4);
    const y = oracle.softmaxRows(x, spec.nRows, spec.rowLen, spec.period, spec.offset);
    fs.writeFileSync(spec.out, Buffer.from(y.buffer, y.byteOffset, y.byteLength));
  } else if (cmd === 'argmax') {
    const spec = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
    fs.writeFileSync(spec.out, JSON.stringify(readRows(spec).map((row) => oracle.argmax(row))));
  } else if (cmd === 'matmulq') {
    const spec = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
    const view = (file, T) => {
      const b = fs.readFileSync(file);
      return new T(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength));
    };
    const y = oracle.matmulQuantized(view(spec.words, Uint32Array), view(spec.scales, Float32Array),
                                     view(spec.x, Float32Array), spec.nTokens, spec.outDim, spec.inDim,
                                     spec.bits, spec.blockSize, spec.bias ? view(spec.bias, Float32Array) : null);
    fs.writeFileSync(spec.out, Buffer.from(y.buffer, y.byteOffset, y.byteLength));
  } else if (cmd === 'worker') {
    const { parentPort, workerData } = require('worker_threads');
    const rows = readRows(workerData);
    parentPort.postMessage(benchSingle(workerData, rows));
  } else {
    process.stderr.write('usage: node node_driver.js exp|mulberry|sample|bench ...\n');
    process.exit(2);
  }
}

main();
