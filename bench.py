#!/usr/bin/env python3
"""Benchmark of the sampling hot path on one MI355X.

A step is one launch of the sampler over one batch: 256 rows x 151,936 f32 logits
(BASELINE.json's headline: top-k 50, top-p 0.9), from device-resident logits, parameters and
results (tabby_sampler_sample_device). Prints ONE JSON line with rows/s, achieved HBM GB/s
of the sampling kernel against MI355X's 8 TB/s, and the Node CPU baseline timed on this
host in the same run.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S] [--no-cpu]
       python bench.py --config N | --host-params | --read-ceiling | --greedy | --softmax
                       (secondary measurements, one JSON line each)
       python bench.py --timeline  (the headline row kernel's phase times, from the timeline
                       build of the library: tabby_amd/lib/libtabby_sampler_timeline.so)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E, AMD's published figure
ROTATE = 4              # distinct input batches per rotation: 4 x 155.6 MB > 256 MB MALL


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--rows", type=int, default=256)
    ap.add_argument("--vocab", type=int, default=151936)
    ap.add_argument("--top-k", type=int, default=50)
    ap.add_argument("--top-p", type=float, default=0.9)
    ap.add_argument("--mixed-params", action="store_true",
                    help="config 3's per-row mix of k/T/p instead of k=50, p=0.9 on every row")
    ap.add_argument("--dtype", choices=["f32", "f16"], default="f32")
    ap.add_argument("--config", type=int, choices=[1, 2, 3, 4, 5], default=None,
                    help="run BASELINE.json's configs[N-1] exactly as generated (parameters, "
                         "dtype and shape) instead of the headline; a secondary measurement")
    ap.add_argument("--guess-fails", action="store_true",
                    help="with --config 5: raise every row's finite logits in the chunks its "
                         "first bound samples by 20, so that pool_row_kernel's guessed bound "
                         "leaves too few candidates on every row and each row is taken again at "
                         "the certain bound; a diagnostic of that path's cost")
    ap.add_argument("--host-params", action="store_true",
                    help="time the host-parameter entry (tabby_sampler_sample: parameters uploaded "
                         "and results read back every call, synchronously) instead of the "
                         "device-resident one; a secondary, PCIe-inclusive measurement")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of known size (reference for the "
                         "FETCH_SIZE / WRITE_SIZE counters) and print its JSON line")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="time a plain read of the headline's rotated logit batches with the "
                         "sampling kernels' own 16-byte nontemporal loads and launch shape "
                         "(tabby_debug_stream_read): the practical read ceiling; also the "
                         "kernel whose FETCH_SIZE calibrates the counter for those loads")
    ap.add_argument("--greedy", action="store_true",
                    help="time the greedy fast path (tabby_argmax_device) on the headline's "
                         "logits; a secondary measurement")
    ap.add_argument("--lmhead", action="store_true",
                    help="time the lm_head fused with sampling (tabby_sampler_sample_lmhead_q4_device) "
                         "against the unfused pair (tabby_lmhead_q4_device, then the sampler) on "
                         "Qwen2.5-0.5B's lm_head shape (151,936 x 896 int4, block 32), one decode "
                         "row (--rows up to 8); a secondary measurement")
    ap.add_argument("--timeline", action="store_true",
                    help="run the headline workload on the timeline build of the library (the "
                         "row kernel with phase timestamps compiled in) and print the phases' "
                         "percentiles over the rows of the last call, in us; a diagnostic")
    ap.add_argument("--timeline-raw", metavar="PATH", default=None,
                    help="with --timeline: also save the last call's raw stamps (rows x 32 "
                         "slots, int64) to PATH as .npy")
    ap.add_argument("--softmax", action="store_true",
                    help="time the attention row softmax (tabby_softmax_rows_device) on a "
                         "prefill shape: 14 heads x 512 queries over 512 positions, causal; a "
                         "secondary measurement")
    return ap.parse_args()


def copy_calibration() -> int:
    """A plain copy of 256 MiB, 10 times: each launch reads and writes exactly 256 MiB, so
    the counters' KiB per dispatch over 262,144 KiB is their scale factor."""
    import torch
    n = 64 * 1024 * 1024  # f32 elements: 256 MiB
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_kib_read_per_launch": n * 4 // 1024,
                      "copy_kib_written_per_launch": n * 4 // 1024, "launches": 10}), flush=True)
    return 0


MEDIAN_RUNS = 7  # repeated timed loops whose median is reported beside the contract's mean


def _timed(fn, steps: int, warmup: int, stream) -> float:
    """Average duration (us) of `steps` back-to-back calls of fn(i), between two HIP events on
    the launch stream, after `warmup` untimed calls."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / steps


def secondary(args) -> int:
    """--read-ceiling, --greedy, --softmax: one JSON line each, not the headline metric."""
    import numpy as np
    import torch

    from tabby_amd import sampler as S
    from tabby_amd import synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    if args.softmax:
        heads, queries = 14, 512
        n_rows, row_len = heads * queries, 512
        g = torch.Generator(device="cpu").manual_seed(7)
        xs = [(torch.randn(n_rows * row_len, generator=g) * 3).to(dev) for _ in range(ROTATE)]
        outs = [torch.empty_like(x) for x in xs]
        us = _timed(lambda i: S.softmax_rows(xs[i % ROTATE], n_rows, row_len, queries, 0,
                                             out=outs[i % ROTATE], stream=stream),
                    args.steps, args.warmup, stream)
        # Each row's causal prefix read once (row r covers r % 512 + 1 entries), every row
        # written once (the masked rest as zeros).
        moved = heads * sum(q + 1 for q in range(queries)) * 4 + n_rows * row_len * 4
        print(json.dumps({
            "metric": "attention row softmax (softmaxRows), 14x512 rows x 512 f32, causal",
            "value": round(moved / (us * 1e-6) / 1e9, 1), "unit": "GB/s", "us_per_call": round(us, 2),
            "rows_per_s": round(n_rows / (us * 1e-6), 1), "bytes_per_call": moved,
            "roofline": {"bound": "hbm", "achieved": round(moved / (us * 1e-6) / 1e9, 1),
                         "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                         "frac": round(moved / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)},
            "dtype": "f32", "data": "synthetic N(0, 3^2) scores, 4 rotated buffers"}), flush=True)
        return 0
    if args.lmhead:
        return lmhead_bench(args, dev, stream)
    w = synth.config(3, rows=args.rows, vocab=args.vocab)
    base = torch.from_numpy(w.logits).to(dev)
    buffers = [torch.roll(base, shifts=(b * 61) % w.rows, dims=0).contiguous() for b in range(ROTATE)]
    del base
    nbytes = w.rows * w.vocab * 4
    if args.read_ceiling:
        sink = torch.zeros(w.rows, dtype=torch.int32, device=dev)
        us = _timed(lambda i: S.stream_read(buffers[i % ROTATE], sink, stream=stream),
                    args.steps, args.warmup, stream)
        gbps = nbytes / (us * 1e-6) / 1e9
        print(json.dumps({
            "metric": "plain read of the headline's logits (read ceiling), 256x151936 f32",
            "value": round(gbps, 1), "unit": "GB/s", "us_per_call": round(us, 2),
            "bytes_per_call": nbytes, "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4),
            "kernel": "stream_read_kernel: one 1,024-lane workgroup per row, 16-byte nontemporal "
                      "loads, 4 in flight per lane, nothing else",
            "data": "config-3 logits, 4 rotated device batches"}), flush=True)
        return 0
    # --greedy
    ids = torch.zeros(w.rows, dtype=torch.int32, device=dev)
    with S.GpuSampler(vocab_max=w.vocab, rows_max=w.rows, k_max=64) as g:
        us = _timed(lambda i: g.argmax_device(buffers[i % ROTATE], ids, stream=stream),
                    args.steps, args.warmup, stream)
        g.argmax_device(buffers[0], ids, stream=stream)
        torch.cuda.synchronize()
    got = ids.cpu().numpy()
    oracle = _oracle()
    logits = w.logits_f32()
    pick = np.linspace(0, w.rows - 1, 16).astype(int)
    bad = [int(r) for r in pick if oracle.argmax(logits[r]) != int(got[r])]
    gbps = nbytes / (us * 1e-6) / 1e9
    print(json.dumps({
        "metric": "greedy rows/sec (argmax fast path), 256x151936 f32 logits",
        "value": round(w.rows / (us * 1e-6), 1), "unit": "rows/s", "us_per_call": round(us, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4)},
        "bytes_per_call": nbytes, "dtype": "f32",
        "data": "config-3 logits, 4 rotated device batches",
        "parity": {"rows_checked": len(pick), "mismatched_rows": bad}}), flush=True)
    return 1 if bad else 0


def lmhead_bench(args, dev, stream) -> int:
    """--lmhead: the fused lm_head + sampling call against the unfused pair, Qwen2.5-0.5B's
    lm_head (151,936 x 896 int4, block 32) and k 40 / p 0.9 / T 0.7 (DEFAULT_SAMPLING)."""
    import numpy as np
    import torch

    from tabby_amd import sampler as S
    from tabby_amd import synth

    vocab, hidden, block = 151936, 896, 32
    rows = min(args.rows, 8) if args.rows != 256 else 1
    words, f16, f32 = synth.lm_head_q4(vocab, hidden, block)
    # Four packed copies of the weights and scales (4 x 76.6 MB > the 256 MB MALL), rotated
    # with the hidden states, so that every call reads its weights from HBM as a decode step
    # does (one lm_head pass per token, the weights evicted by the rest of the model between).
    heads = [S.LmHeadQ4(words, f16, vocab, hidden, block) for _ in range(ROTATE)]
    head = heads[0]
    xs = [torch.from_numpy(synth.hidden_states(rows, hidden, seed=11 + b)).to(dev) for b in range(ROTATE)]
    params = np.zeros(rows, dtype=S.PARAMS_DTYPE)
    params["temperature"], params["top_k"], params["top_p"] = 0.7, 40, 0.9
    params["uniform"] = synth.mulberry32_stream(5, rows)
    pdev = torch.from_numpy(params.view(np.uint8).copy()).to(dev)
    res = torch.zeros(rows * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device=dev)
    logits = torch.empty((rows, vocab), dtype=torch.float32, device=dev)
    g = S.GpuSampler(vocab_max=vocab, rows_max=max(rows, 1), k_max=64)
    fused_us = _timed(lambda i: g.sample_lmhead_q4_device(heads[i % ROTATE], xs[i % ROTATE], pdev, res,
                                                          stream=stream),
                      args.steps, args.warmup, stream)

    def unfused(i):
        heads[i % ROTATE].logits(xs[i % ROTATE], out=logits, stream=stream)
        g.sample_device(logits, pdev, res, stream=stream)
    unfused_us = _timed(unfused, args.steps, args.warmup, stream)
    gemv_us = _timed(lambda i: heads[i % ROTATE].logits(xs[i % ROTATE], out=logits, stream=stream),
                     args.steps, args.warmup, stream)
    # The answer of the fused call against the oracle (matmulQuantized, then the sampler).
    fused = g.sample_lmhead_q4(head, xs[0], params)
    g.close()
    oracle = _oracle()
    ref_logits = oracle.matmul_quantized(words, f32, xs[0].cpu().numpy(), vocab, hidden)
    bad = [r for r in range(rows)
           if oracle.sample_row(ref_logits[r], 40, 0.7, 0.9, float(params["uniform"][r]))["id"] != int(fused["id"][r])]
    weight_bytes = words.nbytes + f16.nbytes
    print(json.dumps({
        "metric": f"lm_head + sampling per decode step, 151936x896 int4 (block 32), {rows} row(s)",
        "value": round(fused_us, 2), "unit": "us", "higher_is_better": False,
        "fused_us": round(fused_us, 2), "unfused_us": round(unfused_us, 2), "gemv_only_us": round(gemv_us, 2),
        "weight_bytes": weight_bytes,
        "roofline": {"bound": "hbm", "achieved": round(weight_bytes / (fused_us * 1e-6) / 1e9, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(weight_bytes / (fused_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)},
        "dtype": "int4 weights, f32 arithmetic",
        "data": "random-init int4 weights (synth.lm_head_q4) in 4 rotated device copies (306 MB, read "
                "from HBM), randomF32 hidden states, 4 rotated",
        "parity": {"rows_checked": rows, "mismatched_rows": bad}}), flush=True)
    return 1 if bad else 0


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # test infrastructure: the CPU leg only (checker and baseline)
    return oracle


def oracle_check(w, res, rows_to_check: int = 16) -> dict:
    """The CPU leg's checker: the C oracle on a sample of the batch's rows against the GPU's
    results for them (ids, consideredCount and maxLogit exact; probability, poolMass and
    sumExp within 1e-5 relative). Outside the timed region."""
    import numpy as np
    oracle = _oracle()
    pick = np.unique(np.linspace(0, w.rows - 1, min(rows_to_check, w.rows)).astype(int))
    logits = w.logits_f32()
    bad = []
    for r in pick:
        o = oracle.sample_row(logits[r], int(w.top_k[r]), float(w.temperature[r]),
                              float(w.top_p[r]), float(w.uniform[r]))
        g = res[r]
        ok = (int(g["status"]) == o["status"] == 0 and int(g["id"]) == o["id"]
              and int(g["considered"]) == o["considered"]
              and np.float32(g["max_logit"]) == np.float32(o["max_logit"]))
        for f in ("probability", "pool_mass", "sum_exp"):
            ok = ok and abs(float(g[f]) - o[f]) <= 1e-5 * abs(o[f])
        if not ok:
            bad.append(int(r))
    return {"rows_checked": int(pick.size), "mismatched_rows": bad}


def cpu_baseline(w, seconds: float) -> dict | None:
    """The Node restatement of the reference CPU sampler (topK sort + sampleFromTopK) on a
    bounded sample of the same rows, single-threaded and across all host cores."""
    oracle = _oracle()

    if not oracle.node_available():
        return None
    import numpy as np
    sample_rows = min(w.rows, 32)
    args = (w.logits_f32()[:sample_rows], w.top_k[:sample_rows], w.temperature[:sample_rows],
            w.top_p[:sample_rows], w.uniform[:sample_rows])
    single = oracle.node_bench(*args, seconds=seconds, threads=1)
    # One worker per host core (Node's os.cpus().length), as the baseline plan states; the CPUs
    # this process may actually run on (affinity and any cgroup quota) are reported beside.
    cores = os.cpu_count() or 1
    multi = oracle.node_bench(*args, seconds=seconds, threads=cores)
    return {
        "value": round(multi["rowsPerSec"], 2),
        "unit": "rows/s",
        "cores": multi["threads"],
        "kind": "port",
        "sample": (f"Node {multi['node']} restatement of sampler.ts (full-row topK sort + "
                   f"sampleFromTopK, V8 Math.exp) over {sample_rows} rows of this workload, "
                   f"cycled for ~{seconds:.0f} s per leg; {multi['rows']} rows on "
                   f"{multi['threads']} worker_threads ({multi['cpu']})"),
        "single_thread": {"value": round(single["rowsPerSec"], 2), "unit": "rows/s", "cores": 1,
                          "rows": single["rows"], "seconds": round(single["seconds"], 2)},
        "usable_cpus": _usable_cpus(),
    }


def _usable_cpus() -> dict:
    """The host's logical CPUs, those this process may run on, and the cgroup CPU quota (if
    any): the worker count above is the first; the rate is whatever the others allow."""
    out = {"host": os.cpu_count()}
    try:
        out["affinity"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            out["cgroup_quota"] = round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        pass
    return out


# The kernels one call of each workload launches (the roofline's "kernel" field).
CALL_KERNELS = {
    None: "row_kernel, one workgroup per row (streaming: max, sum-exp, candidates; then in LDS "
          "the exact top-k, top-p and draw)",
    1: "row_kernel, one workgroup streaming the row and sampling it",
    2: "row_kernel on parts of the row, then wave_merge_kernel merging their lists and sampling",
    3: "row_kernel, one workgroup per row (streaming: max, sum-exp, candidates; then in LDS "
       "the exact top-k, top-p and draw)",
    4: "row_kernel on parts of each row, wave_merge_kernel (statistics, head key, top list), "
       "then the head kernels (head_kernel re-reads the row for its head, head_fast_kernel "
       "finishes it; head_sort_kernel and head_finish_kernel for rows it cannot)",
    5: "pool_row_kernel, one workgroup per row (streaming with candidate appends; then in LDS "
       "the exact top-1024 selection, its sort, top-p and the draw)",
}


def cu_pairs(where, end, pct):
    """Percentiles of the earlier and the later stream end among workgroups that shared a CU."""
    import numpy as np
    first, second = [], []
    for cu in np.unique(where):
        e = np.sort(end[where == cu])
        if len(e) >= 2:
            first.append(e[0])
            second.append(e[-1])
    if not first:
        return None
    return {"cus": len(first), "earlier": pct(np.array(first)), "later": pct(np.array(second))}


def timeline(args) -> int:
    """--timeline: the headline's row_kernel phases, from the timeline library's stamps."""
    import ctypes

    import numpy as np
    import torch

    from tabby_amd import build as B
    from tabby_amd import sampler as S
    from tabby_amd import synth

    lib = S.load_library(B.TIMELINE_LIB_PATH)  # before anything loads the plain library
    lib.tabby_debug_timeline.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.tabby_debug_timeline.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    pool = args.config == 5  # config 5: pool_row_kernel's phases instead of row_kernel's
    if pool:
        w = synth.config(5)
    else:
        w = synth.config(3, rows=args.rows, vocab=args.vocab)
        w.top_k[:] = args.top_k
        w.top_p[:] = args.top_p
    base = torch.from_numpy(w.logits).to(dev)
    params = np.zeros(w.rows, dtype=S.PARAMS_DTYPE)
    params["temperature"], params["top_p"] = w.temperature, w.top_p
    params["uniform"], params["top_k"] = w.uniform, w.top_k
    buffers, pbufs = [], []
    for b in range(ROTATE):
        shift = (b * 61) % w.rows
        buffers.append(torch.roll(base, shifts=shift, dims=0).contiguous())
        pbufs.append(torch.from_numpy(np.roll(params, shift).view(np.uint8).copy()).to(dev))
    results = torch.zeros(w.rows * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device=dev)
    sampler = S.GpuSampler(vocab_max=w.vocab, rows_max=w.rows, k_max=max(64, int(w.top_k.max())))
    stream = torch.cuda.current_stream()
    for i in range(args.warmup + args.steps):
        sampler.sample_device(buffers[i % ROTATE], pbufs[i % ROTATE], results, stream=stream)
    torch.cuda.synchronize()
    slots, groups = 32, 1024
    tl = np.zeros(groups * slots, dtype=np.uint64)
    if lib.tabby_debug_timeline(tl.ctypes.data, tl.nbytes) != 0:
        print("bench: tabby_debug_timeline failed", file=sys.stderr)
        return 1
    tl = tl.reshape(groups, slots)[: w.rows].astype(np.int64)
    if args.timeline_raw:
        np.save(args.timeline_raw, tl)
    start, rt0, rt1 = tl[:, 16], tl[:, 24], tl[:, 25]
    # Shader-clock ticks per us, from each row's start-to-end in both clocks (real time: 100 MHz).
    rate = float(np.median((tl[:, 21] - start) / ((rt1 - rt0) * 1e-2)))
    waves = (tl[:, :16] - start[:, None]) / rate
    last = waves.max(1)

    def pct(a):
        return {p: round(float(np.percentile(a, q)), 2) for p, q in (("p0", 0), ("p50", 50), ("max", 100))}

    if pool:
        phases = {
            "first_bound_ready": pct((tl[:, 22] - start) / rate),
            "first_wave_stream_end": pct(waves.min(1)),
            "last_wave_stream_end": pct(last),
            "barrier_after_stream": pct((tl[:, 17] - start) / rate - last),
            "selection": pct((tl[:, 18] - tl[:, 17]) / rate),
            "selection_key_passes": pct((tl[:, 23] - tl[:, 17]) / rate),
            "selection_index_passes": pct((tl[:, 18] - tl[:, 23]) / rate),
            "gather": pct((tl[:, 19] - tl[:, 18]) / rate),
            "sort": pct((tl[:, 20] - tl[:, 19]) / rate),
            "sample_from_pool": pct((tl[:, 21] - tl[:, 20]) / rate),
            "row_end": pct((rt1 - rt0.min()) * 1e-2),
        }
        print(json.dumps({
            "metric": "pool_row_kernel phase times (us from each row's start; later phases as "
                      f"durations), config 5, last of {args.warmup + args.steps} calls",
            "unit": "us", "rows": w.rows, "vocab": w.vocab, "shader_clock_mhz": round(rate, 1),
            "phases": phases,
            "candidates_per_row": {p: int(v) for p, v in pct(tl[:, 31]).items()},
            # Rows whose guessed first bound left fewer than k candidates (taken again at the
            # certain bound).
            "rows_taken_again": int(np.count_nonzero(tl[:, 29] == 1)),
            "key_passes_per_row": {p: int(v) for p, v in pct(tl[:, 26]).items()},
            "stream_end_by_wave": [round(float(x), 2) for x in waves.mean(0)],
            # The two workgroups on each CU (slot 30: XCC and CU): the earlier and the later
            # to end its stream (us from the first row's start, real time).
            "stream_end_on_cu": cu_pairs(tl[:, 30], last + (rt0 - rt0.min()) * 1e-2, pct),
            "library": os.path.relpath(B.TIMELINE_LIB_PATH, ROOT),
        }))
        return 0
    phases = {
        "first_bound_ready": pct((tl[:, 22] - start) / rate),
        "first_wave_stream_end": pct(waves.min(1)),
        "last_wave_stream_end": pct(last),
        "selection_by_last_wave": pct((tl[:, 29] - start) / rate - last),
        "first_tail_barrier_passed": pct((tl[:, 17] - start) / rate - last),
        "take": pct((tl[:, 18] - tl[:, 17]) / rate),
        "second_tail_barrier": pct((tl[:, 19] - tl[:, 18]) / rate),
        "stats_fold_and_sort": pct((tl[:, 20] - tl[:, 19]) / rate),
        "register_tail": pct((tl[:, 21] - tl[:, 20]) / rate),
        # Inside the register tail (rows that sample; greedy rows skip the draw's stamps).
        "reg_tail_terms": pct((tl[:, 23] - tl[:, 20]) / rate),
        "reg_tail_scans": pct((tl[:, 26] - tl[:, 23]) / rate),
        "reg_tail_cut_and_draw": pct((tl[:, 27] - tl[:, 26]) / rate),
        "reg_tail_margins": pct((tl[:, 28] - tl[:, 27]) / rate),
        "reg_tail_result": pct((tl[:, 21] - tl[:, 28]) / rate),
        "tail_after_last_wave": pct((tl[:, 21] - start) / rate - last),
        "row_end": pct((rt1 - rt0.min()) * 1e-2),
    }
    print(json.dumps({
        "metric": "row_kernel phase times (us from each row's start; tail phases as durations), "
                  f"headline workload, last of {args.warmup + args.steps} calls",
        "unit": "us", "rows": w.rows, "vocab": w.vocab, "shader_clock_mhz": round(rate, 1),
        "phases": phases,
        # Mean stream end by wave index (waves w, w + 4, w + 8, w + 12 share a SIMD, oldest
        # first), and by XCD (workgroup i runs on XCD i mod 8).
        "stream_end_by_wave": [round(float(x), 2) for x in waves.mean(0)],
        "last_wave_end_by_xcd": [round(float(last[np.arange(w.rows) % 8 == x].mean()), 2) for x in range(8)],
        "library": os.path.relpath(B.TIMELINE_LIB_PATH, ROOT),
    }))
    return 0


def main() -> int:
    args = parse_args()
    if args.copy_calibration:
        return copy_calibration()
    if args.timeline:
        if args.gpus != 1:
            print("bench.py measures one GPU only", file=sys.stderr)
            return 2
        return timeline(args)
    if args.read_ceiling or args.greedy or args.softmax or args.lmhead:
        if args.gpus != 1:
            print("bench.py measures one GPU only", file=sys.stderr)
            return 2
        return secondary(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the sampler is "
              f"single-device in this build; rows shard across GPUs with no communication.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from tabby_amd import sampler as S
    from tabby_amd import synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # Workload: config-3 logits (N(0, 3^2) + 8 spikes of +12..+18 per row), generated on the
    # host once; params per row from config 3, with k/p overridden to the headline's.
    if args.config is not None:
        w = synth.config(args.config)
        if args.guess_fails:
            if args.config != 5:
                print("bench: --guess-fails applies to --config 5", file=sys.stderr)
                return 2
            # The sample: claims v < 32 take chunk (v mod 16) s + v // 16, s the largest power of
            # two with 16 s <= the row's chunks (pool_row_kernel's claim order).
            nch = -(-w.vocab // 1024)
            s = 1
            while 32 * s <= nch:
                s *= 2
            sampled = np.zeros(w.vocab, dtype=bool)
            for v in range(32):
                c = (v % 16) * s + v // 16
                sampled[c * 1024:(c + 1) * 1024] = True
            block = w.logits[:, sampled]
            w.logits[:, sampled] = np.where(np.isfinite(block), block + 20.0, block)
    else:
        w = synth.config(3, rows=args.rows, vocab=args.vocab)
        if not args.mixed_params:
            w.top_k[:] = args.top_k
            w.top_p[:] = args.top_p
        if args.dtype == "f16":
            w.logits = w.logits.astype(np.float16)
    itemsize = w.logits.dtype.itemsize
    bytes_per_launch = w.rows * w.vocab * itemsize

    base = torch.from_numpy(w.logits).to(dev)
    params = np.zeros(w.rows, dtype=S.PARAMS_DTYPE)
    params["temperature"], params["top_p"] = w.temperature, w.top_p
    params["uniform"], params["top_k"] = w.uniform, w.top_k
    # ROTATE distinct device batches (rows rolled, params rolled with them).
    buffers, pbufs = [], []
    for b in range(ROTATE):
        shift = (b * 61) % w.rows
        buffers.append(torch.roll(base, shifts=shift, dims=0).contiguous())
        pbufs.append(torch.from_numpy(np.roll(params, shift).view(np.uint8).copy()).to(dev))
    del base
    results = torch.zeros(w.rows * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device=dev)
    k_max = max(64, int(w.top_k.max()))
    sampler = S.GpuSampler(vocab_max=w.vocab, rows_max=w.rows, k_max=k_max)
    stream = torch.cuda.current_stream()

    kcap = 256 if k_max <= 256 else 1024
    whole = bool(np.any((w.top_k <= 0) | (w.top_k >= w.vocab))) and w.vocab > kcap
    flags = S.TABBY_FLAG_FULL_VOCAB if whole else 0

    hparams = [np.roll(params, (b * 61) % w.rows) for b in range(ROTATE)]

    def step(i: int) -> None:
        if args.host_params:
            res_h, _, _ = sampler.sample_params(buffers[i % ROTATE], hparams[i % ROTATE],
                                                stream=stream)
            if res_h["status"].any():
                raise RuntimeError("bench: a row returned a nonzero status")
            return
        sampler.sample_device(buffers[i % ROTATE], pbufs[i % ROTATE], results, flags=flags,
                              stream=stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    res = results.cpu().numpy().view(S.RESULT_DTYPE)
    bad = int(np.count_nonzero(res["status"]))
    if bad:
        print(f"bench: {bad} rows returned a nonzero status", file=sys.stderr)
        return 1

    # Timed region: K back-to-back launches between two HIP events on the launch stream. (An
    # event recorded between every pair of calls costs the stream ~8 us per call on this GPU,
    # so per-call events would measure the events.)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(args.steps):
        step(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_ms = start.elapsed_time(end) / args.steps

    ms_per_step = 1000.0 * wall / args.steps
    rows_per_s = w.rows * args.steps / wall
    achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9

    # The median over repeated runs of the same timed loop (untimed by the driver's contract,
    # reported beside the mean): each run is K back-to-back calls between two events.
    run_means = []
    for _ in range(MEDIAN_RUNS):
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for i in range(args.steps):
            step(i)
        s1.record(stream)
        torch.cuda.synchronize()
        run_means.append(s0.elapsed_time(s1) * 1000.0 / args.steps)
    median_us = float(np.median(run_means))

    # The answer of a timed call, checked after the timed region: batch 0 is the workload's
    # own row order (the others are rotations of it).
    if args.host_params:
        res, _, _ = sampler.sample_params(buffers[0], hparams[0], stream=stream)
    else:
        results.zero_()
        sampler.sample_device(buffers[0], pbufs[0], results, flags=flags, stream=stream)
        torch.cuda.synchronize()
        res = results.cpu().numpy().view(S.RESULT_DTYPE)
    sampler.close()
    check = oracle_check(w, res)

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "sample_kernel_config3_traffic.json")
    headline = (args.config is None and args.dtype == "f32" and not args.mixed_params
                and not args.host_params)
    if os.path.exists(tpath) and headline:
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    cpu = None if args.no_cpu else cpu_baseline(w, args.cpu_seconds)

    dtype_name = "f16" if w.logits.dtype == np.float16 else "f32"
    if args.config is None:
        metric = "sampled rows/sec + achieved HBM GB/s, 256x151936 fp32 logits, top-k50/top-p0.9"
        config = {
            "workload": ("config3-mixed" if args.mixed_params else "config3-headline")
                        + ("-host-params" if args.host_params else ""),
            "rows": w.rows, "vocab": w.vocab,
            "top_k": "per-row {1,20,50,100}" if args.mixed_params else args.top_k,
            "top_p": "per-row {0.8,0.95,1.0}" if args.mixed_params else args.top_p,
            "temperature": "per-row {0.5,0.7,1.0}",
            "parallelism": "single GPU",
        }
    else:
        metric = (f"sampled rows/sec + achieved HBM GB/s, BASELINE configs[{args.config - 1}] "
                  f"({w.rows}x{w.vocab} {dtype_name})")
        ks = sorted(set(int(k) for k in w.top_k))
        config = {"workload": f"config{args.config}" + ("-guess-fails" if args.guess_fails else ""),
                  "rows": w.rows, "vocab": w.vocab,
                  "top_k": ks if len(ks) > 1 else ks[0],
                  "top_p": sorted(set(float(p) for p in w.top_p)),
                  "temperature": sorted(set(float(t) for t in w.temperature)),
                  "parallelism": "single GPU"}
    if args.host_params:
        metric += "; host-parameter entry, PCIe-inclusive (upload, sample, read back, sync)"
        if args.config is not None:
            config["workload"] += "-host-params"
    out = {
        "metric": metric,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_name,
        "data": "synthetic (mulberry32 + Box-Muller, seeded per config; 4 rotated device batches)",
        "config": config,
        "hbm_gbps": round(bytes_per_launch * args.steps / wall / 1e9, 1),
        "kernel_us_avg": round(avg_ms * 1000, 2),
        "kernel_us_median": {"runs": MEDIAN_RUNS, "steps_per_run": args.steps,
                             "us": round(median_us, 2),
                             "min_max_us": [round(min(run_means), 2), round(max(run_means), 2)]},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
            "kernel": (f"one tabby_sampler_sample_device call = {CALL_KERNELS.get(args.config, CALL_KERNELS[None])}; "
                       "duration = HIP-event time of the back-to-back timed calls / steps")
                      if not args.host_params else
                      ("one synchronous tabby_sampler_sample call (parameter upload, the "
                       "sampling kernels, result read-back); duration = HIP-event time / steps"),
            "bytes_per_launch": bytes_per_launch,
            "duration_us": round(avg_ms * 1000, 2),
        },
        "cpu_baseline": cpu,
        "parity": check,
    }
    print(json.dumps(out), flush=True)
    if check["mismatched_rows"]:
        print(f"bench: rows {check['mismatched_rows']} differ from the CPU oracle", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
