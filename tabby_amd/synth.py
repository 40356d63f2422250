"""Synthetic workloads for the five configurations of the sampler benchmark.

Every random quantity comes from mulberry32 streams (the reference's generator,
src/engine/sampler.ts:105-119 and tests/support.ts:7-16), evaluated vectorised: the state
after i+1 steps is seed + (i+1)*0x6d2b79f5 mod 2^32, so a stream is a closed-form function
of its position. Normals use Box-Muller in f64 on pairs of draws. Logits are generated once
on the host and shared by the GPU run and the CPU oracle.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GOLDEN = np.uint64(0x6D2B79F5)
M32 = np.uint64(0xFFFFFFFF)


def mulberry32_stream(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Draws start..start+n-1 of SeededRandom(seed), as f64 (exact: u32 / 2^32)."""
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    s = (np.uint64(seed & 0xFFFFFFFF) + i * GOLDEN) & M32
    t = ((s ^ (s >> np.uint64(15))) * (s | np.uint64(1))) & M32
    t = t ^ ((t + (((t ^ (t >> np.uint64(7))) * (t | np.uint64(61))) & M32)) & M32)
    return ((t ^ (t >> np.uint64(14))) & M32).astype(np.float64) / 4294967296.0


def stream_seed(base: int, row: int, purpose: int) -> int:
    """A distinct, reproducible u32 seed per (base, row, purpose)."""
    x = (base * 0x9E3779B1 + row * 0x85EBCA77 + purpose * 0xC2B2AE3D) & 0xFFFFFFFF
    return int(mulberry32_stream(x, 1)[0] * 4294967296.0) ^ (purpose * 0x27D4EB2F & 0xFFFFFFFF)


def normals(seed: int, n: int, sigma: float) -> np.ndarray:
    """n draws of N(0, sigma^2): Box-Muller (cos branch) on consecutive pairs, f64."""
    u = mulberry32_stream(seed, 2 * n).reshape(n, 2)
    r = np.sqrt(-2.0 * np.log(1.0 - u[:, 0]))  # 1 - u is in (0, 1]
    return sigma * r * np.cos(2.0 * np.pi * u[:, 1])


def js_round(x: np.ndarray) -> np.ndarray:
    """JavaScript Math.round: half rounds toward +inf, and results in [-0.5, 0) are -0."""
    r = np.floor(x + 0.5)
    return np.where((r == 0.0) & (x < 0.0), -0.0, r)


@dataclass
class Workload:
    name: str
    logits: np.ndarray        # [rows, vocab], float32 or float16
    top_k: np.ndarray         # int32 [rows]
    temperature: np.ndarray   # f64 [rows]
    top_p: np.ndarray         # f64 [rows]
    uniform: np.ndarray       # f64 [rows]

    @property
    def rows(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    def logits_f32(self) -> np.ndarray:
        """The values the oracle sees: f16 is widened exactly."""
        return self.logits.astype(np.float32)


def _spiked_row(seed: int, vocab: int, sigma: float, spikes: int) -> np.ndarray:
    row = normals(stream_seed(seed, 0, 1), vocab, sigma)
    if spikes:
        u = mulberry32_stream(stream_seed(seed, 0, 2), 2 * spikes).reshape(spikes, 2)
        pos = np.minimum((u[:, 0] * vocab).astype(np.int64), vocab - 1)
        row[pos] += 12.0 + 6.0 * u[:, 1]  # spikes of +12..+18
    return row


def config(n: int, rows: int | None = None, vocab: int | None = None, seed: int = 2024) -> Workload:
    """BASELINE.json configs[n-1]; rows / vocab may be reduced for quick parity tests."""
    if n == 1:
        V = vocab or 49152
        row = normals(stream_seed(seed, 0, 1), V, 2.5).astype(np.float32)
        u = mulberry32_stream(stream_seed(seed, 0, 3), 1)
        return Workload("config1", row[None, :], np.array([40], np.int32), np.array([0.7]),
                        np.array([0.9]), u)
    if n == 2:
        V = vocab or 151936
        row = _spiked_row(seed, V, 3.0, 8).astype(np.float32)
        u = mulberry32_stream(stream_seed(seed, 0, 3), 1)
        return Workload("config2", row[None, :], np.array([50], np.int32), np.array([0.8]),
                        np.array([0.9]), u)
    if n in (3, 4):
        R = rows or (256 if n == 3 else 64)
        V = vocab or 151936
        logits = np.empty((R, V), dtype=np.float32 if n == 3 else np.float16)
        for r in range(R):
            logits[r] = _spiked_row(stream_seed(seed + n, r, 0), V, 3.0, 8)
        pick = mulberry32_stream(stream_seed(seed + n, 0, 5), 4 * R).reshape(R, 4)
        if n == 3:
            temperature = np.array([0.5, 0.7, 1.0])[(pick[:, 0] * 3).astype(int)]
            top_k = np.array([1, 20, 50, 100], np.int32)[(pick[:, 1] * 4).astype(int)]
            top_p = np.array([0.8, 0.95, 1.0])[(pick[:, 2] * 3).astype(int)]
        else:
            temperature = np.full(R, 0.3)
            top_k = np.zeros(R, np.int32)
            top_p = np.full(R, 0.95)
        return Workload(f"config{n}", logits, top_k, temperature, top_p, pick[:, 3].copy())
    if n == 5:
        R = rows or 512
        V = vocab or 151936
        logits = np.empty((R, V), dtype=np.float32)
        for r in range(R):
            z = normals(stream_seed(seed + 5, r, 0), V, 2.0)
            q = js_round(z * 4.0) * 0.25
            masked = mulberry32_stream(stream_seed(seed + 5, r, 1), V) < 0.3
            q[masked] = -np.inf
            logits[r] = q
        u = mulberry32_stream(stream_seed(seed + 5, 0, 5), R)
        return Workload("config5", logits, np.full(R, 1024, np.int32), np.full(R, 1.0),
                        np.full(R, 0.98), u)
    raise ValueError(f"no config {n}")


def random_workload(rows: int, vocab: int, seed: int, k_choices=(1, 5, 40, 64), ties: bool = False,
                    neg_inf_frac: float = 0.0, temperatures=(0.0, 0.5, 1.0, 2.0),
                    top_ps=(0.5, 0.9, 1.0), sigma: float = 3.0) -> Workload:
    """Assorted rows for parity tests: optional coarse rounding (ties) and -inf masking."""
    logits = np.empty((rows, vocab), dtype=np.float32)
    for r in range(rows):
        z = normals(stream_seed(seed, r, 0), vocab, sigma)
        if ties:
            z = js_round(z * 2.0) * 0.5
        if neg_inf_frac > 0:
            z[mulberry32_stream(stream_seed(seed, r, 1), vocab) < neg_inf_frac] = -np.inf
        logits[r] = z
    pick = mulberry32_stream(stream_seed(seed, 0, 5), 4 * rows).reshape(rows, 4)
    t = np.asarray(temperatures, dtype=np.float64)[(pick[:, 0] * len(temperatures)).astype(int)]
    k = np.asarray(k_choices, dtype=np.int32)[(pick[:, 1] * len(k_choices)).astype(int)]
    p = np.asarray(top_ps, dtype=np.float64)[(pick[:, 2] * len(top_ps)).astype(int)]
    return Workload(f"random{seed}", logits, k, t, p, pick[:, 3].copy())


# ---------------------------------------------------------------------------------------
# The lm_head: int4 block-quantized weights and hidden states (the fused lm_head + sampling
# path). Generated the way the reference's own tests generate them.
# ---------------------------------------------------------------------------------------

def random_f32(count: int, seed: int, scale: float = 1.0, start: int = 0) -> np.ndarray:
    """tests/support.ts:19-24 (randomF32): fround((u * 2 - 1) * scale) for draws start.. of
    SeededRandom(seed)."""
    u = mulberry32_stream(seed, count, start)
    return ((u * 2.0 - 1.0) * scale).astype(np.float32)


def quantize_q4(values: np.ndarray, rows: int, cols: int, block: int = 32):
    """tests/quant.test.ts:83-120 (quantizeQ4 + packScalesF16): per block, the value of
    largest magnitude (the first such) gives scale = peak / -8; levels are
    clamp(round(v / scale + 8), 0, 15) with JavaScript's Math.round, eight per u32 word
    (value j at bits 4j); scales are rounded to f16 (round to nearest even).
    Returns (words u32 [rows * cols / 8], scales_f16 bits u16 [rows * cols / block],
    scales_f32 (the f16 values widened) [rows * cols / block])."""
    v = np.asarray(values, np.float32).reshape(rows, cols // block, block).astype(np.float64)
    first_peak = np.argmax(np.abs(v), axis=2)
    peak = np.take_along_axis(v, first_peak[..., None], axis=2)[..., 0]
    scale = peak / -8.0
    inverse = np.divide(1.0, scale, out=np.zeros_like(scale), where=scale != 0.0)
    level = np.clip(js_round(v * inverse[..., None] + 8.0), 0, 15).astype(np.uint32).reshape(-1, 8)
    words = np.zeros(level.shape[0], dtype=np.uint32)
    for j in range(8):
        words |= level[:, j] << np.uint32(4 * j)
    scales_f16 = scale.astype(np.float32).astype(np.float16).reshape(-1)
    return words, scales_f16.view(np.uint16), scales_f16.astype(np.float32)


def lm_head_q4(vocab: int, hidden: int, block: int = 32, seed: int = 7):
    """A random-init int4 lm_head of vocab x hidden in the reference's layout: every 4-bit
    code uniform in 0..15 (the words are mulberry32 draws), each block's scale
    +-(0.04 .. 0.05) / 8 rounded to f16 -- the magnitude quantize_q4 gives weights drawn as
    the reference's quant test draws them (randomF32 * 0.05). Returns (words u32
    [vocab * hidden / 8], scales_f16 bits u16 [vocab * hidden / block], scales_f32)."""
    words = (mulberry32_stream(seed, vocab * hidden // 8) * 4294967296.0).astype(np.uint32)
    u = mulberry32_stream(seed ^ 0x5CA1E, vocab * hidden // block)
    mag = (0.04 + 0.01 * u) / 8.0
    sign = np.where(mulberry32_stream(seed ^ 0x519, u.size) < 0.5, 1.0, -1.0)
    scales_f16 = (sign * mag).astype(np.float32).astype(np.float16)
    return words, scales_f16.view(np.uint16), scales_f16.astype(np.float32)


def hidden_states(rows: int, hidden: int, seed: int = 0x1234, scale: float = 6.0) -> np.ndarray:
    """rows x hidden f32 activations, randomF32 * scale (scale 6 puts the lm_head's logits
    near N(0, 3^2), the spread of the sampler's configurations)."""
    return random_f32(rows * hidden, seed, scale).reshape(rows, hidden)
