"""Seeded, counter-based synthetic inputs for the decode tail (numpy only).

Every value is a pure function of (seed, stream, index): element i of a stream is
splitmix64's output for state base + (i + 1) * 0x9E3779B97F4A7C15, where base is
splitmix64(seed ^ stream * 0xD1B54A32D192ED03). Any slice can therefore be regenerated on its
own, and the same arrays come out on every machine.

Distributions (the configurations the benchmarks are quoted on):
  nibbles   uniform 0..15, packed low-nibble-first, [V][D/2] bytes
  scale     bf16(|N(0, 0.004)|)                 [V][D/64]
  bias      bf16(-8 * scale + N(0, 1e-4))       [V][D/64]  (scale as its bf16 value)
  gamma     bf16(1 + N(0, 0.02))                [D]
  hidden    fp32 N(0, 1)                        [B][D]
Normals use Box-Muller on two uniforms (the cosine branch); bf16 rounding is round-to-nearest-
even on the truncated mantissa (the reference's rule, tests/test_gpu_kernels.cpp:36-42).
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_MASK = (1 << 64) - 1

# stream ids
S_NIBBLES, S_SCALE, S_BIAS, S_GAMMA, S_HIDDEN = 1, 2, 3, 4, 5
S_HISTORY, S_BAN, S_BIAS_IDS, S_BIAS_VALS, S_PARAMS = 6, 7, 8, 9, 10


def _splitmix_scalar(x: int) -> int:
    x = (x + 0x9E3779B97F4A7C15) & _MASK
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _MASK
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _MASK
    return x ^ (x >> 31)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def u64(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    base = np.uint64(_splitmix_scalar((seed ^ (stream * 0xD1B54A32D192ED03)) & _MASK))
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(base + idx * _GAMMA)


def uniform(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    """float64 in [0, 1)."""
    return (u64(seed, stream, n, start) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    """float64 N(0, 1); draw i uses uniforms 2i and 2i+1 of the stream."""
    u = uniform(seed, stream, 2 * n, 2 * start)
    r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
    return r * np.cos(2.0 * np.pi * u[1::2])


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    w = (w + np.uint64(0x7FFF) + ((w >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return w.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def make_head(vocab: int, hidden: int, seed: int):
    """Returns (W uint8 [V][D/2], S uint16 [V][G], B uint16 [V][G], gamma uint16 [D])."""
    assert hidden % 64 == 0
    G = hidden // 64
    nbytes = vocab * hidden // 2
    W = np.empty(nbytes, dtype=np.uint8)
    chunk = 1 << 24  # u64 words per slice (128 MiB of output)
    nwords = (nbytes + 7) // 8
    for s in range(0, nwords, chunk):
        n = min(chunk, nwords - s)
        words = u64(seed, S_NIBBLES, n, s)
        b = words.view(np.uint8)
        lo = s * 8
        hi = min(nbytes, lo + b.size)
        W[lo:hi] = b[: hi - lo]
    W = W.reshape(vocab, hidden // 2)
    s = np.abs(normal(seed, S_SCALE, vocab * G) * 0.004).astype(np.float32)
    S = f32_to_bf16(s)
    sf = bf16_to_f32(S)
    bias = (-8.0 * sf.astype(np.float64) + normal(seed, S_BIAS, vocab * G) * 1e-4).astype(np.float32)
    B = f32_to_bf16(bias)
    gamma = f32_to_bf16((1.0 + normal(seed, S_GAMMA, hidden) * 0.02).astype(np.float32))
    return W, S.reshape(vocab, G), B.reshape(vocab, G), gamma


def hidden_states(batch: int, hidden: int, seed: int, step: int = 0) -> np.ndarray:
    """fp32 N(0, 1) [batch][hidden]; step selects a disjoint slice of the stream."""
    n = batch * hidden
    return normal(seed, S_HIDDEN, n, step * n).astype(np.float32).reshape(batch, hidden)


def uniform_ids(n: int, vocab: int, seed: int, stream: int = S_HISTORY, start: int = 0) -> np.ndarray:
    return np.minimum((uniform(seed, stream, n, start) * vocab).astype(np.int64), vocab - 1).astype(np.uint32)


def zipf_ids(n: int, vocab: int, s: float, seed: int, stream: int = S_HISTORY, start: int = 0) -> np.ndarray:
    """Zipf(s) over ranks 1..vocab by inverse CDF; rank r maps to id r - 1."""
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = uniform(seed, stream, n, start)
    return np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1).astype(np.uint32)


def ban_mask(vocab: int, frac: float, seed: int, row: int = 0) -> np.ndarray:
    """Bit i set with probability frac (independent per id). Returns uint32 [ceil(V/32)]."""
    u = uniform(seed, S_BAN, vocab, row * vocab)
    bits = (u < frac).astype(np.uint32)
    words = (vocab + 31) // 32
    pad = np.zeros(words * 32, dtype=np.uint32)
    pad[:vocab] = bits
    return (pad.reshape(words, 32) << np.arange(32, dtype=np.uint32)).sum(axis=1, dtype=np.uint64).astype(np.uint32)


def bias_list(n: int, vocab: int, lo: float, hi: float, seed: int, row: int = 0):
    ids = uniform_ids(n, vocab, seed, S_BIAS_IDS, row * n)
    vals = (lo + (hi - lo) * uniform(seed, S_BIAS_VALS, n, row * n)).astype(np.float32)
    return ids, vals
