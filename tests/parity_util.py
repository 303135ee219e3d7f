"""Shared helpers for the GPU parity tests: tolerances, near-tie detection and seeded inputs."""
from __future__ import annotations

import os

import numpy as np

import orc_py as O
import synth

MARGIN_REL = 1e-3       # rows closer than this to a decision boundary are reported, not failed
LOGIT_RTOL = 2e-3       # logits: |got - want| <= 2e-3 * max(|want|, row RMS)
THREADS = max(1, min(16, os.cpu_count() or 1))


def logit_err(got: np.ndarray, want: np.ndarray) -> float:
    """Largest error in units of the tolerance scale max(|want|, rms(want))."""
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin), "non-finite pattern differs"
    if not fin.any():
        return 0.0
    rms = np.sqrt(np.mean(want[fin] ** 2))
    scale = np.maximum(np.abs(want[fin]), rms)
    return float(np.max(np.abs(got[fin] - want[fin]) / scale))


def greedy_near_tie(logits: np.ndarray) -> bool:
    top = np.sort(logits[np.isfinite(logits)])[-2:]
    if top.size < 2:
        return False
    return abs(float(top[1]) - float(top[0])) <= MARGIN_REL * max(abs(float(top[1])), 1e-30)


def sample_near_tie(info: O.SampleInfo, logits: np.ndarray, p: O.Params) -> bool:
    """True when the oracle's decision sits within MARGIN_REL of a boundary: the draw's CDF
    boundary, the nucleus threshold, or the shortlist boundary when it limits the cut."""
    if p.temperature <= 0:
        return greedy_near_tie(logits)
    d = info.denom
    if d > 0:
        if min(info.acc_at - info.r, info.r - info.acc_prev) <= MARGIN_REL * max(info.r, 1e-300):
            return True
    if p.top_p < 1.0 and info.nucleus_run > 0:
        tp = float(np.float32(p.top_p))
        if abs(info.nucleus_run - tp) <= MARGIN_REL * tp or abs(info.nucleus_prev - tp) <= MARGIN_REL * tp:
            return True
    if info.cut == info.shortlist and info.shortlist < logits.size:
        s = np.sort(logits[np.isfinite(logits)])[::-1]
        k = info.shortlist
        if k < s.size and abs(float(s[k - 1]) - float(s[k])) <= MARGIN_REL * max(abs(float(s[k - 1])), 1e-30):
            return True
    # ties among equal logits at the chosen rank are resolved by index on both sides
    return False


def oracle_row(W, S, B, gamma, hidden, p: O.Params, u: float, *, cap=30.0, eps=1e-6, normed=False,
               history=None, bias_ids=None, bias_values=None, ban=None):
    """Oracle decode tail for one row: returns (final logits, SampleInfo)."""
    l = O.head_logits(W, S, B, gamma, hidden, eps=eps, cap=cap, normed=normed, threads=THREADS)
    l = O.apply_modifiers(l, p, cap, history=history, bias_ids=bias_ids, bias_values=bias_values, ban=ban)
    return l, O.sample(l, p, u)


def bf16_round(x: np.ndarray) -> np.ndarray:
    return synth.bf16_to_f32(synth.f32_to_bf16(x))
