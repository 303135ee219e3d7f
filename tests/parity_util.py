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


def oracle_row(W, S, B, gamma, hidden, p: O.Params, u: float, *, cap=30.0, eps=1e-6, normed=False,
               history=None, bias_ids=None, bias_values=None, ban=None):
    """Oracle decode tail for one row: returns (final logits, SampleInfo)."""
    l = O.head_logits(W, S, B, gamma, hidden, eps=eps, cap=cap, normed=normed, threads=THREADS)
    l = O.apply_modifiers(l, p, cap, history=history, bias_ids=bias_ids, bias_values=bias_values, ban=ban)
    return l, O.sample(l, p, u)


def bf16_round(x: np.ndarray) -> np.ndarray:
    return synth.bf16_to_f32(synth.f32_to_bf16(x))


# ---- CDF-interval token checks ---------------------------------------------------------------
#
# A sampled token is accepted when the uniform's target r = u * denom falls inside the token's
# cumulative-weight interval (before, after] in the oracle's survivor order (logit descending, id
# ascending; src/sampling.cpp:122-168, tests/test_sampling.cpp:36-84), widened by a stated
# epsilon. The epsilon is either
#   * "arith": the error the GPU's own arithmetic can make on the SAME logits (used when the
#     oracle sampler runs on the GPU's final logits), or
#   * "margin": MARGIN_REL of r and of top_p, the stated near-tie rule, for rows whose logits come
#     from the oracle chain and so differ from the GPU's within the logit tolerance.
# A token outside the widened interval fails, whatever the row's margin: a selector off by one
# rank misses it unless r lies within epsilon of that one boundary.
#
# GPU arithmetic behind "arith":
#   * full-vocabulary rows: every weight is the hardware exp2 of an fp32 argument,
#     w = exp2(fl(fl(l - m) * fl(log2(e) / T))): at most 3 * 2^-24 * |l - m| / T relative from the
#     argument, 2^-22 from exp2, and 2^-40 absolute from the u64 fixed-point histogram bins (whose
#     sums are then exact integers). The same bound holds for the T = 1 weights of the nucleus and
#     for Z.
#   * shortlist rows: the draw weights exp((l - m) / T) and the nucleus probabilities
#     exp(l - m) / Z are double precision; Z comes from fp32 block sums of 64 hardware exp2 values
#     (relative error below 2e-5).
FULL_VOCAB_FLAG = 1
SHORTLIST_Z_REL = 2e-5
SHORTLIST_DRAW_REL = 1e-12


def _survivor_model(l: np.ndarray, p: O.Params):
    """Oracle survivor order and weights of one row, as numpy double arrays."""
    ld = l.astype(np.float64)
    V = ld.size
    order = np.lexsort((np.arange(V), -ld))
    ls = ld[order]
    m = ls[0]
    with np.errstate(invalid="ignore", over="ignore"):
        d = np.where(np.isfinite(ls), ls - m, -np.inf)
        w1 = np.exp(d)
    full = p.top_k == 0 and (p.flags & FULL_VOCAB_FLAG) != 0
    want = min(p.top_k, V) if p.top_k > 0 else (V if full else min(256, V))
    return order, d, w1, full, want


def draw_check(logits: np.ndarray, p: O.Params, u: float, token: int, *, mode: str = "arith",
               ref_logits: np.ndarray | None = None) -> str:
    """'exact' when `token` is the oracle's token on `logits` (or on ref_logits for mode "margin"),
    'within' when only the widened interval admits it; raises AssertionError otherwise.

    mode "arith": `logits` are the GPU's final logits and epsilon is the GPU arithmetic's bound.
    mode "margin": `logits` are the oracle chain's logits and epsilon is MARGIN_REL (of r for the
    draw, of top_p for the nucleus)."""
    l = np.ascontiguousarray(logits, dtype=np.float32)
    info = O.sample(l, p, u)
    if token == info.token:
        return "exact"
    if p.temperature <= 0.0:
        if mode == "margin" and greedy_near_tie(l):
            top = np.sort(l[np.isfinite(l)])[-1]
            assert abs(float(l[token]) - float(top)) <= MARGIN_REL * max(abs(float(top)), 1e-30), \
                (token, info.token, float(l[token]), float(top))
            return "within"
        raise AssertionError(("greedy token", token, info.token))
    assert info.token != 0xFFFFFFFF, (token, "the oracle finds a degenerate row")
    order, d, w1, full, want = _survivor_model(l, p)
    V = l.size
    Z = float(w1.sum())
    T = float(p.temperature)
    tp = float(np.float32(p.top_p))
    if mode == "arith":
        ad = np.where(np.isfinite(d), np.abs(d), 0.0)
        if full:
            e1 = w1 * (2.0 ** -22 + 3 * 2.0 ** -24 * ad) + 2.0 ** -40
            eps_nuc = 2.0 * float(e1.sum()) / Z
        else:
            eps_nuc = SHORTLIST_Z_REL
    elif mode == "margin":
        eps_nuc = MARGIN_REL * tp
    else:
        raise ValueError(mode)
    run = np.cumsum(w1[:want]) / Z
    # the oracle's cut, and every cut the widened nucleus rule admits
    if p.top_p < 1.0:
        hit = np.nonzero(run >= tp)[0]
        c0 = int(hit[0]) + 1 if hit.size else want
        lo = np.nonzero(run >= tp - eps_nuc)[0]
        hi = np.nonzero(run >= tp + eps_nuc)[0]
        cmin = int(lo[0]) + 1 if lo.size else want
        cmax = int(hi[0]) + 1 if hi.size else want
        cuts = set(range(cmin, cmax + 1))
    else:
        c0 = want
        cuts = {want}
    capk = (lambda c: min(c, p.top_k) if p.top_k > 0 else c)
    cuts = sorted({max(1, capk(c)) for c in cuts})
    c0 = max(1, capk(c0))
    assert c0 in cuts, (c0, cuts)
    assert c0 == info.cut, ("numpy restatement disagrees with the oracle's cut", c0, info.cut)
    pos = np.nonzero(order == token)[0]
    assert pos.size == 1, token
    j = int(pos[0])
    cmax = max(cuts)
    with np.errstate(over="ignore"):
        wT = np.exp(d[:cmax] / T)
    if mode == "arith":
        if full:
            ad = np.where(np.isfinite(d[:cmax]), np.abs(d[:cmax]), 0.0)
            eT = wT * (2.0 ** -22 + 3 * 2.0 ** -24 * ad / T) + 2.0 ** -40
        else:
            eT = wT * SHORTLIST_DRAW_REL
        ecum = np.cumsum(eT)
    A = np.cumsum(wT)
    detail = []
    for c in cuts:
        if j >= c:
            detail.append((c, "token past the cut"))
            continue
        denom = float(A[c - 1])
        r = float(u) * denom
        eps = 2.0 * float(ecum[c - 1]) if mode == "arith" else MARGIN_REL * r
        before = float(A[j - 1]) if j > 0 else 0.0
        after = float(A[j])
        if before - eps < r <= after + eps:
            return "within"
        detail.append((c, j, r, before, after, eps))
    raise AssertionError(("token outside its CDF interval", token, info.token, int(info.rank), j, c0, detail[:3]))


def check_tokens(params, toks, logits, uniforms, *, mode="arith", within_frac=1 / 8, label="") -> dict:
    """draw_check on every row (params: oracle Params per row); at most max(1, n * within_frac)
    rows may need the widened interval. Returns the counts."""
    n = len(params)
    counts = {"rows": n, "exact": 0, "within": 0}
    within = []
    for b in range(n):
        res = draw_check(logits[b], params[b], float(uniforms[b]), int(toks[b]), mode=mode)
        counts[res] += 1
        if res == "within":
            within.append(b)
    print(f"{label}: {counts} within rows {within[:16]}")
    assert counts["within"] <= max(1, int(n * within_frac)), (label, counts, within[:16])
    return counts
