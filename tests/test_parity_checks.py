"""The token checks of the GPU parity tests (parity_util.draw_check / check_tokens) against
deliberately wrong selectors, on the CPU: a check that accepted any token would pass a broken
sampler. Rows shaped like the batched configurations (full-vocabulary top-p 0.9 over ~160,000
survivors; per-row temperatures and top-k; greedy) are sampled by the oracle, then the oracle's
token is replaced by its neighbour in the survivor order, or by a token far from it."""
import numpy as np
import pytest

import orc_py as O
import parity_util as U

V = 262144


def flat_rows(n, seed, sigma=1.0):
    """Softcapped N(0, sigma) logits: at sigma = 1 the top-p 0.9 nucleus keeps ~61 % of the
    vocabulary, like the B = 256 full-vocabulary rows."""
    rng = np.random.default_rng(seed)
    return [O.softcap((rng.standard_normal(V) * sigma).astype(np.float32), 30.0) for _ in range(n)]


def shifted(l, p, u, by):
    info = O.sample(l, p, u)
    order, *_ = U._survivor_model(l, p)
    k = min(max(int(info.rank) + by, 0), V - 1)
    return int(order[k]), info


@pytest.mark.parametrize("by", [1, -1])
def test_full_vocab_rows_reject_a_selector_off_by_one_rank(by):
    n = 10
    rows = flat_rows(n, 11)
    p = O.params(1.0, 0.9, 0, 1.0, 0.0, 0.0, O.FLAG_FULL_VOCAB)
    us = [float(np.float32(u)) for u in np.random.default_rng(12).random(n)]
    good = [O.sample(l, p, u).token for l, u in zip(rows, us)]
    c = U.check_tokens([p] * n, good, rows, us, label="oracle tokens")
    assert c["exact"] == n
    bad = [shifted(l, p, u, by)[0] for l, u in zip(rows, us)]
    with pytest.raises(AssertionError):
        U.check_tokens([p] * n, bad, rows, us, label=f"off by {by}")
    # row by row: most single rows already fail on their own
    fails = 0
    for b in range(n):
        try:
            U.draw_check(rows[b], p, us[b], bad[b])
        except AssertionError:
            fails += 1
    assert fails >= n // 3, fails


def test_mixed_rows_reject_a_selector_off_by_one_rank():
    """Per-row temperature, top-k in {0 (full vocabulary), 20, 40, 100} and top-p, as the B = 32
    mixed configuration."""
    n = 8
    rows = flat_rows(n, 21, sigma=2.0)
    rng = np.random.default_rng(22)
    ks = [0, 20, 40, 100]
    ps = [O.params(float(np.float32(0.3 + 1.2 * rng.random())), float(np.float32(0.8 + 0.2 * rng.random())),
                   ks[b % 4], 1.0, 0.0, 0.0, O.FLAG_FULL_VOCAB if ks[b % 4] == 0 else 0) for b in range(n)]
    us = [float(np.float32(u)) for u in rng.random(n)]
    good = [O.sample(l, p, u).token for l, p, u in zip(rows, ps, us)]
    assert U.check_tokens(ps, good, rows, us, label="oracle tokens")["exact"] == n
    fails = 0
    for b in range(n):
        tok, info = shifted(rows[b], ps[b], us[b], 1)
        if tok == info.token:
            continue
        try:
            U.draw_check(rows[b], ps[b], us[b], tok)
        except AssertionError:
            fails += 1
    assert fails >= n - 2, fails


def test_margin_mode_tolerates_logit_noise_but_not_a_distant_token():
    """Oracle-chain rows: the GPU's logits differ from the oracle's within the tolerance. The
    oracle's own token on slightly perturbed logits passes against the unperturbed ones (within
    the 1e-3 margin); a token 1 % of the survivors away does not."""
    n = 6
    rows = flat_rows(n, 31)
    p = O.params(1.0, 0.9, 0, 1.0, 0.0, 0.0, O.FLAG_FULL_VOCAB)
    rng = np.random.default_rng(32)
    us = [float(np.float32(u)) for u in rng.random(n)]
    noisy = [(l * (1 + 2e-5 * rng.standard_normal(V))).astype(np.float32) for l in rows]
    toks = [O.sample(nl, p, u).token for nl, u in zip(noisy, us)]
    U.check_tokens([p] * n, toks, rows, us, mode="margin", within_frac=1.0, label="noisy logits")
    for b in range(n):
        far, info = shifted(rows[b], p, us[b], 1600 if info_rank_low(rows[b], p, us[b]) else -1600)
        with pytest.raises(AssertionError):
            U.draw_check(rows[b], p, us[b], far, mode="margin")


def info_rank_low(l, p, u):
    info = O.sample(l, p, u)
    return info.rank + 1600 < info.cut


def test_greedy_rows():
    l = np.array([1.0, 5.0, 3.0, 5.0, 2.0], np.float32)
    p = O.params(0.0)
    assert U.draw_check(l, p, 0.5, 1) == "exact"        # ties to the lowest index (:141-144)
    with pytest.raises(AssertionError):
        U.draw_check(l, p, 0.5, 3)                      # the other maximum
    near = np.array([1.0, 5.0, 3.0, 5.004, 2.0], np.float32)
    assert U.draw_check(near, p, 0.5, 1, mode="margin") == "within"
    with pytest.raises(AssertionError):
        U.draw_check(near, p, 0.5, 2, mode="margin")


def test_shortlist_cut_matches_the_oracle():
    """The checker's numpy survivor model must reproduce the oracle's cut (it asserts so on every
    row it widens); exercised here on shortlist and full-vocabulary rows with shifted tokens."""
    rows = flat_rows(4, 41, sigma=3.0)
    for l in rows:
        for p in (O.params(0.8, 0.95, 64, 1.0), O.params(1.2, 0.9, 0, 1.0, 0.0, 0.0, O.FLAG_FULL_VOCAB),
                  O.params(0.7, 1.0, 256, 1.0)):
            tok, info = shifted(l, p, 0.37, 1)
            try:
                U.draw_check(l, p, 0.37, tok)
            except AssertionError as e:
                assert "numpy restatement" not in str(e), e
