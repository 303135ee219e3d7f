"""Pins the oracle (oracle/orc.c) before it is trusted as the parity checker.

Each check is independent of the oracle's own formula: reference known-answer values,
closed forms, long-double brute force, the reference test's differently-ordered formula, and
bit-exact agreement with the reference's own src/sampling.cpp compiled into oracle/_ref.
"""
import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

import orc_py as O
import synth

GOLDEN = Path(__file__).resolve().parent / "golden" / "sampling_golden.json"


def lib():
    return O.orc()


# ---- bf16 -----------------------------------------------------------------------------------

def test_bf16_known_patterns():
    L = lib()
    assert L.orc_bf16_to_f32(0x3F80) == 1.0
    assert L.orc_bf16_to_f32(0xC000) == -2.0
    assert L.orc_f32_to_bf16(1.0) == 0x3F80
    # ties round to even (tests/test_gpu_kernels.cpp:36-42)
    tie_even = np.array([0x3F808000], dtype=np.uint32).view(np.float32)[0]
    tie_odd = np.array([0x3F818000], dtype=np.uint32).view(np.float32)[0]
    assert L.orc_f32_to_bf16(float(tie_even)) == 0x3F80
    assert L.orc_f32_to_bf16(float(tie_odd)) == 0x3F82
    above = np.array([0x3F808001], dtype=np.uint32).view(np.float32)[0]
    assert L.orc_f32_to_bf16(float(above)) == 0x3F81
    x = synth.normal(7, 99, 1000).astype(np.float32)
    assert all(L.orc_f32_to_bf16(float(v)) == b for v, b in zip(x, synth.f32_to_bf16(x)))


# ---- rms_norm (src/cpu_reference.cpp:43-52) -----------------------------------------------------

def test_rms_norm_closed_forms():
    D = 2816
    x = np.full(D, 2.0, dtype=np.float32)
    one = synth.f32_to_bf16(np.ones(D, dtype=np.float32))
    y = O.rms_norm(x, one, 1e-6)
    assert np.allclose(y, 2.0 / np.sqrt(4.0 + 1e-6), rtol=2e-7)
    # plain w, not 1 + w: a weight of 0.5 halves the output
    half = synth.f32_to_bf16(np.full(D, 0.5, dtype=np.float32))
    assert np.allclose(O.rms_norm(x, half, 1e-6), 0.5 * y, rtol=1e-7)
    # unit output RMS and scale invariance for a random vector
    r = synth.normal(3, 1, D).astype(np.float32)
    yr = O.rms_norm(r, None, 0.0)
    assert abs(float(np.sqrt(np.mean(yr.astype(np.float64) ** 2))) - 1.0) < 1e-6
    assert np.allclose(O.rms_norm(r * 8.0, None, 0.0), yr, rtol=1e-6)
    # long-double brute force with eps
    xl = r.astype(np.longdouble)
    want = xl / np.sqrt(np.mean(xl * xl) + np.longdouble(1e-6))
    assert np.max(np.abs(O.rms_norm(r, None, 1e-6) - want.astype(np.float64))) < 2e-6


# ---- matvec (src/cpu_reference.cpp:55-84) --------------------------------------------------------

def _rand_head(V, D, seed):
    W, S, B, g = synth.make_head(V, D, seed)
    return W, S, B


def test_matvec_constant_q_closed_form():
    V, D = 5, 256
    G = D // 64
    _, S, B = _rand_head(V, D, 11)
    x = synth.normal(11, 50, D).astype(np.float32)
    for k in (0, 3, 15):
        W = np.full((V, D // 2), k | (k << 4), dtype=np.uint8)
        got = O.matvec(W, S, B, x)
        sf = synth.bf16_to_f32(S).astype(np.float64)
        bf = synth.bf16_to_f32(B).astype(np.float64)
        sx = x.astype(np.float64).reshape(G, 64).sum(axis=1)
        want = ((sf * k + bf) * sx[None, :]).sum(axis=1)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-5)


def test_matvec_q8_bias_minus8s_is_zero_to_rounding():
    """q = 8 with b = -8s dequantises to w = 0. The reference sums dot per element but sum per
    pair (src/cpu_reference.cpp:74-77), so only rounding survives: |out| << s * sum|x|."""
    V, D = 7, 512
    _, S, _ = _rand_head(V, D, 12)
    B = synth.f32_to_bf16(-8.0 * synth.bf16_to_f32(S))  # exact: power-of-two scaling
    W = np.full((V, D // 2), 0x88, dtype=np.uint8)
    x = synth.normal(12, 50, D).astype(np.float32)
    out = O.matvec(W, S, B, x)
    bound = 64 * 2.0**-23 * 8 * synth.bf16_to_f32(S).max() * np.abs(x).sum()
    assert np.all(np.abs(out) <= bound) and bound < 1e-3


def test_matvec_one_hot_picks_dequantised_weight():
    """One-hot x returns q*s + b of that column: pins nibble order and group indexing."""
    V, D = 9, 192
    W, S, B = _rand_head(V, D, 13)
    sf, bf = synth.bf16_to_f32(S), synth.bf16_to_f32(B)
    for c in (0, 1, 2, 63, 64, 65, 127, 191):
        x = np.zeros(D, dtype=np.float32)
        x[c] = 1.0
        got = O.matvec(W, S, B, x)
        byte = W[:, c // 2]
        q = (byte & 0xF) if c % 2 == 0 else (byte >> 4)
        want = (q.astype(np.float32) * sf[:, c // 64] + bf[:, c // 64]).astype(np.float32)
        assert np.array_equal(got, want)


def test_matvec_brute_force_long_double_and_reference_test_formula():
    V, D = 33, 2816
    W, S, B = _rand_head(V, D, 14)
    x = synth.normal(14, 50, D).astype(np.float32)
    got = O.matvec(W, S, B, x).astype(np.float64)
    q = np.empty((V, D), dtype=np.int64)
    q[:, 0::2] = W & 0xF
    q[:, 1::2] = W >> 4
    sf = np.repeat(synth.bf16_to_f32(S).astype(np.longdouble), 64, axis=1)
    bf = np.repeat(synth.bf16_to_f32(B).astype(np.longdouble), 64, axis=1)
    exact = ((q * sf + bf) * x.astype(np.longdouble)).sum(axis=1).astype(np.float64)
    terms = np.abs((q * sf + bf) * x.astype(np.longdouble)).sum(axis=1).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 3e-6 * terms + 1e-7)
    # the reference test's own formula, acc += (q*s + b) * x per element in fp32
    # (tests/test_gpu_kernels.cpp:155-172), judged with its allclose rule (:66-94)
    w32 = (q.astype(np.float32) * np.repeat(synth.bf16_to_f32(S), 64, axis=1)
           + np.repeat(synth.bf16_to_f32(B), 64, axis=1)).astype(np.float32)
    acc = np.zeros(V, dtype=np.float32)
    for c in range(D):
        acc = (acc + w32[:, c] * x[c]).astype(np.float32)
    assert np.all(np.abs(got - acc) <= 1e-5 + 1e-4 * np.abs(acc))


def test_matvec_threads_bit_identical():
    W, S, B = _rand_head(1000, 256, 15)
    x = synth.normal(15, 50, 256).astype(np.float32)
    assert np.array_equal(O.matvec(W, S, B, x, threads=1), O.matvec(W, S, B, x, threads=7))


# ---- softcap (src/cpu_reference.cpp:535-538) -----------------------------------------------------

def test_softcap():
    z = np.linspace(-200, 200, 4001).astype(np.float32)
    got = O.softcap(z, 30.0)
    want = 30.0 * np.tanh(z.astype(np.float64) / 30.0)
    assert np.allclose(got, want, rtol=3e-7, atol=3e-6)
    assert np.array_equal(got, -O.softcap(-z, 30.0))
    assert O.softcap(np.array([1000.0], dtype=np.float32), 30.0)[0] == 30.0
    assert np.array_equal(O.softcap(z, 0.0), z)


# ---- validate_sampling (src/sampling.cpp:32-54) --------------------------------------------------

def _valid(**kw):
    return bool(lib().orc_validate_sampling(C.byref(O.params(**kw)), None, 0))


def test_validate_reference_matrix():
    # tests/test_sampling.cpp:92-112
    assert _valid(temperature=0.2, top_p=0.95, top_k=64)
    assert _valid(temperature=0.0, top_p=1.0, top_k=0)
    assert not _valid(temperature=-0.1)
    assert not _valid(temperature=0.2, top_p=0.0, top_k=64)
    assert not _valid(temperature=0.2, top_p=1.5, top_k=64)
    assert not _valid(temperature=0.2, top_p=0.95, top_k=257)
    assert not _valid(temperature=0.2, top_p=0.95, top_k=-1)
    assert not _valid(temperature=0.2, top_p=0.95, top_k=64, repetition_penalty=0.0)
    assert not _valid(temperature=0.7, top_p=0.9, top_k=0)
    assert _valid(temperature=0.7, top_p=1.0, top_k=0)
    assert _valid(temperature=0.0, top_p=0.9, top_k=0)
    # extension: the full-vocabulary flag lifts only the top_k rule
    assert _valid(temperature=0.7, top_p=0.9, top_k=0, flags=O.FLAG_FULL_VOCAB)
    assert not _valid(temperature=0.7, top_p=0.9, top_k=300, flags=O.FLAG_FULL_VOCAB)
    assert not _valid(temperature=0.7, presence_penalty=float("nan"))


def test_validate_matches_compiled_reference():
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    for t in (-1.0, 0.0, 0.5, float("inf"), float("nan")):
        for p in (0.0, 0.5, 1.0, 1.01, float("nan")):
            for k in (-1, 0, 1, 256, 257):
                for pen in (0.0, 0.5, 1.0, float("inf")):
                    assert R.ref_validate_sampling(t, p, k, pen) == _valid(
                        temperature=t, top_p=p, top_k=k, repetition_penalty=pen), (t, p, k, pen)


# ---- seeding (src/sampling.cpp:56-72) -----------------------------------------------------------

def test_splitmix_kats_and_seed_for():
    L = lib()
    # tests/test_sampling.cpp:118-121
    assert L.orc_splitmix64(0) == 0xE220A8397B1DCDAF
    assert L.orc_splitmix64(1) == 0x910A2DEC89025CC1
    assert L.orc_splitmix64(2) == 0x975835DE1C9756CE
    assert L.orc_splitmix64(3) == 0x1D0B14E4DB018FED
    vals = [L.orc_seed_for(1, 12345, p) for p in range(10000)]
    assert all(v != 0 for v in vals)
    assert L.orc_seed_for(1, 12345, 0) != L.orc_seed_for(1, 12345, 1)
    assert L.orc_seed_for(1, 12345, 5) != L.orc_seed_for(1, 99, 5)
    R = O.ref()
    if R is not None:
        for hs in (0, 1):
            for seed in (0, 1, 12345, 2**63 + 5):
                for pos in (-3, 0, 1, 77, 100000):
                    assert L.orc_seed_for(hs, seed, pos) == R.ref_seed_for(hs, seed, pos)


# ---- repetition penalty (src/sampling.cpp:74-90) ------------------------------------------------

def _pen(logits, history, p, cap, fn="orc"):
    l = np.array(logits, dtype=np.float32)
    h = np.array(history, dtype=np.uint32)
    if fn == "orc":
        lib().orc_apply_repetition_penalty(l, l.size, h.ctypes.data if h.size else None, h.size, p, cap)
    else:
        O.ref().ref_apply_repetition_penalty(l, l.size, h, h.size, p, cap)
    return l


def test_repetition_penalty_reference_values():
    # tests/test_sampling.cpp:199-228
    v = _pen([10.0, -10.0, 0.0, 29.999], [0, 1, 3, 99999], 2.0, 30.0)
    assert abs(v[0] - 5.0) < 1e-5 and abs(v[1] + 20.0) < 1e-5 and v[2] == 0.0
    assert 14.9 < v[3] < 15.1
    assert np.all(np.abs(v) <= 30.0)
    base = np.array([10.0, -10.0, 0.0, 29.999], dtype=np.float32)
    assert np.array_equal(_pen(base, [0, 1, 3], 1.0, 30.0), base)
    assert np.array_equal(_pen(base, [], 2.0, 30.0), base)
    g = _pen([9.0, 8.0], [0], 2.0, 30.0)
    assert int(np.argmax(g)) == 1
    # per occurrence: an id seen n times is divided n times
    assert _pen([16.0], [0, 0, 0], 2.0, 30.0)[0] == 2.0
    # clamp to +-0.9999 * softcap after each step
    assert _pen([-20.0], [0, 0], 2.0, 30.0)[0] == np.float32(-30.0 * np.float32(0.9999))


def test_repetition_penalty_matches_compiled_reference():
    if O.ref() is None:
        pytest.skip("oracle/_ref not built")
    for seed in range(20):
        V = 1000
        l = (synth.normal(seed, 60, V) * 12).astype(np.float32)
        h = synth.uniform_ids(300, V + 20, seed)  # includes out-of-range ids
        for p in (0.7, 1.0, 1.1, 2.5):
            assert np.array_equal(_pen(l, h, p, 30.0), _pen(l, h, p, 30.0, "ref"))


# ---- sample_token (src/sampling.cpp:92-169) -----------------------------------------------------

def _orc_tok(l, seed, **kw):
    p = O.params(**kw)
    info = O.SampleInfo()
    return int(lib().orc_sample_token(np.ascontiguousarray(l, dtype=np.float32), l.size, C.byref(p),
                                      seed, C.byref(info)))


def test_sample_reference_unit_cases():
    # greedy tie to the lower index (tests/test_sampling.cpp:140-149)
    assert _orc_tok(np.array([1, 5, 3, 5, 2], np.float32), 1) == 1
    assert _orc_tok(np.array([7], np.float32), 1) == 0
    # mlx truncation order reachability (:152-173)
    l = np.array([3.0, 2.5, 2.0, 1.5, -1.0, -2.0, -3.0, -4.0], np.float32)
    seen = {_orc_tok(l, lib().orc_seed_for(1, 7, i), temperature=1.0, top_p=0.9, top_k=2)
            for i in range(4000)}
    assert seen == {0, 1}


def test_sample_matches_compiled_reference_sweep():
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built")
    cfgs = [(0.2, 0.95, 64), (1.0, 0.9, 8), (0.7, 1.0, 256), (0.5, 1.0, 0), (1.5, 0.99, 1),
            (0.8, 0.95, 64), (1.0, 0.5, 256), (0.3, 0.8, 20), (0.0, 1.0, 0)]
    for V in (1, 2, 17, 300, 5000):
        for s in range(6):
            l = (synth.normal(s, 61, V) * 4).astype(np.float32)
            if s == 5:
                l = np.round(l)  # many exact ties
            for (t, p, k) in cfgs:
                for d in range(5):
                    seed = lib().orc_seed_for(1, 1000 + s, d)
                    assert _orc_tok(l, seed, temperature=t, top_p=p, top_k=k) == \
                        R.ref_sample_token(l, V, t, p, k, 1.0, seed), (V, s, t, p, k, d)


def test_sample_matches_compiled_reference_full_vocab_sweep():
    """The reference's own equivalence sweep shape: V = 262144, N(0, 6), 5 configs x 40."""
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built")
    V = 262144
    l = (synth.normal(20260723, 62, V) * 6).astype(np.float32)
    cfgs = [(0.2, 0.95, 64, 1), (1.0, 0.9, 8, 2), (0.7, 1.0, 256, 3), (0.5, 1.0, 0, 4), (1.5, 0.99, 1, 5)]
    for (t, p, k, sd) in cfgs:
        for i in range(40):
            seed = lib().orc_seed_for(1, sd, i)
            assert _orc_tok(l, seed, temperature=t, top_p=p, top_k=k) == R.ref_sample_token(l, V, t, p, k, 1.0, seed)


def test_sample_golden_fixture():
    """Tokens the compiled reference produced (tests/golden/make_golden.py); runs without it."""
    g = json.loads(GOLDEN.read_text())
    for case in g["sample_cases"]:
        V = case["V"]
        l = (synth.normal(case["seed"], 63, V) * case["scale"]).astype(np.float32)
        if case.get("round"):
            l = np.round(l).astype(np.float32)
        for (t, p, k), seeds, toks in zip(case["cfgs"], case["seeds"], case["tokens"]):
            for s, tok in zip(seeds, toks):
                assert _orc_tok(l, s, temperature=t, top_p=p, top_k=k) == tok
    for (seed, pos, hs, want) in g["seed_for"]:
        assert lib().orc_seed_for(hs, seed, pos) == want
    for case in g["penalty_cases"]:
        V = case["V"]
        l = (synth.normal(case["seed"], 64, V) * 12).astype(np.float32)
        h = synth.uniform_ids(case["n"], V + 10, case["seed"])
        got = _pen(l, h, case["p"], 30.0)
        assert got.view(np.uint32).tolist() == case["bits"]


# ---- full-vocabulary extension -------------------------------------------------------------------

def _full_sort_sample(l, t, p, k, u):
    """tests/test_sampling.cpp:36-84 semantics with an injected uniform, via numpy sorting."""
    V = l.size
    idx = np.lexsort((np.arange(V), -l.astype(np.float64)))
    best = float(l[idx[0]])
    total = np.sum(np.exp(l.astype(np.float64) - best))
    cut = V
    if p < 1.0:
        run = np.cumsum(np.exp(l[idx].astype(np.float64) - best) / total)
        hit = np.nonzero(run >= np.float64(np.float32(p)))[0]
        if hit.size:
            cut = int(hit[0]) + 1
    if k > 0:
        cut = min(cut, k)
    cut = max(1, cut)
    q = np.exp((l[idx[:cut]].astype(np.float64) - best) / np.float64(np.float32(t)))
    acc = np.cumsum(q)
    r = np.float64(np.float32(u)) * acc[-1]
    hit = np.nonzero(acc >= r)[0]
    return int(idx[hit[0]]) if hit.size else int(idx[cut - 1])


def test_full_vocab_matches_numpy_full_sort():
    for s in range(8):
        V = 3000
        l = (synth.normal(s, 65, V) * 3).astype(np.float32)
        if s % 3 == 0:
            l = np.round(l * 2) / 2
        for (t, p, k) in [(1.0, 0.9, 0), (0.7, 0.5, 0), (1.3, 1.0, 0), (0.5, 0.95, 40)]:
            for j in range(10):
                u = float(synth.uniform(s, 66, 1, j)[0])
                info = O.sample(l, O.params(temperature=t, top_p=p, top_k=k, flags=O.FLAG_FULL_VOCAB), u)
                # sequential double sums vs numpy cumsum can differ only in the last bits
                assert info.token == _full_sort_sample(l, t, p, k, u)


def test_parity_mode_equals_full_vocab_with_topk():
    l = (synth.normal(5, 67, 20000) * 5).astype(np.float32)
    for k in (1, 20, 256):
        for j in range(10):
            u = float(synth.uniform(5, 68, 1, j)[0])
            a = O.sample(l, O.params(temperature=0.8, top_p=0.9, top_k=k), u)
            b = O.sample(l, O.params(temperature=0.8, top_p=0.9, top_k=k, flags=O.FLAG_FULL_VOCAB), u)
            assert a.token == b.token


# ---- Philox4x32-10 (Random123 known-answer vectors) ---------------------------------------------

def test_philox_kat():
    L = lib()
    def run(ctr, key):
        out = np.zeros(4, np.uint32)
        L.orc_philox4x32_10(np.array(ctr, np.uint32), np.array(key, np.uint32), out)
        return out.tolist()
    assert run([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert run([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert run([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0]) == \
        [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]
    u = O.philox_uniform(0, 0)
    assert u == (0x6627E8D5 >> 8) / 2**24


# ---- modifier extensions (closed forms; parity unpinned against the reference) ----------------

def test_modifier_closed_forms():
    l = np.array([1.0, 2.0, -3.0, 4.0, 5.0], np.float32)
    p = O.params(temperature=1.0, repetition_penalty=2.0, presence_penalty=0.5, frequency_penalty=0.25)
    out = O.apply_modifiers(l, p, 30.0, history=[0, 2, 2, 9], bias_ids=[0, 4, 4, 7],
                            bias_values=np.array([1.0, 0.5, 0.25, 3.0], np.float32),
                            ban=np.array([1 << 3], np.uint32))
    # id 0: bias +1 -> 2, penalty /2 -> 1, presence -0.5, frequency -0.25*1 -> 0.25
    assert out[0] == np.float32(0.25)
    assert out[1] == 2.0
    # id 2: no bias, -3 * 2 * 2 = -12, -0.5, -0.25*2 -> -13
    assert out[2] == np.float32(-13.0)
    assert out[3] == -np.inf                  # banned
    assert out[4] == np.float32(5.75)         # 0.5 + 0.25 summed, then added once


def test_embed_row_closed_form_and_one_hot_matvec():
    """Embedding lookup (src/cpu_reference.cpp:108-124, :323-329) pinned two ways: a row whose
    nibbles are all k dequantises to (k s + b) per group, scaled by sqrtf(D); and the unscaled
    row equals the (separately pinned) matvec against one-hot inputs, element by element."""
    V, D = 8, 128
    W, S, B, _ = synth.make_head(V, D, 5)
    W = W.copy()
    W[3, :] = 0x77  # row 3: every nibble 7
    G = D // 64
    sf = synth.bf16_to_f32(S).reshape(V, G)
    bf = synth.bf16_to_f32(B).reshape(V, G)
    scale = np.float32(np.sqrt(np.float32(D)))
    got = O.embed(W, S, B, 3)
    want = np.repeat((np.float32(7) * sf[3] + bf[3]).astype(np.float32), 64) * scale
    assert np.array_equal(got, want.astype(np.float32))
    for row in (0, 5, V - 1):
        e = O.embed(W, S, B, row)
        for c in (0, 1, 63, 64, D - 1):
            x = np.zeros(D, np.float32)
            x[c] = 1.0
            unscaled = O.matvec(W, S, B, x)[row]
            assert np.float32(unscaled) * scale == e[c], (row, c)
