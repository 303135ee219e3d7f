"""The in-engine C++ caller (tests/integration/runner_tail.cpp: a ForwardRunner-shaped class that
creates the head from a bundle and runs generate_tokens, src/runner.cpp:818-898) loaded in this
process through ctypes. Every emitted token is replayed on the oracle with the reference's own
seed map (seed_for(position) -> next_uniform, src/sampling.cpp:18-28, :63-72, at the GPU runner's
positions, src/runner.cpp:847, :898) and the repetition penalty over the prompt plus the tokens so
far. The replay is teacher-forced on the GPU's tokens, so a near-tie (counted, never silently
dropped) cannot send the two trajectories apart. The device history must end as the prompt followed
by every emitted token, as the reference's history vector does."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import bundle_util as BU
import orc_py as O
import parity_util as U
import synth
import turbo_decode_tail as T

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "integration" / "_build" / "librunner_tail.so"
V, D = 65536, 2816
ALPHA = 0.03  # stand-in layers: hidden = ALPHA * embedding + z[position]


@pytest.fixture(scope="module")
def bundle(tmp_path_factory):
    W, S, B, g = synth.make_head(V, D, 41)
    p = tmp_path_factory.mktemp("bundle") / "resident.bin"
    BU.write_resident(p, BU.head_tensors(W, S, B, g))
    return p, (W, S, B, g)


def runner_lib():
    T.load()  # the product library first: the runner links the same file
    if not LIB.exists():
        raise FileNotFoundError(f"{LIB} is missing: build it with `make -C tests/integration`")
    lib = C.CDLL(str(LIB))
    u32p, f32p = C.POINTER(C.c_uint32), C.POINTER(C.c_float)
    lib.tail_generate.restype = C.c_int
    lib.tail_generate.argtypes = [C.c_char_p, C.c_float, C.c_float, f32p, C.c_uint32, C.c_float, u32p, C.c_uint32,
                                  C.c_float, C.c_float, C.c_int, C.c_float, C.c_int, C.c_uint64, C.c_int, u32p,
                                  u32p, u32p, C.c_char_p, C.c_size_t]
    return lib


def generate(lib, path, z, prompt, p, has_seed, seed, steps):
    toks = np.zeros(steps, np.uint32)
    hist = np.zeros(prompt.size + steps, np.uint32)
    hl = C.c_uint32(0)
    err = C.create_string_buffer(512)
    u32 = lambda a: a.ctypes.data_as(C.POINTER(C.c_uint32))  # noqa: E731
    ok = lib.tail_generate(str(path).encode(), 30.0, 1e-6, z.ctypes.data_as(C.POINTER(C.c_float)), z.shape[0],
                           ALPHA, u32(prompt), prompt.size, p.temperature, p.top_p, p.top_k, p.repetition_penalty,
                           has_seed, seed, steps, u32(toks), u32(hist), C.byref(hl), err, 512)
    assert ok, err.value.decode()
    return toks, hist[:hl.value]


def replay(head, z, prompt, p, has_seed, seed, toks):
    """Oracle tokens at every emitted position, given the GPU's previous tokens."""
    W, S, B, g = head
    hist = [int(t) for t in prompt]
    prev, pos = int(prompt[-1]), prompt.size - 1  # the last prefill step emits the first token
    near = 0
    for t, got in enumerate(toks):
        e = O.embed(W, S, B, prev)
        h = (np.float32(ALPHA) * e).astype(np.float32) + z[pos]
        l = O.head_logits(W, S, B, g, h, threads=U.THREADS)
        l = O.apply_modifiers(l, p, 30.0, history=np.array(hist, np.uint32))
        # the oracle chain's logits differ from the device's within the logit tolerance: the
        # token must sit inside its CDF interval there, widened by the stated margin
        if U.draw_check(l, p, O.reference_uniform(has_seed, seed, pos), int(got), mode="margin") == "within":
            near += 1
        hist.append(int(got))
        prev, pos = int(got), pos + 1
    return near


@pytest.mark.parametrize("kind", ["sampled_seeded", "sampled_unseeded", "greedy"])
def test_runner_generate_tokens_matches_oracle_replay(bundle, kind):
    path, head = bundle
    lib = runner_lib()
    prompt = synth.uniform_ids(16, V, 42)
    if kind == "greedy":
        p, has_seed, seed, steps = O.params(0.0, 1.0, 0, 1.0), 0, 0, 24
    elif kind == "sampled_seeded":
        p, has_seed, seed, steps = O.params(0.8, 0.95, 64, 1.1), 1, 20260801, 80
    else:
        p, has_seed, seed, steps = O.params(1.0, 0.9, 40, 1.3), 0, 0, 24
    z = synth.hidden_states(prompt.size + steps, D, 43)
    toks, hist = generate(lib, path, z, prompt, p, has_seed, seed, steps)
    assert np.all(toks < V)
    # the device history: the prompt, then every emitted token (src/runner.cpp:858, :878)
    assert np.array_equal(hist, np.concatenate([prompt, toks]))
    near = replay(head, z, prompt, p, has_seed, seed, toks)
    distinct = np.unique(toks).size
    print(f"{kind}: {steps} tokens, {distinct} distinct, {near} near-tie mismatches")
    assert near <= max(1, steps // 20)
    if kind != "greedy":
        assert distinct > steps // 4  # the stand-in keeps the distribution far from one-hot


def test_runner_reports_errors_through_the_last_error_channel(bundle):
    path, _ = bundle
    lib = runner_lib()
    prompt = synth.uniform_ids(4, V, 44)
    z = synth.hidden_states(prompt.size + 4, D, 45)
    # top_p < 1 with top_k == 0 and T > 0: validate_sampling rejects it (src/sampling.cpp:49-53)
    p = O.params(0.7, 0.5, 0, 1.0)
    toks = np.zeros(4, np.uint32)
    hist = np.zeros(8, np.uint32)
    hl = C.c_uint32(0)
    err = C.create_string_buffer(512)
    u32 = lambda a: a.ctypes.data_as(C.POINTER(C.c_uint32))  # noqa: E731
    ok = lib.tail_generate(str(path).encode(), 30.0, 1e-6, z.ctypes.data_as(C.POINTER(C.c_float)), z.shape[0],
                           ALPHA, u32(prompt), prompt.size, p.temperature, p.top_p, p.top_k, p.repetition_penalty,
                           1, 5, 4, u32(toks), u32(hist), C.byref(hl), err, 512)
    assert not ok
    assert "top_p < 1" in err.value.decode()
    assert "top_p < 1" in T.last_error()
