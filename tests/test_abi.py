"""C-ABI checks that need no GPU: the library loads, exports every symbol the header declares,
and its host-side helpers (validate_sampling, splitmix64, seed_for, the per-row uniform) agree
with the oracle. No compute call is made here."""
import ctypes as C
import re
from pathlib import Path

import numpy as np

import orc_py as O
import turbo_decode_tail as T

HEADER = Path(__file__).resolve().parents[1] / "include" / "turbo_decode_tail.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"TURBO_DT_API\s+[^;(]*?\b(turbo_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert sorted(T.EXPORTS) == declared_symbols()


def test_library_exports_every_declared_symbol():
    lib = T.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_struct_layouts():
    assert C.sizeof(T.TurboSamplingRow) == 56
    assert C.sizeof(T.TurboRowReport) == 56
    assert C.sizeof(T.TurboStepOutputs) == 24


def test_abi_version_and_struct_sizes():
    """The library reports the header's ABI version and, per struct, the size it was built with;
    the ctypes mirror's layouts must agree with both."""
    lib = T.load()
    ver = int(re.search(r"#define TURBO_DT_ABI_VERSION (\d+)u", HEADER.read_text()).group(1))
    assert lib.turbo_abi_version() == ver
    for which, st in enumerate((T.TurboLMHeadDesc, T.TurboBundleTensor, T.TurboSamplingRow, T.TurboStepInputs,
                                T.TurboRowReport, T.TurboStepOutputs)):
        assert lib.turbo_abi_struct_size(which) == C.sizeof(st), st.__name__
    assert lib.turbo_abi_struct_size(99) == 0


def test_splitmix_and_seed_for():
    lib = T.load()
    assert lib.turbo_splitmix64(0) == 0xE220A8397B1DCDAF
    assert lib.turbo_splitmix64(3) == 0x1D0B14E4DB018FED
    L = O.orc()
    for hs in (0, 1):
        for seed in (0, 5, 12345, 2**64 - 1):
            for pos in (-1, 0, 1, 1000, 2**31 - 1):
                assert lib.turbo_seed_for(hs, seed, pos) == L.orc_seed_for(hs, seed, pos)


def test_validate_matches_oracle():
    grid = []
    for t in (-0.5, 0.0, 0.7, float("nan")):
        for p in (0.0, 0.5, 1.0, 1.2):
            for k in (-1, 0, 64, 256, 257):
                for pen in (0.0, 1.0, 1.1):
                    for fl in (0, 1):
                        grid.append((t, p, k, pen, fl))
    for (t, p, k, pen, fl) in grid:
        row = T.row_default(temperature=t, top_p=p, top_k=k, repetition_penalty=pen, flags=fl)
        ok, why = T.validate(row)
        want = bool(O.orc().orc_validate_sampling(
            C.byref(O.params(temperature=t, top_p=p, top_k=k, repetition_penalty=pen, flags=fl)), None, 0))
        assert ok == want, (t, p, k, pen, fl, why)
        assert (why == "") == ok
    assert not T.validate(T.row_default(rng=7))[0]
    assert not T.validate(T.row_default(flags=4))[0]
    assert not T.validate(T.row_default(temperature=1.0, presence_penalty=float("inf")))[0]


def test_row_uniform_matches_oracle():
    for seed in (0, 1, 20260721, 2**63 + 11):
        for ctr in (0, 1, 511, 2**40 + 3):
            r = T.row_default(seed=seed, counter=ctr)
            assert T.row_uniform(r) == O.philox_uniform(seed, ctr)
            r = T.row_default(rng=T.TURBO_RNG_REFERENCE, has_seed=1, seed=seed, counter=ctr % 100000)
            assert T.row_uniform(r) == O.reference_uniform(1, seed, ctr % 100000)
    r = T.row_default(rng=T.TURBO_RNG_REFERENCE, has_seed=0, counter=17)
    assert T.row_uniform(r) == O.reference_uniform(0, 0, 17)


def test_create_rejects_bad_descriptors_before_touching_a_device():
    lib = T.load()
    d = T.TurboLMHeadDesc()
    lib.turbo_lmhead_desc_default(C.byref(d))
    assert (d.vocab_size, d.hidden_size, d.group_size) == (262144, 2816, 64)
    assert abs(d.final_logit_softcap - 30.0) < 1e-7
    d.group_size = 32
    assert not lib.turbo_lmhead_create(C.byref(d))
    assert "group_size" in T.last_error()
    lib.turbo_lmhead_desc_default(C.byref(d))
    d.hidden_size = 100
    assert not lib.turbo_lmhead_create(C.byref(d))
    assert "hidden_size" in T.last_error()
    lib.turbo_lmhead_desc_default(C.byref(d))
    assert not lib.turbo_lmhead_create(C.byref(d))  # NULL tables
    assert "NULL" in T.last_error()
    # a successful host-only call clears the thread-local error (c_api.h:74-78)
    assert T.validate(T.row_default())[0]
    assert T.last_error() == ""


def test_null_handle_errors():
    lib = T.load()
    assert lib.turbo_lmhead_synchronize(None) == 0
    assert "handle" in T.last_error()
    lib.turbo_lmhead_destroy(None)  # no-op


def test_reference_rng_position_must_fit_an_int():
    """TURBO_RNG_REFERENCE maps counter to the reference's int position (src/sampling.cpp:63):
    negative positions as 64-bit two's complement are accepted, values outside int are rejected."""
    ok = lambda c: T.validate(T.row_default(rng=T.TURBO_RNG_REFERENCE, counter=c))  # noqa: E731
    assert ok(0)[0] and ok(2**31 - 1)[0] and ok(2**64 - 1)[0] and ok(2**64 - 2**31)[0]
    for c in (2**31, 2**40, 2**64 - 2**31 - 1):
        good, why = ok(c)
        assert not good and "int position" in why, c
    # Philox counters are unrestricted
    assert T.validate(T.row_default(counter=2**63 + 5))[0]
