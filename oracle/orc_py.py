"""ctypes access to the oracle (oracle/_build/liborc.so) and, when built, the compiled
reference sampling code (oracle/_ref/libref_sampling.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU
baseline. The product library never uses it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORC_SO = HERE / "_build" / "liborc.so"
REF_SO = HERE / "_ref" / "libref_sampling.so"
FLAG_FULL_VOCAB = 1

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")


class Params(C.Structure):
    _fields_ = [
        ("temperature", C.c_float),
        ("top_p", C.c_float),
        ("top_k", C.c_int),
        ("repetition_penalty", C.c_float),
        ("presence_penalty", C.c_float),
        ("frequency_penalty", C.c_float),
        ("flags", C.c_uint32),
    ]


class SampleInfo(C.Structure):
    _fields_ = [
        ("token", C.c_uint32),
        ("shortlist", C.c_uint32),
        ("cut", C.c_uint32),
        ("rank", C.c_uint32),
        ("max_logit", C.c_float),
        ("second_logit", C.c_float),
        ("total", C.c_double),
        ("nucleus_run", C.c_double),
        ("nucleus_prev", C.c_double),
        ("denom", C.c_double),
        ("r", C.c_double),
        ("acc_prev", C.c_double),
        ("acc_at", C.c_double),
        ("u", C.c_float),
    ]


def params(temperature=0.0, top_p=1.0, top_k=0, repetition_penalty=1.0, presence_penalty=0.0,
           frequency_penalty=0.0, flags=0) -> Params:
    return Params(temperature, top_p, top_k, repetition_penalty, presence_penalty,
                  frequency_penalty, flags)


_orc = None
_ref = None


def orc() -> C.CDLL:
    global _orc
    if _orc is None:
        if not ORC_SO.exists():
            subprocess.run(["make", "-s", "-C", str(HERE), "orc"], check=True)
        lib = C.CDLL(str(ORC_SO))
        lib.orc_bf16_to_f32.restype = C.c_float
        lib.orc_bf16_to_f32.argtypes = [C.c_uint16]
        lib.orc_f32_to_bf16.restype = C.c_uint16
        lib.orc_f32_to_bf16.argtypes = [C.c_float]
        lib.orc_rms_norm.argtypes = [_f32p, C.c_void_p, C.c_size_t, C.c_float, _f32p]
        lib.orc_matvec_int4.argtypes = [_u8p, _u16p, _u16p, C.c_uint32, _f32p, _f32p, C.c_uint32, C.c_uint32]
        lib.orc_matvec_int4_mt.argtypes = [_u8p, _u16p, _u16p, C.c_uint32, C.c_uint32, _f32p, _f32p, C.c_int]
        lib.orc_softcap.argtypes = [_f32p, C.c_size_t, C.c_float]
        lib.orc_embed_row.argtypes = [_u8p, _u16p, _u16p, C.c_uint32, C.c_uint32, _f32p]
        lib.orc_validate_sampling.restype = C.c_int
        lib.orc_validate_sampling.argtypes = [C.POINTER(Params), C.c_char_p, C.c_size_t]
        lib.orc_splitmix64.restype = C.c_uint64
        lib.orc_splitmix64.argtypes = [C.c_uint64]
        lib.orc_seed_for.restype = C.c_uint64
        lib.orc_seed_for.argtypes = [C.c_int, C.c_uint64, C.c_int]
        lib.orc_next_uniform.restype = C.c_float
        lib.orc_next_uniform.argtypes = [C.POINTER(C.c_uint64)]
        lib.orc_apply_repetition_penalty.argtypes = [_f32p, C.c_uint32, C.c_void_p, C.c_size_t, C.c_float, C.c_float]
        lib.orc_sample_token_u.restype = C.c_uint32
        lib.orc_sample_token_u.argtypes = [_f32p, C.c_uint32, C.POINTER(Params), C.c_float, C.POINTER(SampleInfo)]
        lib.orc_sample_token.restype = C.c_uint32
        lib.orc_sample_token.argtypes = [_f32p, C.c_uint32, C.POINTER(Params), C.c_uint64, C.POINTER(SampleInfo)]
        lib.orc_philox4x32_10.argtypes = [_u32p, _u32p, _u32p]
        lib.orc_philox_uniform.restype = C.c_float
        lib.orc_philox_uniform.argtypes = [C.c_uint64, C.c_uint64]
        lib.orc_apply_logit_bias.argtypes = [_f32p, C.c_uint32, _u32p, _f32p, C.c_size_t]
        lib.orc_apply_presence_frequency.argtypes = [_f32p, C.c_uint32, _u32p, C.c_size_t, C.c_float, C.c_float]
        lib.orc_apply_ban.argtypes = [_f32p, C.c_uint32, _u32p]
        lib.orc_apply_modifiers.argtypes = [_f32p, C.c_uint32, C.POINTER(Params), C.c_float,
                                            C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p,
                                            C.c_size_t, C.c_void_p]
        lib.orc_time_decode_steps.restype = C.c_int
        lib.orc_time_decode_steps.argtypes = [_u8p, _u16p, _u16p, C.c_void_p, C.c_uint32, C.c_uint32,
                                              C.c_float, C.c_float, _f32p, C.c_uint32, C.c_uint64, C.c_int,
                                              C.POINTER(Params), C.c_uint64, _u32p, C.c_size_t, C.c_size_t,
                                              _u32p, np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")]
        _orc = lib
    return _orc


def ref() -> C.CDLL | None:
    """The compiled reference sampling code, or None when it is not built."""
    global _ref
    if _ref is None and REF_SO.exists():
        lib = C.CDLL(str(REF_SO))
        lib.ref_validate_sampling.restype = C.c_int
        lib.ref_validate_sampling.argtypes = [C.c_float, C.c_float, C.c_int, C.c_float]
        lib.ref_splitmix64.restype = C.c_ulonglong
        lib.ref_splitmix64.argtypes = [C.c_ulonglong]
        lib.ref_seed_for.restype = C.c_ulonglong
        lib.ref_seed_for.argtypes = [C.c_int, C.c_ulonglong, C.c_int]
        lib.ref_apply_repetition_penalty.argtypes = [_f32p, C.c_uint, _u32p, C.c_ulonglong, C.c_float, C.c_float]
        lib.ref_sample_token.restype = C.c_uint
        lib.ref_sample_token.argtypes = [_f32p, C.c_uint, C.c_float, C.c_float, C.c_int, C.c_float, C.c_ulonglong]
        _ref = lib
    return _ref


# ---- numpy-friendly wrappers ------------------------------------------------------------------

def rms_norm(x: np.ndarray, gamma: np.ndarray | None, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.uint16)
    orc().orc_rms_norm(x, None if g is None else g.ctypes.data, x.size, eps, out)
    return out


def matvec(W, S, B, x, threads: int = 1) -> np.ndarray:
    V = W.shape[0]
    D = W.shape[1] * 2
    out = np.empty(V, dtype=np.float32)
    orc().orc_matvec_int4_mt(np.ascontiguousarray(W), np.ascontiguousarray(S), np.ascontiguousarray(B),
                             V, D, np.ascontiguousarray(x, dtype=np.float32), out, threads)
    return out


def embed(W, S, B, token: int) -> np.ndarray:
    """Embedding row `token` of the tied table, scaled by sqrt(hidden)."""
    D = W.shape[1] * 2
    out = np.empty(D, dtype=np.float32)
    orc().orc_embed_row(np.ascontiguousarray(W), np.ascontiguousarray(S), np.ascontiguousarray(B), D, token, out)
    return out


def softcap(z: np.ndarray, cap: float) -> np.ndarray:
    z = np.array(z, dtype=np.float32, copy=True)
    orc().orc_softcap(z, z.size, cap)
    return z


def head_logits(W, S, B, gamma, hidden, eps=1e-6, cap=30.0, normed=False, threads=1) -> np.ndarray:
    """Final RMSNorm (unless normed) -> tied head -> softcap, one row."""
    x = hidden if normed else rms_norm(hidden, gamma, eps)
    return softcap(matvec(W, S, B, x, threads), cap)


def apply_modifiers(logits: np.ndarray, p: Params, softcap_v: float, history=None, bias_ids=None,
                    bias_values=None, ban=None) -> np.ndarray:
    l = np.array(logits, dtype=np.float32, copy=True)
    h = None if history is None else np.ascontiguousarray(history, dtype=np.uint32)
    bi = None if bias_ids is None else np.ascontiguousarray(bias_ids, dtype=np.uint32)
    bv = None if bias_values is None else np.ascontiguousarray(bias_values, dtype=np.float32)
    bn = None if ban is None else np.ascontiguousarray(ban, dtype=np.uint32)
    orc().orc_apply_modifiers(l, l.size, C.byref(p), softcap_v,
                              None if h is None else h.ctypes.data, 0 if h is None else h.size,
                              None if bi is None else bi.ctypes.data,
                              None if bv is None else bv.ctypes.data, 0 if bi is None else bi.size,
                              None if bn is None else bn.ctypes.data)
    return l


def sample(logits: np.ndarray, p: Params, u: float) -> SampleInfo:
    info = SampleInfo()
    l = np.ascontiguousarray(logits, dtype=np.float32)
    orc().orc_sample_token_u(l, l.size, C.byref(p), u, C.byref(info))
    return info


def philox_uniform(seed: int, counter: int) -> float:
    return float(orc().orc_philox_uniform(seed, counter))


def reference_uniform(has_seed: int, seed: int, position: int) -> float:
    s = C.c_uint64(orc().orc_seed_for(has_seed, seed, position))
    return float(orc().orc_next_uniform(C.byref(s)))


def time_decode_steps(W, S, B, gamma, hidden, p: Params, seed: int, history, *, first_counter=0,
                      threads=1, eps=1e-6, cap=30.0):
    """Runs hidden.shape[0] decode steps of one row in C (RMSNorm -> head -> softcap ->
    modifiers -> sampler, the token appended to the history) and returns (tokens, seconds per
    step). The timing is taken inside the C loop; no Python runs between its clock reads."""
    hidden = np.ascontiguousarray(hidden, dtype=np.float32)
    n, D = hidden.shape
    V = W.shape[0]
    hist = np.zeros(len(history) + n, dtype=np.uint32)
    hist[:len(history)] = history
    toks = np.zeros(n, dtype=np.uint32)
    secs = np.zeros(n, dtype=np.float64)
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.uint16)
    ok = orc().orc_time_decode_steps(np.ascontiguousarray(W), np.ascontiguousarray(S), np.ascontiguousarray(B),
                                     None if g is None else g.ctypes.data, V, D, eps, cap, hidden, n,
                                     first_counter, threads, C.byref(p), seed, hist, len(history), hist.size,
                                     toks, secs)
    if not ok:
        raise MemoryError("orc_time_decode_steps: allocation failed")
    return toks, secs
