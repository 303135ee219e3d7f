"""ctypes binding of libturbo_decode_tail.so (include/turbo_decode_tail.h).

The library is the product; this module only mirrors its C ABI for Python callers (tests,
bench). Device buffers are passed as raw pointers (``tensor.data_ptr()`` of torch CUDA tensors
works); torch is not required by this module.

Loading fails loudly when the library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libturbo_decode_tail.so"

TURBO_RNG_PHILOX = 0
TURBO_RNG_REFERENCE = 1
TURBO_ROW_FULL_VOCAB = 1
TURBO_HIDDEN_F32 = 0
TURBO_HIDDEN_BF16 = 1
TURBO_STEP_NORMED = 1
TURBO_STEP_APPEND_HISTORY = 2
TURBO_STATUS_HISTORY_FULL = 1

# Every symbol include/turbo_decode_tail.h declares.
EXPORTS = (
    "turbo_abi_version",
    "turbo_abi_struct_size",
    "turbo_lmhead_last_error",
    "turbo_lmhead_desc_default",
    "turbo_lmhead_create",
    "turbo_lmhead_destroy",
    "turbo_lmhead_set_stream",
    "turbo_lmhead_synchronize",
    "turbo_lmhead_limits",
    "turbo_sampling_row_default",
    "turbo_validate_sampling",
    "turbo_splitmix64",
    "turbo_seed_for",
    "turbo_row_uniform",
    "turbo_lmhead_step",
    "turbo_lmhead_rms_norm",
    "turbo_lmhead_logits",
    "turbo_lmhead_greedy",
    "turbo_softcap",
    "turbo_apply_repetition_penalty",
    "turbo_sample_logits",
    "turbo_lmhead_enable_head_timing",
    "turbo_lmhead_head_kernel_time",
    "turbo_int4_matvec",
    "turbo_lmhead_embed",
    "turbo_bundle_decode_header",
    "turbo_bundle_find_tensor",
    "turbo_lmhead_create_from_bundle",
    "turbo_sample_logits_noalloc",
    "turbo_int4_matrix_create",
    "turbo_int4_matrix_load",
    "turbo_int4_matrix_destroy",
    "turbo_int4_matvec_grouped",
)

TURBO_NOALLOC_MAX_BATCH = 4
TURBO_NOALLOC_MAX_VOCAB = 262144


class TurboLMHeadDesc(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_uint32),
        ("hidden_size", C.c_uint32),
        ("group_size", C.c_uint32),
        ("final_logit_softcap", C.c_float),
        ("rms_norm_eps", C.c_float),
        ("weights_on_device", C.c_int),
        ("weight", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
        ("norm_weight", C.c_void_p),
        ("device", C.c_int),
    ]


class TurboSamplingRow(C.Structure):
    _fields_ = [
        ("temperature", C.c_float),
        ("top_p", C.c_float),
        ("top_k", C.c_int),
        ("repetition_penalty", C.c_float),
        ("presence_penalty", C.c_float),
        ("frequency_penalty", C.c_float),
        ("rng", C.c_int),
        ("has_seed", C.c_int),
        ("seed", C.c_uint64),
        ("counter", C.c_uint64),
        ("flags", C.c_uint32),
    ]


class TurboStepInputs(C.Structure):
    _fields_ = [
        ("batch", C.c_int),
        ("hidden", C.c_void_p),
        ("hidden_dtype", C.c_int),
        ("flags", C.c_uint32),
        ("rows", C.POINTER(TurboSamplingRow)),
        ("history", C.c_void_p),
        ("history_stride", C.c_uint32),
        ("history_len", C.c_void_p),
        ("ban_bits", C.c_void_p),
        ("ban_stride", C.c_uint32),
        ("bias_ids", C.c_void_p),
        ("bias_values", C.c_void_p),
        ("bias_stride", C.c_uint32),
        ("bias_count", C.c_void_p),
        ("uniforms", C.c_void_p),
    ]


class TurboRowReport(C.Structure):
    _fields_ = [
        ("max_logit", C.c_float),
        ("u", C.c_float),
        ("shortlist", C.c_uint32),
        ("cut", C.c_uint32),
        ("rank", C.c_uint32),
        ("path", C.c_uint32),
        ("total", C.c_double),
        ("denom", C.c_double),
        ("r", C.c_double),
        ("status", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


class TurboStepOutputs(C.Structure):
    _fields_ = [
        ("tokens", C.c_void_p),
        ("logits", C.c_void_p),
        ("report", C.c_void_p),
    ]


class TurboBundleTensor(C.Structure):
    _fields_ = [
        ("dtype", C.c_uint32),
        ("shape", C.c_uint32 * 4),
        ("file_offset", C.c_uint64),
        ("size_bytes", C.c_uint64),
        ("scale_offset", C.c_uint64),
        ("scale_size", C.c_uint64),
        ("bias_offset", C.c_uint64),
        ("bias_size", C.c_uint64),
        ("quantized", C.c_uint32),
        ("rows", C.c_uint32),
        ("in_dim", C.c_uint32),
        ("bits", C.c_uint32),
    ]


_lib = None


def load(path: os.PathLike | str | None = None) -> C.CDLL:
    """Loads the built library (raises if it is missing)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build it with `python turbo-winfare_amd/build.py` "
            "(there is no fallback implementation)")
    lib = C.CDLL(str(p))
    vp, u32, i32, f32 = C.c_void_p, C.c_uint32, C.c_int, C.c_float
    sig = {
        "turbo_abi_version": (u32, []),
        "turbo_abi_struct_size": (C.c_size_t, [i32]),
        "turbo_lmhead_last_error": (C.c_char_p, []),
        "turbo_lmhead_desc_default": (None, [C.POINTER(TurboLMHeadDesc)]),
        "turbo_lmhead_create": (vp, [C.POINTER(TurboLMHeadDesc)]),
        "turbo_lmhead_destroy": (None, [vp]),
        "turbo_lmhead_set_stream": (i32, [vp, vp]),
        "turbo_lmhead_synchronize": (i32, [vp]),
        "turbo_lmhead_limits": (i32, [vp, C.POINTER(i32), C.POINTER(i32)]),
        "turbo_sampling_row_default": (None, [C.POINTER(TurboSamplingRow)]),
        "turbo_validate_sampling": (i32, [C.POINTER(TurboSamplingRow)]),
        "turbo_splitmix64": (C.c_uint64, [C.c_uint64]),
        "turbo_seed_for": (C.c_uint64, [i32, C.c_uint64, i32]),
        "turbo_row_uniform": (f32, [C.POINTER(TurboSamplingRow)]),
        "turbo_lmhead_step": (i32, [vp, C.POINTER(TurboStepInputs), C.POINTER(TurboStepOutputs)]),
        "turbo_lmhead_rms_norm": (i32, [vp, vp, i32, vp]),
        "turbo_lmhead_logits": (i32, [vp, vp, i32, i32, i32, vp]),
        "turbo_lmhead_greedy": (i32, [vp, vp, i32, i32, vp]),
        "turbo_softcap": (i32, [vp, vp, C.c_size_t, f32]),
        "turbo_apply_repetition_penalty": (i32, [vp, vp, u32, vp, u32, f32, f32]),
        "turbo_sample_logits": (i32, [vp, vp, C.POINTER(TurboStepInputs), C.POINTER(TurboStepOutputs)]),
        "turbo_lmhead_enable_head_timing": (i32, [vp, i32]),
        "turbo_lmhead_head_kernel_time": (i32, [vp, C.POINTER(C.c_double), C.POINTER(i32), i32]),
        "turbo_int4_matvec": (i32, [vp, vp, i32, i32, vp]),
        "turbo_lmhead_embed": (i32, [vp, vp, i32, vp]),
        "turbo_bundle_decode_header": (i32, [vp, C.c_size_t, C.POINTER(C.c_uint64)]),
        "turbo_bundle_find_tensor": (i32, [C.c_char_p, C.c_char_p, C.POINTER(TurboBundleTensor)]),
        "turbo_lmhead_create_from_bundle": (vp, [C.c_char_p, f32, f32, i32]),
        "turbo_sample_logits_noalloc": (i32, [vp, u32, f32, vp, C.POINTER(TurboStepInputs),
                                              C.POINTER(TurboStepOutputs)]),
        "turbo_int4_matrix_create": (vp, [u32, u32, i32]),
        "turbo_int4_matrix_load": (i32, [vp, vp, vp, vp, i32, vp]),
        "turbo_int4_matrix_destroy": (None, [vp]),
        "turbo_int4_matvec_grouped": (i32, [C.POINTER(vp), i32, C.POINTER(vp), C.POINTER(vp), vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    return load().turbo_lmhead_last_error().decode()


class TurboError(RuntimeError):
    pass


def _ok(rc: int) -> None:
    if not rc:
        raise TurboError(last_error())


def row_default(**kw) -> TurboSamplingRow:
    r = TurboSamplingRow()
    load().turbo_sampling_row_default(C.byref(r))
    for k, v in kw.items():
        setattr(r, k, v)
    return r


def validate(row: TurboSamplingRow) -> tuple[bool, str]:
    ok = bool(load().turbo_validate_sampling(C.byref(row)))
    return ok, ("" if ok else last_error())


def row_uniform(row: TurboSamplingRow) -> float:
    return float(load().turbo_row_uniform(C.byref(row)))


def _ptr(t) -> int | None:
    if t is None:
        return None
    return int(t.data_ptr()) if hasattr(t, "data_ptr") else int(t)


def bundle_decode_header(data: bytes) -> tuple[int, int, int]:
    """(index_size, resident_size, entry_count) of a resident.bin header."""
    out = (C.c_uint64 * 3)()
    buf = C.create_string_buffer(bytes(data), len(data))
    _ok(load().turbo_bundle_decode_header(C.addressof(buf), len(data), out))
    return int(out[0]), int(out[1]), int(out[2])


def bundle_find_tensor(resident_path, name: str) -> TurboBundleTensor:
    t = TurboBundleTensor()
    _ok(load().turbo_bundle_find_tensor(str(resident_path).encode(), name.encode(), C.byref(t)))
    return t


class LMHead:
    """Owns one turbo_lmhead handle. Arrays: numpy (host) or torch CUDA tensors (device)."""

    @classmethod
    def from_bundle(cls, resident_path, *, softcap: float = 30.0, eps: float = 1e-6, device: int = 0):
        """Head from a .gturbo bundle's resident.bin (model.embed_tokens.weight + model.norm.weight)."""
        self = cls.__new__(cls)
        self.lib = load()
        h = self.lib.turbo_lmhead_create_from_bundle(str(resident_path).encode(), softcap, eps, device)
        if not h:
            raise TurboError(last_error())
        t = bundle_find_tensor(resident_path, "model.embed_tokens.weight")
        self.vocab, self.hidden = int(t.rows), int(t.in_dim)
        self.h = h
        return self

    def __init__(self, weight, scales, biases, norm_weight=None, *, vocab: int, hidden: int,
                 softcap: float = 30.0, eps: float = 1e-6, on_device: bool = False, device: int = 0):
        self.lib = load()
        d = TurboLMHeadDesc()
        self.lib.turbo_lmhead_desc_default(C.byref(d))
        d.vocab_size = vocab
        d.hidden_size = hidden
        d.final_logit_softcap = softcap
        d.rms_norm_eps = eps
        d.weights_on_device = 1 if on_device else 0
        d.device = device

        def hp(a):
            if a is None:
                return None
            if on_device:
                return _ptr(a)
            return a.ctypes.data

        d.weight, d.scales, d.biases, d.norm_weight = hp(weight), hp(scales), hp(biases), hp(norm_weight)
        self.vocab, self.hidden = vocab, hidden
        h = self.lib.turbo_lmhead_create(C.byref(d))
        if not h:
            raise TurboError(last_error())
        self.h = h

    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.turbo_lmhead_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self) -> None:
        _ok(self.lib.turbo_lmhead_synchronize(self.h))

    def set_stream(self, stream) -> None:
        """stream: a hipStream_t as an int (torch.cuda.Stream.cuda_stream) or None for the null stream."""
        _ok(self.lib.turbo_lmhead_set_stream(self.h, stream))

    def limits(self) -> tuple[int, int]:
        mb, mm = C.c_int(), C.c_int()
        _ok(self.lib.turbo_lmhead_limits(self.h, C.byref(mb), C.byref(mm)))
        return mb.value, mm.value

    def rms_norm(self, x, batch: int, out) -> None:
        _ok(self.lib.turbo_lmhead_rms_norm(self.h, _ptr(x), batch, _ptr(out)))

    def matvec(self, x, batch: int, out, *, dtype: int = TURBO_HIDDEN_F32) -> None:
        """out[b][r] = sum_c w[r][c] x[b][c] (no norm, no softcap); device buffers."""
        _ok(self.lib.turbo_int4_matvec(self.h, _ptr(x), dtype, batch, _ptr(out)))

    def embed(self, tokens, n: int, out) -> None:
        """out[i] = embedding row tokens[i] (dequantised, times sqrt(hidden)); device buffers."""
        _ok(self.lib.turbo_lmhead_embed(self.h, _ptr(tokens), n, _ptr(out)))

    def logits(self, x, batch: int, out, *, dtype: int = TURBO_HIDDEN_F32, softcap: bool = True) -> None:
        _ok(self.lib.turbo_lmhead_logits(self.h, _ptr(x), dtype, batch, 1 if softcap else 0, _ptr(out)))

    def greedy(self, x, batch: int, tokens, *, dtype: int = TURBO_HIDDEN_F32) -> None:
        _ok(self.lib.turbo_lmhead_greedy(self.h, _ptr(x), dtype, batch, _ptr(tokens)))

    @staticmethod
    def make_inputs(batch, rows, *, hidden=None, dtype=TURBO_HIDDEN_F32, flags=0, history=None,
                    history_len=None, ban=None, bias_ids=None, bias_values=None, bias_count=None,
                    uniforms=None):
        arr = (TurboSamplingRow * batch)(*rows)
        inp = TurboStepInputs()
        inp.batch = batch
        inp.hidden = _ptr(hidden)
        inp.hidden_dtype = dtype
        inp.flags = flags
        inp.rows = C.cast(arr, C.POINTER(TurboSamplingRow))
        if history is not None:
            inp.history = _ptr(history)
            inp.history_stride = int(history.shape[1])
            inp.history_len = _ptr(history_len)
        if ban is not None:
            inp.ban_bits = _ptr(ban)
            inp.ban_stride = int(ban.shape[1])
        if bias_ids is not None:
            inp.bias_ids = _ptr(bias_ids)
            inp.bias_values = _ptr(bias_values)
            inp.bias_stride = int(bias_ids.shape[1])
            inp.bias_count = _ptr(bias_count)
        inp.uniforms = _ptr(uniforms)
        return inp, arr  # keep arr alive with the struct

    def step(self, inp: TurboStepInputs, tokens, logits=None, report=None) -> None:
        out = TurboStepOutputs(_ptr(tokens), _ptr(logits), _ptr(report))
        _ok(self.lib.turbo_lmhead_step(self.h, C.byref(inp), C.byref(out)))

    def sample_logits(self, logits, inp: TurboStepInputs, tokens, report=None) -> None:
        out = TurboStepOutputs(_ptr(tokens), None, _ptr(report))
        _ok(self.lib.turbo_sample_logits(self.h, _ptr(logits), C.byref(inp), C.byref(out)))

    def enable_head_timing(self, on: bool = True, every: int = 1) -> None:
        """Time every `every`-th head launch with HIP events (0 launches when off)."""
        _ok(self.lib.turbo_lmhead_enable_head_timing(self.h, max(1, int(every)) if on else 0))

    def head_kernel_time(self, reset: bool = False) -> tuple[float, int]:
        ms, n = C.c_double(), C.c_int()
        _ok(self.lib.turbo_lmhead_head_kernel_time(self.h, C.byref(ms), C.byref(n), 1 if reset else 0))
        return ms.value, n.value


class Int4Matrix:
    """One turbo_int4_matrix handle (the table only). Arrays: numpy (host) or torch CUDA tensors."""

    def __init__(self, rows: int, in_dim: int, device: int = 0):
        self.lib = load()
        self.rows, self.in_dim = rows, in_dim
        self.h = self.lib.turbo_int4_matrix_create(rows, in_dim, device)
        if not self.h:
            raise TurboError(last_error())

    def load_weights(self, weight, scales, biases, *, on_device: bool = False, stream=None) -> None:
        hp = (lambda a: _ptr(a)) if on_device else (lambda a: a.ctypes.data)
        _ok(self.lib.turbo_int4_matrix_load(self.h, hp(weight), hp(scales), hp(biases), 1 if on_device else 0,
                                            stream))

    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.turbo_int4_matrix_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matvec_grouped(matrices, xs, outs, stream=None) -> None:
    """turbo_int4_matvec_grouped: out[i] = matrices[i] @ xs[i], one launch (device buffers)."""
    n = len(matrices)
    mats = (C.c_void_p * max(n, 1))(*[m.h for m in matrices])
    xp = (C.c_void_p * max(n, 1))(*[_ptr(x) for x in xs])
    op = (C.c_void_p * max(n, 1))(*[_ptr(o) for o in outs])
    _ok(load().turbo_int4_matvec_grouped(mats, n, xp, op, stream))


def sample_logits_noalloc(logits, vocab: int, inp: TurboStepInputs, tokens, report=None, *,
                          softcap: float = 30.0, stream=None) -> None:
    """turbo_sample_logits_noalloc: the sampler over caller logits with no handle (static scratch)."""
    out = TurboStepOutputs(_ptr(tokens), None, _ptr(report))
    _ok(load().turbo_sample_logits_noalloc(stream, vocab, softcap, _ptr(logits), C.byref(inp), C.byref(out)))


def softcap(z, n: int, cap: float, stream=None) -> None:
    _ok(load().turbo_softcap(stream, _ptr(z), n, cap))


def apply_repetition_penalty(logits, vocab: int, history, n: int, penalty: float, softcap: float,
                             stream=None) -> None:
    _ok(load().turbo_apply_repetition_penalty(stream, _ptr(logits), vocab, _ptr(history), n,
                                              penalty, softcap))
