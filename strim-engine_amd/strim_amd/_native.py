"""ctypes binding of libstrim_sampler.so (the C ABI in include/strim_sampler.h).

The library is built in-tree by strim-engine_amd/build.py. There is no fallback: if
the shared object is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_NAME = "libstrim_sampler.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

# status codes (include/strim_sampler.h)
OK, EINVAL, EEMPTY, ENONFINITE, ECAPACITY, EHIP, ENOMEM = 0, -1, -2, -3, -4, -5, -6
STATUS_NAMES = {OK: "OK", EINVAL: "EINVAL", EEMPTY: "EEMPTY", ENONFINITE: "ENONFINITE",
                ECAPACITY: "ECAPACITY", EHIP: "EHIP", ENOMEM: "ENOMEM"}
DTYPE_F32, DTYPE_BF16 = 0, 1
NOISE_ICDF, NOISE_GUMBEL = 0, 1
FLAG_TOPK_KEEP_TIES, FLAG_NOISE_BY_RANK, FLAG_SCORE_NO_LSE = 1, 2, 4
FLAG_SAMPLER_COMPAT = 7

# Every symbol include/strim_sampler.h declares.
EXPORTS = (
    "strim_version",
    "strim_default_params",
    "strim_check_params",
    "strim_ctx_create",
    "strim_ctx_destroy",
    "strim_sample",
    "strim_sample_noalloc",
    "strim_verify",
    "strim_mask_logits",
    "strim_head_logits",
    "strim_head_greedy",
    "strim_draft_argmax",
    "strim_profile_begin",
    "strim_profile_end",
    "strim_kernel_name",
    "strim_grammar_create",
    "strim_grammar_destroy",
    "strim_grammar_set_dfa",
    "strim_grammar_append_states",
    "strim_grammar_set_next",
    "strim_grammar_pending",
    "strim_grammar_drop_masks",
    "strim_grammar_masks",
    "strim_grammar_advance",
    "strim_request_keys",
    "strim_request_advance",
)
KERNEL_COUNT = 8
NOALLOC_MAX_ROWS, NOALLOC_MAX_VOCAB = 32, 262144  # strim_sample_noalloc limits


class StrimError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: {STATUS_NAMES.get(code, code)}")
        self.code = code


class SamplingParams(ctypes.Structure):
    """strim_sampling_params (48 bytes)."""

    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("flags", ctypes.c_uint32),
        ("seed", ctypes.c_uint64),
        ("position", ctypes.c_uint64),
    ]


assert ctypes.sizeof(SamplingParams) == 48

PARAMS_DTYPE = np.dtype(
    [("temperature", "<f4"), ("top_k", "<i4"), ("top_p", "<f4"), ("min_p", "<f4"),
     ("repetition_penalty", "<f4"), ("presence_penalty", "<f4"),
     ("frequency_penalty", "<f4"), ("flags", "<u4"), ("seed", "<u8"), ("position", "<u8")],
    align=True,
)
assert PARAMS_DTYPE.itemsize == 48


def params_array(n: int, **kw) -> np.ndarray:
    """Host param rows of plain sampling (T=1, no top-k/top-p, extensions off, as
    strim_default_params), overridden by kw (scalar or per-row sequence)."""
    p = np.zeros(n, dtype=PARAMS_DTYPE)
    p["temperature"] = 1.0
    p["top_p"] = 1.0
    p["repetition_penalty"] = 1.0
    for key, val in kw.items():
        p[key] = val
    return p


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        L.strim_version.restype = ctypes.c_char_p
        L.strim_version.argtypes = []
        L.strim_default_params.restype = None
        L.strim_default_params.argtypes = [P]
        L.strim_check_params.restype = ctypes.c_int
        L.strim_check_params.argtypes = [P, I32]
        L.strim_ctx_create.restype = ctypes.c_int
        L.strim_ctx_create.argtypes = [ctypes.POINTER(ctypes.c_void_p), I32, I32, I32]
        L.strim_ctx_destroy.restype = ctypes.c_int
        L.strim_ctx_destroy.argtypes = [P]
        L.strim_sample.restype = ctypes.c_int
        L.strim_sample.argtypes = [P, P, P, I32, I32, I32, I64, P, P, I64, P, P, I32, I32, P,
                                   P, P, P]
        L.strim_sample_noalloc.restype = ctypes.c_int
        L.strim_sample_noalloc.argtypes = [P, P, I32, I32, I32, I64, P, P, I64, P, P, I32, I32,
                                           P, P, P]
        L.strim_verify.restype = ctypes.c_int
        L.strim_verify.argtypes = [P, P, P, I32, I32, I32, I32, P, I32, P, P, P, P, I64, P, P,
                                   I32, I32, P, P, P, P, P, P]
        L.strim_mask_logits.restype = ctypes.c_int
        L.strim_mask_logits.argtypes = [P, P, I32, I32, I32, I64, P, I64, P]
        L.strim_head_logits.restype = ctypes.c_int
        L.strim_head_logits.argtypes = [P, P, I64, I32, I32, P, ctypes.c_float, P, P, I64, I32,
                                        P, I64]
        L.strim_head_greedy.restype = ctypes.c_int
        L.strim_head_greedy.argtypes = [P, P, P, I64, I32, I32, P, ctypes.c_float, P, P, I64,
                                        I32, P, I64, P, P]
        L.strim_draft_argmax.restype = ctypes.c_int
        L.strim_draft_argmax.argtypes = [P, P, I32, I32, I32, I64, P, P]
        L.strim_profile_begin.restype = ctypes.c_int
        L.strim_profile_begin.argtypes = [P, I32]
        L.strim_profile_end.restype = ctypes.c_int
        L.strim_profile_end.argtypes = [P, P, P]
        L.strim_kernel_name.restype = ctypes.c_char_p
        L.strim_kernel_name.argtypes = [I32]
        L.strim_grammar_create.restype = ctypes.c_int
        L.strim_grammar_create.argtypes = [ctypes.POINTER(ctypes.c_void_p), I32, I32, P, P, P,
                                           I32, P, I32, I32]
        L.strim_grammar_destroy.restype = ctypes.c_int
        L.strim_grammar_destroy.argtypes = [P]
        L.strim_grammar_set_dfa.restype = ctypes.c_int
        L.strim_grammar_set_dfa.argtypes = [P, P, I32, P, P]
        L.strim_grammar_append_states.restype = ctypes.c_int
        L.strim_grammar_append_states.argtypes = [P, P, I32, P, P, ctypes.POINTER(ctypes.c_int32)]
        L.strim_grammar_set_next.restype = ctypes.c_int
        L.strim_grammar_set_next.argtypes = [P, P, I32, P, P]
        L.strim_grammar_pending.restype = ctypes.c_int
        L.strim_grammar_pending.argtypes = [P, P, P, I32, ctypes.POINTER(ctypes.c_int32)]
        L.strim_grammar_drop_masks.restype = ctypes.c_int
        L.strim_grammar_drop_masks.argtypes = [P, P, I32, I32]
        L.strim_grammar_masks.restype = ctypes.c_int
        L.strim_grammar_masks.argtypes = [P, P, P, I32, P, I64]
        L.strim_grammar_advance.restype = ctypes.c_int
        L.strim_grammar_advance.argtypes = [P, P, P, I32, P, I32, P]
        L.strim_request_keys.restype = ctypes.c_int
        L.strim_request_keys.argtypes = [P, P, P, I32, P, I32, P]
        L.strim_request_advance.restype = ctypes.c_int
        L.strim_request_advance.argtypes = [P, P, P, I32, P, I32, P, P]
        _lib = L
    return _lib


def check(code: int, what: str) -> None:
    if code != OK:
        raise StrimError(code, what)


def version() -> str:
    return lib().strim_version().decode()


def check_params(params: np.ndarray) -> int:
    p = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
    return int(lib().strim_check_params(p.ctypes.data_as(ctypes.c_void_p), p.size))
