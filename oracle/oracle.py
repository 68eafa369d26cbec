"""ctypes front end of the CPU oracle (oracle/strim_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP library and the timed CPU
baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it. The product package never does.

Every function takes and returns numpy arrays. bf16 logits must be converted to
float32 by the caller (exact). The C source documents the semantics and cites the
reference lines (Sources/StrimCore/SpecSampling.swift, Sources/StrimEngine/Sampler.swift,
Sources/StrimCore/TokenMask.swift).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libstrim_oracle.so"

# fp64 decision margin below which a GPU/oracle id mismatch is a documented fp tie.
TIE_EPS = 1e-6

STRIM_OK, STRIM_EINVAL, STRIM_EEMPTY, STRIM_ENONFINITE, STRIM_ECAPACITY = 0, -1, -2, -3, -4
NOISE_ICDF, NOISE_GUMBEL = 0, 1
FLAG_TOPK_KEEP_TIES, FLAG_NOISE_BY_RANK, FLAG_SCORE_NO_LSE = 1, 2, 4
FLAG_SAMPLER_COMPAT = 7

# Same layout as strim_sampling_params in include/strim_sampler.h (48 bytes).
PARAMS_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_k", "<i4"),
        ("top_p", "<f4"),
        ("min_p", "<f4"),
        ("repetition_penalty", "<f4"),
        ("presence_penalty", "<f4"),
        ("frequency_penalty", "<f4"),
        ("flags", "<u4"),
        ("seed", "<u8"),
        ("position", "<u8"),
    ],
    align=True,
)
assert PARAMS_DTYPE.itemsize == 48

ROW_RESULT_DTYPE = np.dtype(
    [
        ("token", "<i4"),
        ("status", "<i4"),
        ("n_allowed", "<i4"),
        ("n_kept", "<i4"),
        ("m", "<f4"),
        ("pad", "<f4"),
        ("sum_kept", "<f8"),
        ("margin", "<f8"),
    ],
    align=True,
)
assert ROW_RESULT_DTYPE.itemsize == 40


def make_params(n: int, **kw) -> np.ndarray:
    """Param array of n rows of plain sampling (T=1, no top-k/top-p, extensions off),
    overridden by kw (scalars or per-row sequences)."""
    p = np.zeros(n, dtype=PARAMS_DTYPE)
    p["temperature"] = 1.0
    p["top_k"] = 0
    p["top_p"] = 1.0
    p["min_p"] = 0.0
    p["repetition_penalty"] = 1.0
    p["presence_penalty"] = 0.0
    p["frequency_penalty"] = 0.0
    p["flags"] = 0
    p["seed"] = 0
    p["position"] = 0
    for key, val in kw.items():
        p[key] = val
    return p


def build(force: bool = False) -> Path:
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "-B" if force else "libstrim_oracle.so"],
                       check=True)
    return LIB_PATH


def build_mutant(mutant: int, out: Path) -> Path:
    """A variant of the oracle compiled with SO_MUTANT=mutant (a planted indexing mistake,
    see strim_oracle.c), written to `out`. For the tests' discrimination checks only."""
    subprocess.run(["make", "-s", "-B", "-C", str(HERE), f"OUT={Path(out).resolve()}",
                    f"EXTRA=-DSO_MUTANT={int(mutant)}"], check=True)
    return Path(out)


_lib = None


class use_library:
    """Context manager: route every oracle call through the library at `path` (a mutant
    built by build_mutant) until the block ends."""

    def __init__(self, path):
        self.path = Path(path)

    def __enter__(self):
        global _lib
        self._saved = _lib
        _lib = _load(self.path)
        return self

    def __exit__(self, *exc):
        global _lib
        _lib = self._saved
        return False


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = _load(LIB_PATH)
    return _lib


def _load(path: Path):
    L = ctypes.CDLL(str(path))
    P, I32, I64, U64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64
    L.so_mix.restype = U64
    L.so_mix.argtypes = [U64, U64]
    L.so_philox4x32_10.argtypes = [P, P, P]
    L.so_uniform.restype = ctypes.c_float
    L.so_uniform.argtypes = [U64, U64, U64]
    L.so_uniforms.argtypes = [U64, U64, I64, P]
    L.so_gumbel.restype = ctypes.c_double
    L.so_gumbel.argtypes = [ctypes.c_float]
    L.so_process_row.restype = I32
    L.so_process_row.argtypes = [P, I32, P, P, I32, P, I32, P, P]
    L.so_sample_batch.argtypes = [P, I32, I32, P, P, I64, P, P, I32, I32, P, P, P, I32]
    L.so_verify_batch.argtypes = [P, I32, I32, I32, P, I32, P, P, P, P, I64, P, P, I32, I32,
                                  P, P, P, P, P, P, P, P, I32]
    L.so_trie_build.restype = P
    L.so_trie_build.argtypes = [I32, P, P, P]
    L.so_trie_free.argtypes = [P]
    L.so_trie_nodes.restype = I32
    L.so_trie_nodes.argtypes = [P]
    L.so_grammar_mask.argtypes = [P, I32, P, I32, I32, P, P, I32, P]
    L.so_grammar_advance_bytes.restype = I32
    L.so_grammar_advance_bytes.argtypes = [I32, P, ctypes.c_uint32, P]
    L.so_grammar_verify_keys.argtypes = [I32, P, P, I32, P, P, I32, P, I32, P]
    L.so_request_keys.argtypes = [I32, P, P, I32, P, P, I32, P, I32, P]
    L.so_request_advance.argtypes = [I32, P, P, I32, P, P, I32, P, I32, P, P]
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def mix(seed: int, position: int) -> int:
    return int(lib().so_mix(seed, position))


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().so_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def uniforms(seed: int, position: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().so_uniforms(seed, position, n, _ptr(out))
    return out


def gumbel(u: float) -> float:
    return float(lib().so_gumbel(u))


def process_row(x, params, mask=None, history=None, extra=None):
    x = _c(x, np.float32)
    V = x.shape[-1]
    p = _c(params, PARAMS_DTYPE).reshape(1)
    mask = _c(mask, np.uint32)
    h = _c(history, np.int32)
    e = _c(extra, np.int32)
    out = np.zeros(V, dtype=np.float32)
    st = lib().so_process_row(_ptr(x), V, _ptr(mask), _ptr(h), 0 if h is None else h.size,
                              _ptr(e), 0 if e is None else e.size, _ptr(p), _ptr(out))
    return int(st), out


def sample(x, params, mask=None, history=None, history_len=None, noise_mode=NOISE_ICDF,
           noise=None, want_probs=False, nthreads=0):
    """Batched oracle sample. x float32 [B,V]. Returns a dict of numpy arrays."""
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None]
    B, V = x.shape
    p = _c(params, PARAMS_DTYPE).reshape(B)
    mask = _c(mask, np.uint32)
    mstride = 0 if mask is None else mask.reshape(B, -1).shape[1]
    h = _c(history, np.int32)
    H = 0 if h is None else h.reshape(B, -1).shape[1]
    hl = _c(history_len, np.int32)
    nz = _c(noise, np.float32)
    res = np.zeros(B, dtype=ROW_RESULT_DTYPE)
    probs = np.zeros((B, V), dtype=np.float32) if want_probs else None
    lib().so_sample_batch(_ptr(x), B, V, _ptr(p), _ptr(mask), mstride, _ptr(h), _ptr(hl), H,
                          noise_mode, _ptr(nz), _ptr(res), _ptr(probs), nthreads)
    out = {name: res[name].copy() for name in ROW_RESULT_DTYPE.names if name != "pad"}
    out["probs"] = probs
    return out


def verify(target, k, draft_tokens, params, draft_logits=None, draft_to_full=None, mask=None,
           history=None, history_len=None, noise_mode=NOISE_ICDF, noise=None, want_probs=False,
           nthreads=0):
    """Batched oracle verify. target float32 [B,k+1,V]; draft_tokens int32 [B,k]."""
    t = _c(target, np.float32)
    B = t.shape[0]
    V = t.shape[-1]
    t = t.reshape(B, k + 1, V)
    dt = _c(draft_tokens, np.int32).reshape(B, max(k, 0))
    p = _c(params, PARAMS_DTYPE).reshape(B)
    dl = _c(draft_logits, np.float32)
    Vd = 0 if dl is None else dl.shape[-1]
    tab = _c(draft_to_full, np.int32)
    mask = _c(mask, np.uint32)
    mstride = 0 if mask is None else mask.reshape(B * (k + 1), -1).shape[1]
    h = _c(history, np.int32)
    H = 0 if h is None else h.reshape(B, -1).shape[1]
    hl = _c(history_len, np.int32)
    nz = _c(noise, np.float32)
    acc = np.zeros(B, dtype=np.int32)
    tok = np.zeros(B, dtype=np.int32)
    racc = np.zeros((B, max(k, 1)), dtype=np.int32)
    rtok = np.zeros((B, k + 1), dtype=np.int32)
    st = np.zeros(B, dtype=np.int32)
    mg = np.zeros(B, dtype=np.float64)
    probs = np.zeros((B, k + 1, V), dtype=np.float32) if want_probs else None
    lib().so_verify_batch(_ptr(t), B, k, V, _ptr(dl), Vd, _ptr(tab), _ptr(dt), _ptr(p), _ptr(mask),
                          mstride, _ptr(h), _ptr(hl), H, noise_mode, _ptr(nz), _ptr(acc), _ptr(tok),
                          _ptr(racc), _ptr(rtok), _ptr(st), _ptr(mg), _ptr(probs), nthreads)
    return {"accepted": acc, "token": tok, "row_accept": racc[:, :k], "row_token": rtok,
            "status": st, "margin": mg, "probs": probs}


def pack_mask(allowed: np.ndarray) -> np.ndarray:
    """bool [..., V] -> uint32 [..., ceil(V/32)], bit (i & 31) of word (i >> 5)."""
    allowed = np.asarray(allowed, dtype=bool)
    V = allowed.shape[-1]
    W = (V + 31) // 32
    pad = np.zeros(allowed.shape[:-1] + (W * 32,), dtype=bool)
    pad[..., :V] = allowed
    bits = pad.reshape(allowed.shape[:-1] + (W, 32)).astype(np.uint64)
    return (bits << np.arange(32, dtype=np.uint64)).sum(axis=-1).astype(np.uint32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16 value, returned as float32 (exact)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


def bf16_bits(x_f32_bf16exact: np.ndarray) -> np.ndarray:
    """float32 values that are exact bf16 -> uint16 bit patterns."""
    return (np.ascontiguousarray(x_f32_bf16exact, dtype=np.float32).view(np.uint32) >> 16).astype(
        np.uint16)


if __name__ == "__main__":  # pragma: no cover
    print(os.fspath(build(force=True)))


# ---------------------------------------------------------------------------------
# grammar masks (oracle/grammar_oracle.c)
# ---------------------------------------------------------------------------------
class GrammarOracle:
    """The reference's host mask production (GrammarVocab.swift:16-112) over a vocabulary
    given as byte strings; masks are packed u32 words like strim_grammar_masks."""

    def __init__(self, tokens, width: int, eos=(), skip=None):
        self.count = len(tokens)
        lens = np.array([len(t) for t in tokens], dtype=np.int64)
        self.offsets = np.zeros(self.count + 1, dtype=np.uint32)
        self.offsets[1:] = np.cumsum(lens)
        self.bytes = np.frombuffer(b"".join(bytes(t) for t in tokens) + b"\0", dtype=np.uint8).copy()
        self.skip = None if skip is None else np.ascontiguousarray(skip, dtype=np.uint8)
        self.width = int(width)
        self.eos = np.ascontiguousarray(eos, dtype=np.int32)
        self._trie = lib().so_trie_build(self.count, _ptr(self.offsets), _ptr(self.bytes),
                                         _ptr(self.skip))
        self.next = None
        self.flags = None

    def __del__(self):  # pragma: no cover - best effort
        if getattr(self, "_trie", None):
            lib().so_trie_free(self._trie)
            self._trie = None

    def nodes(self) -> int:
        return int(lib().so_trie_nodes(self._trie))

    def set_dfa(self, next_table, flags):
        self.next = np.ascontiguousarray(next_table, dtype=np.int32)
        self.flags = np.ascontiguousarray(flags, dtype=np.uint8)

    def mask(self, key: int) -> np.ndarray:
        out = np.zeros((self.width + 31) // 32, dtype=np.uint32)
        lib().so_grammar_mask(self._trie, self.width, _ptr(self.eos), len(self.eos),
                              len(self.flags), _ptr(self.next), _ptr(self.flags), int(key),
                              _ptr(out))
        return out

    def advance(self, state: int, token_bytes: bytes) -> int:
        b = np.frombuffer(bytes(token_bytes) + b"\0", dtype=np.uint8).copy()
        return int(lib().so_grammar_advance_bytes(int(state), _ptr(b), len(token_bytes),
                                                  _ptr(self.next)))

    def verify_keys(self, state, tokens) -> np.ndarray:
        st = np.ascontiguousarray(state, dtype=np.int32)
        tk = np.ascontiguousarray(tokens, dtype=np.int32).reshape(len(st), -1)
        k = tk.shape[1]
        out = np.zeros((len(st), k + 1), dtype=np.int32)
        lib().so_grammar_verify_keys(self.count, _ptr(self.offsets), _ptr(self.bytes),
                                     len(self.flags), _ptr(self.next), _ptr(st), len(st),
                                     _ptr(tk), k, _ptr(out))
        return out

    def request_keys(self, states, drafts=None) -> np.ndarray:
        """RequestConstraint.key / verifyMask keys [B][k + 1] of REQUEST_STATE_DTYPE rows."""
        st = np.ascontiguousarray(states, dtype=REQUEST_STATE_DTYPE).reshape(-1)
        B = len(st)
        tk = (np.zeros((B, 0), np.int32) if drafts is None
              else np.ascontiguousarray(drafts, dtype=np.int32).reshape(B, -1))
        k = tk.shape[1]
        out = np.zeros((B, k + 1), dtype=np.int32)
        lib().so_request_keys(self.count, _ptr(self.offsets), _ptr(self.bytes), len(self.flags),
                              _ptr(self.next), _ptr(st), B, _ptr(tk) if k else None, k,
                              _ptr(out))
        return out

    def request_advance(self, states, last, drafts=None, accepted=None) -> np.ndarray:
        """RequestConstraint.advance by drafts[0 .. accepted) then last; returns new states."""
        st = np.ascontiguousarray(states, dtype=REQUEST_STATE_DTYPE).reshape(-1).copy()
        B = len(st)
        tk = (np.zeros((B, 0), np.int32) if drafts is None
              else np.ascontiguousarray(drafts, dtype=np.int32).reshape(B, -1))
        acc = None if accepted is None else np.ascontiguousarray(accepted, dtype=np.int32)
        ls = np.ascontiguousarray(last, dtype=np.int32).reshape(B)
        lib().so_request_advance(self.count, _ptr(self.offsets), _ptr(self.bytes),
                                 len(self.flags), _ptr(self.next), _ptr(st), B,
                                 _ptr(tk) if tk.shape[1] else None, tk.shape[1], _ptr(acc),
                                 _ptr(ls))
        return st


# RequestConstraint.State and its constants (strim_request_state, 24 bytes)
REQUEST_STATE_DTYPE = np.dtype([("g", "<i4"), ("in_think", "<i4"), ("count", "<i4"),
                                ("budget", "<i4"), ("close_id", "<i4"), ("violated", "<i4")])
