"""On-device grammar masks: the host mirror of the reference's grammar runtime over the C ABI
(include/strim_grammar.h).

`DeviceGrammar` stands for the reference's GrammarRuntime plus DeviceMasks
(Sources/StrimEngine/GrammarVocab.swift:56-113, RequestConstraint.swift:5-60): the
vocabulary bytes, the DFA and the per-state mask cache live on the GPU, masks come out as
the packed u32 words `Context.sample` / `Context.verify` take, and verify-row keys are
stepped by the drafts on the device (RequestConstraint.verifyMask,
RequestConstraint.swift:134-152). Keys: a DFA state (>= 0), FREE (-1) or forced(id).

Per-request constraint state (RequestConstraint.State with its budget and close id,
RequestConstraint.swift:62-109) is a device tensor of REQUEST_STATE rows: `request_keys`
gives the next-token and verify-row keys (the thinking budget's forced close id included)
and `request_advance` steps the states by the emitted tokens, both on the device.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _native as N

FREE = -1
ACCEPTING = 1  # STRIM_DFA_ACCEPTING
CONSUMING = 2  # STRIM_DFA_CONSUMING


# strim_request_state: {g, in_think, count, budget, close_id, violated}
REQUEST_STATE = np.dtype([("g", "<i4"), ("in_think", "<i4"), ("count", "<i4"),
                          ("budget", "<i4"), ("close_id", "<i4"), ("violated", "<i4")])


def request_states(n: int, grammar_state=-1, in_think=False, budget=None, close_id=-1):
    """Host REQUEST_STATE rows for new requests (RequestConstraint.init,
    RequestConstraint.swift:79-83): grammar_state is the DFA start (-1 for no grammar),
    in_think the startsInThink flag, budget None for no thinking budget."""
    s = np.zeros(n, dtype=REQUEST_STATE)
    s["g"] = grammar_state
    s["in_think"] = np.asarray(in_think, dtype=np.int32)
    s["budget"] = -1 if budget is None else budget
    s["close_id"] = close_id
    return s


def states_to_device(states: np.ndarray, device: int = 0) -> torch.Tensor:
    """REQUEST_STATE rows -> int32 [n, 6] on the GPU (the C struct's layout)."""
    a = np.ascontiguousarray(states, dtype=REQUEST_STATE).view(np.int32).reshape(-1, 6)
    return torch.from_numpy(a.copy()).to(f"cuda:{device}")


def states_from_device(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.cpu().numpy(), dtype=np.int32).view(REQUEST_STATE).reshape(-1)


def forced(token_id: int) -> int:
    """The key of a row that allows only `token_id` (DeviceMasks.only)."""
    return -2 - int(token_id)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _np_ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _stream(stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


class DeviceGrammar:
    """Vocabulary + DFA + mask cache on one GPU.

    tokens: byte strings per id (GrammarEngine.tokenBytes); width: logits width; eos: the
    end-of-turn ids; skip: ids never in a grammar mask (control tokens);
    cache_states: states whose masks stay cached in HBM (width / 8 bytes each).
    """

    def __init__(self, tokens, width: int, eos=(), skip=None, device: int = 0,
                 cache_states: int = 1024):
        self.count = len(tokens)
        self.width = int(width)
        self.words = (self.width + 31) // 32
        self.device = device
        self.tokens = [bytes(t) for t in tokens]
        lens = np.array([len(t) for t in self.tokens], dtype=np.int64)
        offsets = np.zeros(self.count + 1, dtype=np.uint32)
        offsets[1:] = np.cumsum(lens)
        data = np.frombuffer(b"".join(self.tokens) + b"\0", dtype=np.uint8).copy()
        sk = None if skip is None else np.ascontiguousarray(skip, dtype=np.uint8)
        if sk is not None and sk.shape != (self.count,):
            raise ValueError("skip must have one entry per token")
        ev = np.ascontiguousarray(list(eos), dtype=np.int32)
        h = ctypes.c_void_p()
        N.check(N.lib().strim_grammar_create(ctypes.byref(h), device, self.count,
                                             _np_ptr(offsets), _np_ptr(data), _np_ptr(sk),
                                             self.width, _np_ptr(ev), len(ev), cache_states),
                "strim_grammar_create")
        self._h = h
        self.n_states = 0

    @property
    def handle(self):
        if self._h is None:
            raise ValueError("grammar is closed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            N.lib().strim_grammar_destroy(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    def set_dfa(self, next_table, flags, stream=None) -> None:
        """Installs a fully materialised DFA: next_table [S][256] (-1 dead), flags [S]."""
        nt = np.ascontiguousarray(next_table, dtype=np.int32)
        fl = np.ascontiguousarray(flags, dtype=np.uint8)
        if nt.ndim != 2 or nt.shape[1] != 256 or fl.shape != (nt.shape[0],):
            raise ValueError("next_table must be [S][256] and flags [S]")
        N.check(N.lib().strim_grammar_set_dfa(self.handle, _stream(stream), nt.shape[0],
                                              _np_ptr(nt), _np_ptr(fl)),
                "strim_grammar_set_dfa")
        self.n_states = nt.shape[0]

    def masks(self, keys: torch.Tensor, out: torch.Tensor | None = None,
              stream=None) -> torch.Tensor:
        """Mask words [n][words] (int32 view of the u32 words) for device keys [n]."""
        if keys.dtype != torch.int32 or not keys.is_cuda or keys.dim() != 1:
            raise ValueError("keys must be a 1-D int32 CUDA tensor")
        keys = keys.contiguous()
        n = keys.numel()
        if out is None:
            out = torch.empty((n, self.words), dtype=torch.int32, device=keys.device)
        if out.dim() != 2 or out.shape[0] != n or out.shape[1] < self.words or out.stride(1) != 1:
            raise ValueError("out must be [n][>= words] with unit column stride")
        N.check(N.lib().strim_grammar_masks(self.handle, _stream(stream), _ptr(keys), n,
                                            _ptr(out), out.stride(0)),
                "strim_grammar_masks")
        return out

    def mask(self, key: int) -> torch.Tensor:
        """GrammarRuntime.mask for one key: [words] int32."""
        k = torch.tensor([int(key)], dtype=torch.int32, device=f"cuda:{self.device}")
        return self.masks(k)[0]

    def advance(self, state: torch.Tensor, tokens: torch.Tensor, stream=None) -> torch.Tensor:
        """Keys [B][k + 1] of the verify rows: state [B] int32, tokens [B][k] int32."""
        if state.dtype != torch.int32 or tokens.dtype != torch.int32:
            raise ValueError("state and tokens must be int32")
        state = state.contiguous()
        B = state.numel()
        tokens = tokens.reshape(B, -1).contiguous()
        k = tokens.shape[1]
        out = torch.empty((B, k + 1), dtype=torch.int32, device=state.device)
        N.check(N.lib().strim_grammar_advance(self.handle, _stream(stream), _ptr(state), B,
                                              _ptr(tokens) if k > 0 else None, k, _ptr(out)),
                "strim_grammar_advance")
        return out

    def verify_masks(self, state: torch.Tensor, drafts: torch.Tensor, stream=None):
        """RequestConstraint.verifyMask on the device: (keys [B][k + 1],
        masks [B * (k + 1)][words]) with the rows in the order strim_verify reads them."""
        keys = self.advance(state, drafts, stream)
        return keys, self.masks(keys.reshape(-1), stream=stream)

    # ---- per-request constraint state --------------------------------------------
    @staticmethod
    def _check_states(states: torch.Tensor) -> int:
        if states.dtype != torch.int32 or not states.is_cuda or states.dim() != 2 \
                or states.shape[1] != 6 or not states.is_contiguous():
            raise ValueError("states must be a contiguous int32 CUDA tensor [B, 6]")
        return states.shape[0]

    def request_keys(self, states: torch.Tensor, drafts: torch.Tensor | None = None,
                     stream=None) -> torch.Tensor:
        """RequestConstraint.key / verifyMask on the device: keys [B][k + 1] of the next
        row and of the rows after each draft (states unchanged)."""
        B = self._check_states(states)
        if drafts is not None and drafts.numel() > 0:
            drafts = drafts.reshape(B, -1).to(torch.int32).contiguous()
            k = drafts.shape[1]
        else:
            drafts, k = None, 0
        out = torch.empty((B, k + 1), dtype=torch.int32, device=states.device)
        N.check(N.lib().strim_request_keys(self.handle, _stream(stream), _ptr(states), B,
                                           _ptr(drafts), k, _ptr(out)),
                "strim_request_keys")
        return out

    def request_advance(self, states: torch.Tensor, last: torch.Tensor,
                        drafts: torch.Tensor | None = None,
                        accepted: torch.Tensor | None = None, stream=None) -> None:
        """RequestConstraint.advance on the device, in place: each request takes
        drafts[b][0 .. accepted[b]) and then last[b] (strim_verify's outputs), or last[b]
        alone (strim_sample's)."""
        B = self._check_states(states)
        last = last.reshape(B).to(torch.int32).contiguous()
        if drafts is not None and drafts.numel() > 0:
            drafts = drafts.reshape(B, -1).to(torch.int32).contiguous()
            k = drafts.shape[1]
        else:
            drafts, k = None, 0
        acc = None if accepted is None else accepted.reshape(B).to(torch.int32).contiguous()
        N.check(N.lib().strim_request_advance(self.handle, _stream(stream), _ptr(states), B,
                                              _ptr(drafts), k, _ptr(acc), _ptr(last)),
                "strim_request_advance")
