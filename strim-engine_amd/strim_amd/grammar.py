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

Several grammars share one device table (GrammarEngine's programs,
GrammarVocab.swift:116-147): `add_program` registers a host DFA that interns its states
lazily (the GrammarDFA interface: `start`, `next(s, b)`, `accepting(s)`,
`consuming(s)`, GrammarDFA.swift:13-58). Its states enter the table as the device walks
reach them: a walk that meets a transition not interned yet reports it, the host asks the
program for the target and appends or fills the table, and the masks are produced again
(`masks` and `request_keys` run that loop while programs are registered). At most
`max_programs` programs keep cached masks; the least recently used one's masks are
dropped (GrammarEngine.runtime and trim, GrammarVocab.swift:132-156).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _native as N

FREE = -1
ACCEPTING = 1  # STRIM_DFA_ACCEPTING
CONSUMING = 2  # STRIM_DFA_CONSUMING
DEAD = -1  # STRIM_DFA_DEAD
UNKNOWN = -2  # STRIM_DFA_UNKNOWN: a table entry not interned yet
UNRESOLVED = 0x7FFFFFFF  # STRIM_GRAMMAR_UNRESOLVED: a key walk met an UNKNOWN entry


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


class _Program:
    """A registered host DFA: its local states' global ids, and the inverse."""

    def __init__(self, key, dfa):
        self.key = key
        self.dfa = dfa
        self.glob = {}  # local state -> global id
        self.ranges = []  # (first, n) of its appended global ids
        self.last_used = 0
        self.resident = True  # its masks may be cached


class DeviceGrammar:
    """Vocabulary + DFA table + mask cache on one GPU.

    tokens: byte strings per id (GrammarEngine.tokenBytes); width: logits width; eos: the
    end-of-turn ids; skip: ids never in a grammar mask (control tokens);
    cache_slots: mask rows kept in HBM (width / 8 bytes each), the cache's budget; the
    default holds the reference's 32 MB mask budget at width 151,936
    (GrammarVocab.swift:124).
    """

    MAX_PROGRAMS = 16  # GrammarEngine.maxPrograms (GrammarVocab.swift:123)

    def __init__(self, tokens, width: int, eos=(), skip=None, device: int = 0,
                 cache_slots: int | None = None, max_programs: int = MAX_PROGRAMS):
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
        if cache_slots is None:
            cache_slots = max(2, (32 << 20) // (self.words * 4))
        h = ctypes.c_void_p()
        N.check(N.lib().strim_grammar_create(ctypes.byref(h), device, self.count,
                                             _np_ptr(offsets), _np_ptr(data), _np_ptr(sk),
                                             self.width, _np_ptr(ev), len(ev), cache_slots),
                "strim_grammar_create")
        self._h = h
        self.n_states = 0
        self.max_programs = int(max_programs)
        self._programs = {}  # key -> _Program
        self._owner = {}  # global id -> (program, local state)
        self._tick = 0

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

    @staticmethod
    def _table(next_table, flags):
        nt = np.ascontiguousarray(next_table, dtype=np.int32)
        fl = np.ascontiguousarray(flags, dtype=np.uint8)
        if nt.ndim != 2 or nt.shape[1] != 256 or fl.shape != (nt.shape[0],):
            raise ValueError("next_table must be [S][256] and flags [S]")
        return nt, fl

    def set_dfa(self, next_table, flags, stream=None) -> None:
        """Replaces the table with one DFA: next_table [S][256] (DEAD, UNKNOWN or a
        state), flags [S]. Registered programs are forgotten."""
        nt, fl = self._table(next_table, flags)
        N.check(N.lib().strim_grammar_set_dfa(self.handle, _stream(stream), nt.shape[0],
                                              _np_ptr(nt), _np_ptr(fl)),
                "strim_grammar_set_dfa")
        self.n_states = nt.shape[0]
        self._programs.clear()
        self._owner.clear()

    def append_states(self, next_table, flags, stream=None) -> int:
        """Appends states (entries are global ids, DEAD or UNKNOWN); returns the first
        new id. Cached masks stay."""
        nt, fl = self._table(next_table, flags)
        first = ctypes.c_int32()
        N.check(N.lib().strim_grammar_append_states(self.handle, _stream(stream), nt.shape[0],
                                                    _np_ptr(nt), _np_ptr(fl),
                                                    ctypes.byref(first)),
                "strim_grammar_append_states")
        self.n_states += nt.shape[0]
        return int(first.value)

    def set_next(self, where, to, stream=None) -> None:
        """Fills UNKNOWN entries: entry where[i] (state * 256 + byte) becomes to[i]."""
        w = np.ascontiguousarray(where, dtype=np.int64)
        t = np.ascontiguousarray(to, dtype=np.int32)
        if w.shape != t.shape or w.ndim != 1:
            raise ValueError("where and to must be 1-D of one length")
        N.check(N.lib().strim_grammar_set_next(self.handle, _stream(stream), w.size,
                                               _np_ptr(w), _np_ptr(t)),
                "strim_grammar_set_next")

    def pending(self, cap: int = 1 << 16, stream=None) -> np.ndarray:
        """The UNKNOWN entries (state * 256 + byte) walks met since the last call."""
        out = np.empty(cap, dtype=np.int64)
        n = ctypes.c_int32()
        N.check(N.lib().strim_grammar_pending(self.handle, _stream(stream), _np_ptr(out), cap,
                                              ctypes.byref(n)),
                "strim_grammar_pending")
        return out[:n.value].copy()

    def drop_masks(self, first: int, n: int, stream=None) -> None:
        """Forgets the cached masks of states [first, first + n)."""
        N.check(N.lib().strim_grammar_drop_masks(self.handle, _stream(stream), int(first),
                                                 int(n)),
                "strim_grammar_drop_masks")

    # ---- programs: lazily interned DFAs in the shared table ----------------------
    def _intern(self, prog: _Program, locals_, stream=None):
        """Appends the program's local states not in the table yet (rows all UNKNOWN)."""
        new = [s for s in dict.fromkeys(locals_) if s not in prog.glob]
        if not new:
            return
        fl = np.array([(ACCEPTING if prog.dfa.accepting(s) else 0)
                       | (CONSUMING if prog.dfa.consuming(s) else 0) for s in new], np.uint8)
        nt = np.full((len(new), 256), UNKNOWN, dtype=np.int32)
        first = self.append_states(nt, fl, stream)
        prog.ranges.append((first, len(new)))
        for i, s in enumerate(new):
            prog.glob[s] = first + i
            self._owner[first + i] = (prog, s)

    def add_program(self, key, dfa, stream=None) -> int:
        """Registers (or touches) the program `key` served by the host DFA `dfa`;
        returns the global id of its start state. Past max_programs programs, the least
        recently used one's cached masks are dropped (its states stay resolvable)."""
        self._tick += 1
        prog = self._programs.get(key)
        if prog is None:
            prog = _Program(key, dfa)
            self._programs[key] = prog
            self._intern(prog, [dfa.start], stream)
        prog.last_used = self._tick
        prog.resident = True
        resident = [p for p in self._programs.values() if p.resident]
        if len(resident) > self.max_programs:
            old = min(resident, key=lambda p: p.last_used)
            for first, n in old.ranges:
                self.drop_masks(first, n, stream)
            old.resident = False
        return prog.glob[prog.dfa.start]

    def resolve(self, stream=None) -> int:
        """Fills every UNKNOWN entry walks have met: the owning program's DFA gives each
        target, interned if new. Returns how many entries were filled."""
        done = 0
        while True:
            pend = self.pending(stream=stream)
            if pend.size == 0:
                return done
            targets, new = [], {}
            for e in pend.tolist():
                gs, b = divmod(int(e), 256)
                if gs not in self._owner:
                    raise ValueError(f"state {gs} belongs to no registered program")
                prog, ls = self._owner[gs]
                t = prog.dfa.next(ls, b)
                targets.append((prog, t))
                if t >= 0:
                    new.setdefault(id(prog), (prog, []))[1].append(t)
            for prog, ts in new.values():
                self._intern(prog, ts, stream)
            to = [prog.glob[t] if t >= 0 else DEAD for prog, t in targets]
            self.set_next(pend, to, stream)
            done += pend.size

    def masks(self, keys: torch.Tensor, out: torch.Tensor | None = None,
              stream=None, resolve: bool | None = None) -> torch.Tensor:
        """Mask words [n][words] (int32 view of the u32 words) for device keys [n]. With
        programs registered (or resolve=True) the walks' unknown entries are filled and
        the masks produced again until none is met."""
        if resolve is None:
            resolve = bool(self._programs)
        while True:
            out = self._masks(keys, out, stream)
            if not resolve or self.resolve(stream) == 0:
                return out

    def _masks(self, keys, out, stream):
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
                     stream=None, resolve: bool | None = None) -> torch.Tensor:
        """RequestConstraint.key / verifyMask on the device: keys [B][k + 1] of the next
        row and of the rows after each draft (states unchanged). With programs registered
        (or resolve=True), draft walks that meet unknown entries are resolved and the
        keys computed again."""
        if resolve is None:
            resolve = bool(self._programs)
        while True:
            out = self._request_keys(states, drafts, stream)
            if not resolve or self.resolve(stream) == 0:
                return out

    def _request_keys(self, states, drafts, stream):
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
