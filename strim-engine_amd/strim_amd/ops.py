"""Device-tensor front end of the C ABI.

Torch is used only to hold device memory and the current HIP stream; every
computation runs in libstrim_sampler.so. Inputs must already live on the GPU.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _native as N


def _ptr(t) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return N.DTYPE_BF16
    if t.dtype == torch.float32:
        return N.DTYPE_F32
    raise TypeError(f"logits must be bfloat16 or float32, got {t.dtype}")


def host_params(params) -> np.ndarray:
    """strim_sampling_params rows as a contiguous host array (the C ABI reads them at
    call time; the caller may reuse the memory as soon as the call returns)."""
    return np.ascontiguousarray(params, dtype=N.PARAMS_DTYPE).reshape(-1)


def _pp(p: np.ndarray) -> ctypes.c_void_p:
    return p.ctypes.data_as(ctypes.c_void_p)


def _check_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("every tensor argument must be on the GPU")
        if t is not None and not t.is_contiguous():
            raise ValueError("tensor arguments must be contiguous")


def _row_stride(t: torch.Tensor) -> int:
    """Elements between rows (a single row may carry any stride, e.g. 0 from a
    broadcast view: its own length is passed)."""
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def _check_rows(t: torch.Tensor) -> None:
    """Logits may have a row stride > V, but each row must be contiguous."""
    if not t.is_cuda:
        raise ValueError("logits must be on the GPU")
    if t.dim() != 2 or t.stride(1) != 1 or _row_stride(t) < t.shape[1]:
        raise ValueError("logits must be [R, V] with contiguous rows (row stride >= V)")


class Context:
    """strim_ctx: scratch for up to max_rows rows of up to max_vocab tokens."""

    def __init__(self, device: int = 0, max_rows: int = 64, max_vocab: int = 262144):
        self.device = device
        self.max_rows = max_rows
        self.max_vocab = max_vocab
        h = ctypes.c_void_p()
        with torch.cuda.device(device):
            N.check(N.lib().strim_ctx_create(ctypes.byref(h), device, max_rows, max_vocab),
                    "strim_ctx_create")
        self._h = h

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            torch.cuda.synchronize(self.device)
            N.check(N.lib().strim_ctx_destroy(self._h), "strim_ctx_destroy")
            self._h = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    # -------------------------------------------------------------------------
    def profile_begin(self, max_launches: int) -> None:
        N.check(N.lib().strim_profile_begin(self._h, max_launches), "strim_profile_begin")

    def profile_end(self) -> dict:
        """{kernel name: (total ms, launches)} since profile_begin (synchronises)."""
        tot = np.zeros(N.KERNEL_COUNT, np.float64)
        cnt = np.zeros(N.KERNEL_COUNT, np.int64)
        N.check(N.lib().strim_profile_end(self._h, tot.ctypes.data_as(ctypes.c_void_p),
                                          cnt.ctypes.data_as(ctypes.c_void_p)),
                "strim_profile_end")
        return {N.lib().strim_kernel_name(i).decode(): (float(tot[i]), int(cnt[i]))
                for i in range(N.KERNEL_COUNT)}

    def sample(self, logits: torch.Tensor, params, mask: torch.Tensor | None = None,
               history: torch.Tensor | None = None, history_len: torch.Tensor | None = None,
               noise_mode: int = N.NOISE_ICDF, noise: torch.Tensor | None = None,
               want_probs: bool = False, out_ids: torch.Tensor | None = None,
               out_status: torch.Tensor | None = None, stream=None):
        """strim_sample over logits [B,V]. Returns (ids int32[B], status int32[B],
        probs float32[B,V] or None), all on the device."""
        if logits.dim() == 1:
            logits = logits.unsqueeze(0)
        B, V = logits.shape
        dev = logits.device
        p = host_params(params)
        if p.size != B:
            raise ValueError(f"need {B} param rows, got {p.size}")
        _check_rows(logits)
        _check_cuda(mask, history, history_len, noise)
        if out_ids is None:
            out_ids = torch.empty(B, dtype=torch.int32, device=dev)
        if out_status is None:
            out_status = torch.empty(B, dtype=torch.int32, device=dev)
        probs = torch.empty(B, V, dtype=torch.float32, device=dev) if want_probs else None
        H = 0 if history is None else history.shape[-1]
        mstride = 0 if mask is None else mask.shape[-1]
        rc = N.lib().strim_sample(self._h, _stream(stream), _ptr(logits), _dtype_code(logits),
                                  B, V, _row_stride(logits), _pp(p), _ptr(mask), mstride,
                                  _ptr(history), _ptr(history_len), H, noise_mode, _ptr(noise),
                                  _ptr(out_ids), _ptr(out_status), _ptr(probs))
        N.check(rc, "strim_sample")
        return out_ids, out_status, probs

    def bind_sample(self, logits: torch.Tensor, params, mask: torch.Tensor | None = None,
                    history: torch.Tensor | None = None,
                    history_len: torch.Tensor | None = None, noise_mode: int = N.NOISE_ICDF,
                    noise: torch.Tensor | None = None, out_ids: torch.Tensor | None = None,
                    out_status: torch.Tensor | None = None, stream=None) -> "BoundCall":
        """strim_sample with every argument converted once: calling the result launches
        the step again on the same buffers (the tensors must stay alive). For loops that
        reuse buffers, such as a decode loop or HIP-graph capture."""
        if logits.dim() == 1:
            logits = logits.unsqueeze(0)
        B, V = logits.shape
        dev = logits.device
        p = host_params(params)
        if p.size != B:
            raise ValueError(f"need {B} param rows, got {p.size}")
        _check_rows(logits)
        _check_cuda(mask, history, history_len, noise)
        if out_ids is None:
            out_ids = torch.empty(B, dtype=torch.int32, device=dev)
        if out_status is None:
            out_status = torch.empty(B, dtype=torch.int32, device=dev)
        H = 0 if history is None else history.shape[-1]
        mstride = 0 if mask is None else mask.shape[-1]
        args = [self._h, None, _ptr(logits), _dtype_code(logits), B, V,
                _row_stride(logits), _pp(p), _ptr(mask), mstride, _ptr(history), _ptr(history_len),
                H, noise_mode, _ptr(noise), _ptr(out_ids), _ptr(out_status), None]
        keep = (logits, p, mask, history, history_len, noise, out_ids, out_status)
        return BoundCall(N.lib().strim_sample, args, keep, out_ids, out_status, stream)

    def verify(self, target_logits: torch.Tensor, draft_tokens: torch.Tensor | None, params,
               draft_logits: torch.Tensor | None = None,
               draft_to_full: torch.Tensor | None = None, mask: torch.Tensor | None = None,
               history: torch.Tensor | None = None, history_len: torch.Tensor | None = None,
               noise_mode: int = N.NOISE_ICDF, noise: torch.Tensor | None = None,
               row_outputs: bool = True, stream=None):
        """strim_verify over target [B,k+1,V]. Returns a dict of device tensors:
        accepted [B], token [B], status [B], row_accept [B,k], row_token [B,k+1]."""
        B, k1, V = target_logits.shape
        k = k1 - 1
        dev = target_logits.device
        p = host_params(params)
        if p.size != B:
            raise ValueError(f"need {B} param rows, got {p.size}")
        _check_cuda(target_logits, draft_tokens, draft_logits, draft_to_full, mask, history,
                    history_len, noise)
        acc = torch.empty(B, dtype=torch.int32, device=dev)
        tok = torch.empty(B, dtype=torch.int32, device=dev)
        st = torch.empty(B, dtype=torch.int32, device=dev)
        racc = torch.empty(B, max(k, 1), dtype=torch.int32, device=dev) if row_outputs else None
        rtok = torch.empty(B, k + 1, dtype=torch.int32, device=dev) if row_outputs else None
        H = 0 if history is None else history.shape[-1]
        mstride = 0 if mask is None else mask.shape[-1]
        Vd = 0 if draft_logits is None else draft_logits.shape[-1]
        if draft_logits is not None:
            if draft_logits.dtype != target_logits.dtype:
                raise ValueError("draft_logits must have the target logits' dtype")
            if tuple(draft_logits.shape) != (B, k, Vd) or not draft_logits.is_contiguous():
                raise ValueError(f"draft_logits must be contiguous [{B}, {k}, Vd]")
            if draft_to_full is None or draft_to_full.numel() != Vd:
                raise ValueError("draft_to_full must hold Vd ids")
        rc = N.lib().strim_verify(self._h, _stream(stream), _ptr(target_logits),
                                  _dtype_code(target_logits), B, k, V, _ptr(draft_logits), Vd,
                                  _ptr(draft_to_full), _ptr(draft_tokens), _pp(p), _ptr(mask),
                                  mstride, _ptr(history), _ptr(history_len), H, noise_mode,
                                  _ptr(noise), _ptr(acc), _ptr(tok), _ptr(racc), _ptr(rtok),
                                  _ptr(st))
        N.check(rc, "strim_verify")
        return {"accepted": acc, "token": tok, "status": st,
                "row_accept": None if racc is None else racc[:, :k], "row_token": rtok}


    def bind_verify(self, target_logits: torch.Tensor, draft_tokens: torch.Tensor, params,
                    draft_logits: torch.Tensor | None = None,
                    draft_to_full: torch.Tensor | None = None,
                    noise_mode: int = N.NOISE_GUMBEL, noise: torch.Tensor | None = None,
                    stream=None) -> "BoundCall":
        """strim_verify with every argument converted and the outputs allocated once:
        calling the result launches the verify again on the same buffers (for HIP-graph
        capture). Its out_ids / out_status are the accepted counts and the tokens."""
        B, k1, V = target_logits.shape
        k = k1 - 1
        dev = target_logits.device
        p = host_params(params)
        if p.size != B:
            raise ValueError(f"need {B} param rows, got {p.size}")
        _check_cuda(target_logits, draft_tokens, draft_logits, draft_to_full, noise)
        Vd = 0 if draft_logits is None else draft_logits.shape[-1]
        if draft_logits is not None and (tuple(draft_logits.shape) != (B, k, Vd)
                                         or not draft_logits.is_contiguous()
                                         or draft_logits.dtype != target_logits.dtype):
            raise ValueError(f"draft_logits must be contiguous [{B}, {k}, Vd] of the target dtype")
        acc = torch.empty(B, dtype=torch.int32, device=dev)
        tok = torch.empty(B, dtype=torch.int32, device=dev)
        st = torch.empty(B, dtype=torch.int32, device=dev)
        args = [self._h, None, _ptr(target_logits), _dtype_code(target_logits), B, k, V,
                _ptr(draft_logits), Vd, _ptr(draft_to_full), _ptr(draft_tokens), _pp(p), None, 0,
                None, None, 0, noise_mode, _ptr(noise), _ptr(acc), _ptr(tok), None, None,
                _ptr(st)]
        keep = (target_logits, draft_tokens, p, draft_logits, draft_to_full, noise, acc, tok, st)
        call = BoundCall(N.lib().strim_verify, args, keep, acc, tok, stream, "strim_verify")
        call.status = st
        return call


def mask_logits(logits: torch.Tensor, mask_words: torch.Tensor | None, stream=None):
    """maskLogits (TokenMask.swift:15-17): float32 logits with disallowed tokens at -inf."""
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    R, V = logits.shape
    _check_rows(logits)
    _check_cuda(mask_words)
    out = torch.empty(R, V, dtype=torch.float32, device=logits.device)
    mstride = 0 if mask_words is None else mask_words.shape[-1]
    N.check(N.lib().strim_mask_logits(_stream(stream), _ptr(logits), _dtype_code(logits), R, V,
                                      _row_stride(logits), _ptr(mask_words), mstride, _ptr(out)),
            "strim_mask_logits")
    return out


def head_logits(hidden: torch.Tensor, lm_head: torch.Tensor,
                norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                out: torch.Tensor | None = None, xn: torch.Tensor | None = None, stream=None):
    """The producer of the logits: final RMSNorm and dense lm_head of the decode step
    (QwenModel.swift:202-212; Weights.swift:244-255,270-273) on the GPU. hidden bf16 [B, K],
    lm_head bf16 [V, K], norm_weight bf16 [K] (None: hidden is already normalised).
    Returns bf16 logits [B, V] (or fills `out`), the layout sample/verify take."""
    if hidden.dim() == 1:
        hidden = hidden.unsqueeze(0)
    for t in (hidden, lm_head, norm_weight, out, xn):
        _check_cuda(t)
        if t is not None and t.dtype != torch.bfloat16:
            raise TypeError("head_logits takes bf16 tensors")
    B, K = hidden.shape
    V = lm_head.shape[0]
    if lm_head.shape[1] != K:
        raise ValueError(f"lm_head is [{lm_head.shape[0]}, {lm_head.shape[1]}], hidden K={K}")
    if out is None:
        out = torch.empty(B, V, dtype=torch.bfloat16, device=hidden.device)
    if norm_weight is not None and xn is None:
        xn = torch.empty(B, K, dtype=torch.bfloat16, device=hidden.device)
    N.check(N.lib().strim_head_logits(_stream(stream), _ptr(hidden), _row_stride(hidden), B, K,
                                      _ptr(norm_weight), float(eps), _ptr(xn), _ptr(lm_head),
                                      _row_stride(lm_head), V, _ptr(out), _row_stride(out)),
            "strim_head_logits")
    return out


def head_greedy(ctx: "Context", hidden: torch.Tensor, lm_head: torch.Tensor,
                norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                out_logits: torch.Tensor | None = None, xn: torch.Tensor | None = None,
                ids: torch.Tensor | None = None, status: torch.Tensor | None = None,
                stream=None):
    """Hidden -> greedy token with the pick fused into the producer (strim_head_greedy):
    the first maximum of each row's bf16 logits, which strim_sample gives for a T <= 0 row
    without penalties, mask or filters. out_logits None: the logits are not written.
    Returns (ids, status) int32 [B]."""
    if hidden.dim() == 1:
        hidden = hidden.unsqueeze(0)
    for t in (hidden, lm_head, norm_weight, out_logits, xn):
        _check_cuda(t)
        if t is not None and t.dtype != torch.bfloat16:
            raise TypeError("head_greedy takes bf16 tensors")
    B, K = hidden.shape
    V = lm_head.shape[0]
    if lm_head.shape[1] != K:
        raise ValueError(f"lm_head is [{lm_head.shape[0]}, {lm_head.shape[1]}], hidden K={K}")
    if norm_weight is not None and xn is None:
        xn = torch.empty(B, K, dtype=torch.bfloat16, device=hidden.device)
    if ids is None:
        ids = torch.empty(B, dtype=torch.int32, device=hidden.device)
    if status is None:
        status = torch.empty(B, dtype=torch.int32, device=hidden.device)
    N.check(N.lib().strim_head_greedy(ctx.handle, _stream(stream), _ptr(hidden),
                                      _row_stride(hidden), B, K, _ptr(norm_weight), float(eps),
                                      _ptr(xn), _ptr(lm_head), _row_stride(lm_head), V,
                                      _ptr(out_logits),
                                      _row_stride(out_logits) if out_logits is not None else 0,
                                      _ptr(ids), _ptr(status)),
            "strim_head_greedy")
    return ids, status


def draft_argmax(draft_logits: torch.Tensor, draft_to_full: torch.Tensor | None = None,
                 stream=None):
    """MTP.nextTokenIndex (MTP.swift:104-111): table[argmax(draft logits)] per row."""
    if draft_logits.dim() == 1:
        draft_logits = draft_logits.unsqueeze(0)
    R, Vd = draft_logits.shape
    _check_rows(draft_logits)
    _check_cuda(draft_to_full)
    out = torch.empty(R, dtype=torch.int32, device=draft_logits.device)
    N.check(N.lib().strim_draft_argmax(_stream(stream), _ptr(draft_logits),
                                       _dtype_code(draft_logits), R, Vd, _row_stride(draft_logits),
                                       _ptr(draft_to_full), _ptr(out)), "strim_draft_argmax")
    return out


def pack_mask(allowed: torch.Tensor) -> torch.Tensor:
    """bool [..., V] -> int32 words [..., ceil(V/32)], bit (i & 31) of word (i >> 5)
    (the byte layout of the reference's UInt64 bitset, GrammarVocab.swift:77-86)."""
    V = allowed.shape[-1]
    W = (V + 31) // 32
    pad = torch.zeros(allowed.shape[:-1] + (W * 32,), dtype=torch.int64, device=allowed.device)
    pad[..., :V] = allowed.to(torch.int64)
    bits = pad.reshape(allowed.shape[:-1] + (W, 32))
    words = (bits << torch.arange(32, device=allowed.device, dtype=torch.int64)).sum(-1)
    return _to_i32(words)


def _to_i32(words: torch.Tensor) -> torch.Tensor:
    w = words & 0xFFFFFFFF
    w = torch.where(w >= (1 << 31), w - (1 << 32), w)
    return w.to(torch.int32)


class BoundCall:
    """A strim_sample call with its ctypes arguments prepared (see Context.bind_sample).
    It launches on the given stream, or on the current stream at call time (so a graph
    capture records it)."""

    def __init__(self, fn, args, keep, out_ids, out_status, stream=None, name="strim_sample"):
        self._fn = fn
        self._args = args
        self._keep = keep
        self._stream = stream
        self._name = name
        self.out_ids = out_ids
        self.out_status = out_status

    def __call__(self) -> None:
        self._args[1] = _stream(self._stream)
        rc = self._fn(*self._args)
        if rc != N.OK:
            raise N.StrimError(rc, self._name)
