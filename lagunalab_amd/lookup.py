"""Prompt-lookup drafting and greedy acceptance for speculative decoding.

Mirrors ``laguna_mlx/dflash.py``:

* :class:`NgramIndex` -- the reference's host-side index (``dflash.py:145-167``): same
  constructor, ``ids`` / ``last`` attributes and ``extend`` / ``propose`` semantics.
* :class:`DeviceNgramIndex` -- the same proposals for a token history that lives on the GPU:
  ``propose`` runs the ``lq_ngram_propose`` scan kernel over the device history.
* :func:`ngram_propose` -- one scan: most recent earlier match of the last ``g`` ids of
  ``hist[:T]`` and up to ``n`` following ids (bit-exact with the reference's brute force).
* :func:`greedy_accept` -- argmax of each verify row (first index on ties) and the longest
  draft prefix equal to it (``dflash.py:195-198``), on the GPU.
"""
from __future__ import annotations

import torch

from . import _lib


class NgramIndex:
    """Host-side draft source of the prompt-lookup loop (``laguna_mlx/dflash.py:145-167``).

    ``last`` maps each g-token window of the history to the position where it most recently
    began; a window enters the map only once at least one token follows it, so the window formed
    by the newest g tokens is never its own match. ``propose(n)`` looks that newest window up and
    returns the (at most n) tokens that followed its latest earlier occurrence, cut at the end of
    the history; ``[]`` when there is none. The result equals a brute-force backward scan, and
    the device scan ``lq_ngram_propose`` returns the same ids."""

    def __init__(self, g):
        self.g, self.ids, self.last = g, [], {}

    def extend(self, tokens):
        g, ids = self.g, self.ids
        for t in tokens:
            ids.append(int(t))
            s = len(ids) - g - 1
            if s >= 0:
                self.last[tuple(ids[s:s + g])] = s

    def propose(self, n):
        t, g = len(self.ids), self.g
        s = self.last.get(tuple(self.ids[t - g:])) if t >= g else None
        return [] if s is None else self.ids[s + g:min(s + g + n, t)]


def _scratch(device, nbytes, cache={}):
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    t = cache.get(key)
    if t is None or t.numel() < nbytes:
        t = torch.empty(max(int(nbytes), 4096), dtype=torch.uint8, device=device)
        cache[key] = t
    return t


def ngram_propose(hist: torch.Tensor, T: int | None = None, g: int = 3, n: int = 4,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """Scan the int32 device history ``hist[:T]``. Returns the device result
    ``int32 [2 + n]``: ``[count, pos, id_0 .. id_{count-1}, ...]`` (``pos = -1`` if no match)."""
    lib = _lib.load()
    dev = _lib.require_device(hist, out)
    if hist.dtype != torch.int32 or hist.dim() != 1:
        raise ValueError("hist must be a 1-D int32 tensor")
    hist = hist.contiguous()
    T = hist.numel() if T is None else int(T)
    if not 0 <= T <= hist.numel():
        raise ValueError(f"T={T} outside [0, {hist.numel()}]")
    if out is None:
        out = torch.empty(2 + n, dtype=torch.int32, device=dev)
    ws = _scratch(dev, lib.lq_ngram_workspace_bytes(T))
    st = lib.lq_ngram_propose(hist.data_ptr(), T, int(g), int(n), out.data_ptr(), ws.data_ptr(),
                              ws.numel(), _lib.stream_ptr(dev))
    _lib.check(st, "lq_ngram_propose")
    return out


def greedy_accept(logits: torch.Tensor, drafts: torch.Tensor,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """``logits`` fp32 [L, V] (device), ``drafts`` int32 [m] (device), m <= L-1. Returns the device
    result int32 ``[2 + L]``: ``[k, next_token, argmax_0 .. argmax_{L-1}]``."""
    lib = _lib.load()
    dev = _lib.require_device(logits, drafts, out)
    if logits.dtype != torch.float32 or logits.dim() != 2:
        raise ValueError("logits must be a 2-D float32 tensor")
    if drafts.dtype != torch.int32:
        raise ValueError("drafts must be int32")
    logits = logits.contiguous()
    drafts = drafts.contiguous()
    L, V = logits.shape
    if out is None:
        out = torch.empty(2 + L, dtype=torch.int32, device=dev)
    ws = _scratch(dev, lib.lq_accept_workspace_bytes(L, V))
    st = lib.lq_greedy_accept(logits.data_ptr(), L, V, drafts.data_ptr(), drafts.numel(),
                              out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(st, "lq_greedy_accept")
    return out


class DeviceNgramIndex:
    """:class:`NgramIndex` proposals over a device-resident history (``int32 [capacity]``)."""

    def __init__(self, g, device, capacity=1 << 16):
        self.g = g
        self.device = torch.device(device)
        self.hist = torch.empty(capacity, dtype=torch.int32, device=self.device)
        self.length = 0

    @property
    def ids(self):
        return self.hist[:self.length].tolist()

    def extend(self, tokens):
        if torch.is_tensor(tokens):
            t = tokens.to(device=self.device, dtype=torch.int32).reshape(-1)
        else:
            t = torch.tensor([int(x) for x in tokens], dtype=torch.int32, device=self.device)
        k = t.numel()
        if self.length + k > self.hist.numel():
            cap = max(2 * self.hist.numel(), self.length + k)
            h = torch.empty(cap, dtype=torch.int32, device=self.device)
            h[:self.length] = self.hist[:self.length]
            self.hist = h
        self.hist[self.length:self.length + k] = t
        self.length += k

    def propose(self, n):
        r = ngram_propose(self.hist, self.length, self.g, max(1, n)).tolist()
        cnt = min(r[0], n)
        return r[2:2 + cnt]
