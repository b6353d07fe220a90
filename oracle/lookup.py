"""Oracle: prompt-lookup n-gram drafting and greedy acceptance.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

What it restates.

* :func:`lookup` -- the brute-force definition the reference tests hold its index to
  (``tests/test_dflash.py:90-98``; the same function in ``scripts/lookup_acceptance.py:64-75``):
  the tokens that followed the most recent *earlier* occurrence of ``ids[t-g:t]`` (start
  ``s <= t - g - 1``), up to ``n`` of them and never past ``t``; ``[]`` when ``t < g`` or there
  is no earlier occurrence.
* :class:`DictIndex` -- the reference's incremental dict index (``laguna_mlx/dflash.py:145-167``):
  ``extend`` indexes the gram starting at ``len(ids) - g - 1`` as the most recent occurrence.
* :func:`propose_scan` -- the same answer as one NumPy backward scan over an int32 history,
  returned in the device result format ``(count, pos, ids)``: ``pos`` is the matched start ``s``
  (``-1`` if none), ``count`` the number of ids returned.
* :func:`greedy_accept` -- ``dflash.py:195-198``: ``pred = argmax`` per verify row (first index
  wins ties, NumPy/torch convention), ``k`` = longest prefix with ``drafts[k] == pred[k]``,
  next token ``pred[k]``.

Parity status: pinned. :func:`lookup` is checked against the reference's hand-traced known
answers (``tests/test_lookup_acceptance.py:7-19``); :class:`DictIndex` and :func:`propose_scan`
against :func:`lookup` exhaustively on the reference's sequences (``tests/test_dflash.py:101-105``);
:func:`greedy_accept` against hand-built cases with ties and every prefix length.
"""
from __future__ import annotations

import numpy as np


def lookup(ids, t, g, n):
    """Brute force: continuation after the latest earlier occurrence of ids[t-g:t]."""
    if t < g:
        return []
    key = tuple(ids[t - g:t])
    for s in range(t - g - 1, -1, -1):
        if tuple(ids[s:s + g]) == key:
            return list(ids[s + g:min(s + g + n, t)])
    return []


class DictIndex:
    """g-gram -> most recent start, built as tokens arrive (``dflash.py:145-167``)."""

    def __init__(self, g):
        self.g, self.ids, self.last = g, [], {}

    def extend(self, tokens):
        for t in tokens:
            self.ids.append(int(t))
            s = len(self.ids) - self.g - 1
            if s >= 0:
                self.last[tuple(self.ids[s:s + self.g])] = s

    def propose(self, n):
        t, g = len(self.ids), self.g
        s = self.last.get(tuple(self.ids[t - g:])) if t >= g else None
        return [] if s is None else self.ids[s + g:min(s + g + n, t)]


def propose_scan(hist, T, g, n):
    """Vectorised backward scan over ``hist[:T]`` (int32). Returns (count, pos, ids list)."""
    h = np.asarray(hist[:T], dtype=np.int64)
    if g < 1 or T < g or T - g - 1 < 0:
        return 0, -1, []
    key = h[T - g:T]
    S = T - g  # candidate starts s in [0, T-g-1]
    ok = np.ones(S, dtype=bool)
    for j in range(g):
        ok &= h[j:j + S] == key[j]
    hits = np.flatnonzero(ok)
    if hits.size == 0:
        return 0, -1, []
    s = int(hits[-1])
    out = h[s + g:min(s + g + n, T)]
    return int(out.size), s, [int(x) for x in out]


def greedy_accept(logits, drafts):
    """logits [L, V] (L >= len(drafts) + 1); drafts: m ids. Returns (k, next_token)."""
    pred = np.argmax(np.asarray(logits), axis=-1)
    k = 0
    while k < len(drafts) and int(drafts[k]) == int(pred[k]):
        k += 1
    return k, int(pred[k])
