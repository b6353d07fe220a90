"""Greedy and prompt-lookup speculative generation on the decode path.

Drop-in for the token loops of ``laguna_mlx/dflash.py``:

* :func:`generate_greedy` -- ``dflash.py:102-112``: prefill, then one token per step, argmax
  (first index on ties). The reference's token oracle.
* :func:`generate_lookup` -- ``dflash.py:170-213``: prompt-lookup speculative decoding whose
  output equals :func:`generate_greedy`. Each step verifies ``[token] + drafts`` in one forward
  pass (a causal block of ``1 + len(drafts)`` rows), accepts the longest draft prefix that equals
  the per-row argmax (``lq_greedy_accept`` on the device), trims the rejected rows from every
  cache and appends the accepted tokens to the n-gram index.

``model(tokens, cache=...)`` takes int64 token ids ``[1, L]`` on the model's device and returns
logits ``[1, L, V]``. :func:`generate_greedy` builds its caches with ``model.make_cache()``
(the reference's ``target.make_cache()``); :func:`generate_lookup` with
``make_trimmable_cache(model, slack=n_draft + 1)`` as the reference does, or with any factory of
trimmable caches passed as ``make_cache`` (e.g. ``make_quantized_cache(model, 8,
fused_decode=True, trim_slack=n_draft + 1)``, whose verify blocks then run on the fused causal
kernel).
"""
from __future__ import annotations

import time

import torch

from .cache import make_trimmable_cache
from .lookup import NgramIndex, greedy_accept


def _ids(tokens, device):
    return torch.tensor([[int(t) for t in tokens]], dtype=torch.int64, device=device)


def generate_greedy(model, prompt, max_tokens, eos=(), cache=None):
    """Greedy decoding (``dflash.py:102-112``). Returns the generated token ids."""
    prompt = [int(t) for t in prompt]
    dev = next(model.parameters()).device
    cache = model.make_cache() if cache is None else cache
    logits = model(_ids(prompt, dev), cache=cache)[0, -1]
    out = []
    while True:
        t = int(torch.argmax(logits.float()))
        out.append(t)
        if t in eos or len(out) >= max_tokens:
            return out
        logits = model(_ids([t], dev), cache=cache)[0, -1]


def generate_lookup(model, prompt, max_tokens, eos=(), g=4, n_draft=7, adaptive=False,
                    prefill_step=2048, make_cache=None):
    """Greedy prompt-lookup speculative decoding (``dflash.py:170-213``); the tokens equal
    :func:`generate_greedy`'s. Returns ``(tokens, stats)``."""
    prompt = [int(t) for t in prompt]
    dev = next(model.parameters()).device
    cache = make_cache() if make_cache else make_trimmable_cache(model, slack=n_draft + 1)
    t0 = time.perf_counter()
    logits = None
    for a in range(0, len(prompt), prefill_step):
        logits = model(_ids(prompt[a:a + prefill_step], dev), cache=cache)[0, -1]
    torch.cuda.synchronize(dev)
    prefill_s = time.perf_counter() - t0
    token = int(torch.argmax(logits.float()))
    index = NgramIndex(g)
    index.extend(prompt + [token])  # the index covers the prompt and the first greedy token
    out, cap = [], n_draft
    stats = {"steps": 0, "drafted": 0, "accepted": 0, "steps_with_draft": 0}
    while True:
        drafts = index.propose(cap)  # [] -> plain one-token step
        logits = model(_ids([token] + drafts, dev), cache=cache)[0]  # [1 + len(drafts), V]
        d = torch.tensor(drafts, dtype=torch.int32, device=dev)
        r = greedy_accept(logits.float(), d).tolist()
        k, nxt = r[0], r[1]
        stats["steps"] += 1
        stats["drafted"] += len(drafts)
        stats["accepted"] += k
        stats["steps_with_draft"] += bool(drafts)
        for t in [token] + drafts[:k]:
            out.append(t)
            if t in eos or len(out) >= max_tokens:
                return out, {**stats, "mean_accepted": stats["accepted"] / stats["steps"],
                             "prefill_s": prefill_s}
        for c in cache:
            c.trim(len(drafts) - k)
        token = nxt
        index.extend(drafts[:k] + [token])
        if adaptive:
            cap = min(n_draft, 1 + k)
