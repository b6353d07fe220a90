"""Teacher-forced replay quality metric: how far a model served over a given KV cache drifts from a
reference run of the same model, on the positions of a token sequence whose next token is an
assistant token.

Restates ``replay/replay.py:23-50`` (``assistant_logprobs``), ``:63-90`` (the top-64 reference of
``build_ref``) and ``:93-114`` (``score``) in torch, for any engine given as
``forward(ids [1, L] int64, cache) -> logits [1, L, V]`` with a cache factory, which is the
reference's own ``forward`` / ``make_cache`` hook:

* the sequence goes through the model in chunks of ``chunk`` tokens (teacher forcing), and from
  ``step_from`` on one token at a time, so that the scored positions there run the single-token
  decode step (the fused 8-bit decode kernel over a ``fused_decode`` cache);
* at every position p with ``mask[p + 1]`` the log-softmax over the vocabulary (float32);
* the reference keeps, per position, its top-64 token ids (largest first) and their log-probs;
* the score per position is KL(ref || model) over those 64 ids,
  ``sum exp(ref_lp) (ref_lp - model_lp)``, reported as mean and 99th percentile, plus the
  top-1 agreement (the model's argmax equals the reference's first id).

Sessions, tokenizer and captured references of real models are not part of this package: the
caller supplies ``ids`` / ``mask`` and builds the reference with :func:`build_ref` from the run it
trusts (for instance the same model over a plain bf16 cache).
"""
from __future__ import annotations

import time

import numpy as np
import torch

TOPK = 64
SUB = 256  # positions per log-softmax batch


def assistant_logprobs(forward, ids, mask, make_cache, chunk=2048, step_from=None, device=None):
    """Yields (positions int64 [n], logprobs float32 [n, V]) for the positions whose next token is
    an assistant token (``mask[p + 1]``), in order. ``ids``, ``mask``: 1-D sequences of equal
    length. Positions ``>= step_from`` are fed one token per forward call. ``device``: where the
    token ids go (default: that of the first parameter of ``forward``, else the CPU)."""
    ids = np.asarray(ids, dtype=np.int64)
    mask = np.asarray(mask, dtype=bool)
    if ids.shape != mask.shape or ids.ndim != 1:
        raise ValueError("ids and mask must be 1-D sequences of one length")
    target = np.zeros_like(mask)
    target[:-1] = mask[1:]
    n = len(ids)
    step_from = n if step_from is None else max(0, min(int(step_from), n))
    bounds = list(range(0, step_from, chunk)) + list(range(step_from, n))
    bounds = [(a, min(a + chunk, step_from) if a < step_from else a + 1) for a in bounds]
    if device is None:
        params = forward.parameters() if isinstance(forward, torch.nn.Module) else iter(())
        device = next(params, torch.empty(0)).device
    cache = make_cache()
    for a, b in bounds:
        x = torch.from_numpy(ids[None, a:b]).to(device)
        with torch.no_grad():
            logits = forward(x, cache)[0]
        sel = np.nonzero(target[a:b])[0]
        for s in range(0, len(sel), SUB):
            part = sel[s:s + SUB]
            lp = logits[torch.from_numpy(part).to(logits.device)].float()
            yield part + a, torch.log_softmax(lp, dim=-1)


def build_ref(forward, ids, mask, make_cache, chunk=2048, step_from=None, device=None):
    """The reference of :func:`score`: per scored position its top-64 ids (largest log-prob
    first) and their log-probs, as numpy arrays ``pos``, ``top_ids``, ``top_lp``."""
    pos, top_ids, top_lp = [], [], []
    for p, lp in assistant_logprobs(forward, ids, mask, make_cache, chunk, step_from, device):
        vals, idx = torch.topk(lp, TOPK, dim=-1, largest=True, sorted=True)
        pos.append(p)
        top_ids.append(idx.cpu().numpy())
        top_lp.append(vals.cpu().numpy())
    if not pos:
        raise ValueError("no assistant tokens to score")
    return {"pos": np.concatenate(pos), "top_ids": np.concatenate(top_ids),
            "top_lp": np.concatenate(top_lp)}


def score(forward, ids, mask, make_cache, ref, chunk=2048, step_from=None, device=None):
    """KL top-64 (mean, p99) and top-1 agreement of ``forward`` over ``make_cache`` against
    ``ref`` (:func:`build_ref`) on the same ``ids`` / ``mask``."""
    kls, agree, i = [], [], 0
    t0 = time.perf_counter()
    for p, lp in assistant_logprobs(forward, ids, mask, make_cache, chunk, step_from, device):
        k = len(p)
        if not (p == ref["pos"][i:i + k]).all():
            raise ValueError("position mismatch vs reference")
        tid = torch.from_numpy(ref["top_ids"][i:i + k]).to(lp.device)
        rlp = torch.from_numpy(ref["top_lp"][i:i + k]).to(lp.device)
        i += k
        mlp = torch.gather(lp, 1, tid)
        kls.append((rlp.exp() * (rlp - mlp)).sum(dim=-1).cpu().numpy())
        agree.append((lp.argmax(dim=-1) == tid[:, 0]).cpu().numpy())
    dt = time.perf_counter() - t0
    if i != len(ref["pos"]):
        raise ValueError("the reference holds more positions than were scored")
    kl, ag = np.concatenate(kls), np.concatenate(agree)
    return {"tokens": int(len(ids)), "assistant_tokens": int(len(kl)),
            "kl_top64_mean": float(kl.mean()), "kl_top64_p99": float(np.percentile(kl, 99)),
            "top1_agree": float(ag.mean()), "tok_per_s": len(ids) / dt}
