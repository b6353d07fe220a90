"""Replay quality metric (lagunalab_amd.replay, restating replay/replay.py:23-114 of the
reference) on the CPU: self-score, a closed-form KL, chunking invariance, mismatch errors."""
import numpy as np
import pytest
import torch

from lagunalab_amd import replay as R
from tiny_model import TinyLM


def _session(n=300, seed=0):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, 1024, n)
    mask = np.zeros(n, bool)
    mask[50:120] = True   # two assistant turns
    mask[200:290] = True
    return ids, mask


@pytest.fixture(scope="module")
def tiny():
    return TinyLM(device="cpu", seed=2)


def test_self_score_is_zero(tiny):
    """The reference run scored against itself: KL exactly 0, top-1 agreement 1, and the scored
    positions are those whose next token is an assistant token."""
    ids, mask = _session()
    ref = R.build_ref(tiny, ids, mask, tiny.make_cache, chunk=128)
    want_pos = np.nonzero(mask[1:])[0]
    np.testing.assert_array_equal(ref["pos"], want_pos)
    assert ref["top_ids"].shape == (len(want_pos), 64) and ref["top_lp"].shape == (len(want_pos), 64)
    assert (np.diff(ref["top_lp"], axis=1) <= 0).all()  # largest first
    s = R.score(tiny, ids, mask, tiny.make_cache, ref, chunk=128)
    assert s["kl_top64_mean"] == 0.0 and s["kl_top64_p99"] == 0.0 and s["top1_agree"] == 1.0
    assert s["assistant_tokens"] == len(want_pos) and s["tokens"] == len(ids)


class _Table:
    """forward(x, cache) -> logits rows of a fixed table at the positions of x (a cache-free
    engine: the cache only counts the position)."""

    def __init__(self, table):
        self.table = torch.from_numpy(table)

    def make_cache(self):
        return [0]

    def __call__(self, x, cache):
        a = cache[0]
        cache[0] += x.shape[1]
        return self.table[a:a + x.shape[1]][None]


def test_kl_closed_form():
    """KL(ref || model) over the reference's top 64 ids and the top-1 agreement against a float64
    computation from the two logit tables directly."""
    rng = np.random.default_rng(3)
    n, V = 90, 200
    a = (rng.standard_normal((n, V)) * 3).astype(np.float32)
    b = a + (rng.standard_normal((n, V)) * 0.3).astype(np.float32)
    b[::7] = a[::7]  # some rows identical
    mask = np.zeros(n, bool)
    mask[10:40] = True
    mask[60:] = True
    ids = rng.integers(0, V, n)
    ref = R.build_ref(_Table(a), ids, mask, _Table(a).make_cache, chunk=16)
    tb = _Table(b)
    s = R.score(tb, ids, mask, tb.make_cache, ref, chunk=16, step_from=50)
    pos = np.nonzero(mask[1:])[0]
    la = a[pos].astype(np.float64)
    lb = b[pos].astype(np.float64)
    la -= np.log(np.exp(la - la.max(1, keepdims=True)).sum(1, keepdims=True)) + la.max(1, keepdims=True)
    lb -= np.log(np.exp(lb - lb.max(1, keepdims=True)).sum(1, keepdims=True)) + lb.max(1, keepdims=True)
    top = np.argsort(-la, axis=1)[:, :64]
    ra, rb = np.take_along_axis(la, top, 1), np.take_along_axis(lb, top, 1)
    kl = (np.exp(ra) * (ra - rb)).sum(1)
    assert abs(s["kl_top64_mean"] - kl.mean()) <= 1e-5 * max(1.0, kl.mean())
    assert abs(s["kl_top64_p99"] - np.percentile(kl, 99)) <= 1e-4 * max(1.0, kl.max())
    assert s["top1_agree"] == pytest.approx(float((lb.argmax(1) == top[:, 0]).mean()))


def test_one_token_steps_match_chunks(tiny):
    """Feeding the tail one token per call (the decode path) instead of in chunks changes only
    rounding: the score against the chunked reference stays near zero."""
    ids, mask = _session(seed=1)
    ref = R.build_ref(tiny, ids, mask, tiny.make_cache, chunk=128)
    s = R.score(tiny, ids, mask, tiny.make_cache, ref, chunk=64, step_from=150)
    assert s["kl_top64_mean"] < 1e-4 and s["top1_agree"] >= 0.99


def test_mismatched_reference_raises(tiny):
    ids, mask = _session()
    ref = R.build_ref(tiny, ids, mask, tiny.make_cache, chunk=128)
    other = mask.copy()
    other[150] = True
    with pytest.raises(ValueError, match="position mismatch"):
        R.score(tiny, ids, other, tiny.make_cache, ref, chunk=128)
    with pytest.raises(ValueError, match="one length"):
        R.build_ref(tiny, ids, mask[:-1], tiny.make_cache)
