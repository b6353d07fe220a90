"""Host-side generation plumbing on the CPU: the trimmable sliding-window cache
(``tests/test_spec_cache.py:18-38`` of the reference), the rotating window cache under chunked
updates, and the greedy loop over plain bf16 caches. The HIP paths are in test_gpu_model.py."""
import numpy as np
import pytest
import torch

from lagunalab_amd.cache import (KVCache, RotatingKVCache, TrimmableWindowCache,
                                 make_quantized_cache, make_trimmable_cache)
from lagunalab_amd.generate import generate_greedy
from tiny_model import TinyLM


@pytest.fixture(scope="module")
def model():
    return TinyLM(lm_head_scale=1.0, attn_dtype=torch.float32)


def _ids(n, seed=4, vocab=1024):
    return torch.tensor(np.random.default_rng(seed).integers(0, vocab, size=(1, n)))


def _cache(model):
    # slack 4 with window 8, so truncation happens constantly in a 30-token run
    return [TrimmableWindowCache(8, slack=4) if isinstance(c, TrimmableWindowCache) else c
            for c in make_trimmable_cache(model)]


def _chunks(n0=13, n=30):
    return [(0, 5), (5, 12), (12, n0)] + [(i, i + 1) for i in range(n0, n)]


@torch.no_grad()
def test_decode_matches_full_forward_with_truncation(model):
    ids = _ids(30)
    full = model(ids)
    cache = _cache(model)
    outs = [model(ids[:, a:b], cache=cache) for a, b in _chunks()]
    torch.testing.assert_close(torch.cat(outs, dim=1), full, atol=1e-4, rtol=1e-3)
    assert cache[1].keys.shape[2] <= 8 + 4 + 1 and cache[1].offset == 30


@torch.no_grad()
def test_trim_after_window_wrap_forgets_rejected_tokens(model):
    ids = _ids(30)
    full = model(ids)
    cache = _cache(model)
    model(ids[:, :20], cache=cache)
    model(_ids(5, seed=99), cache=cache)  # a rejected draft block
    for c in cache:
        assert c.trim(5) == 5
    out = model(ids[:, 20:], cache=cache)
    torch.testing.assert_close(out, full[:, 20:], atol=1e-4, rtol=1e-3)


def test_trim_is_clamped_to_stored_rows():
    c = TrimmableWindowCache(4, slack=2)
    k = torch.randn(1, 2, 3, 16)
    c.update_and_fetch(k, k)
    assert c.trim(10) == 3 and c.offset == 0 and c.keys.shape[2] == 0
    assert c.trim(1) == 0


@torch.no_grad()
def test_rotating_window_cache_matches_full_forward(model):
    """Sliding layers of the quantized cache keep only the window; chunked prefill followed by
    single-token steps equals the full forward pass."""
    ids = _ids(30, seed=7)
    full = model(ids)
    cache = [RotatingKVCache(8) if lt == "sliding_attention" else KVCache()
             for lt in model.args.layer_types]
    outs = [model(ids[:, a:b], cache=cache) for a, b in [(0, 11), (11, 20), (20, 23)] +
            [(i, i + 1) for i in range(23, 30)]]
    torch.testing.assert_close(torch.cat(outs, dim=1), full, atol=1e-4, rtol=1e-3)


def test_quantized_cache_factory_layout(model):
    cache = make_quantized_cache(model, 8, fused_decode=True)
    kinds = [type(c).__name__ for c in cache]
    assert kinds == ["DequantKVCache", "RotatingKVCache", "DequantKVCache"]
    assert all(c.fused_decode for c in cache if hasattr(c, "fused_decode"))
    cache = make_quantized_cache(model, 8, fused_decode=True, trim_slack=8)
    assert isinstance(cache[1], TrimmableWindowCache) and cache[1].slack == 8
    assert all(c.is_trimmable() for c in cache)


@torch.no_grad()
def test_greedy_plain_cache_equals_recompute(model):
    """The cached greedy loop equals re-running the whole sequence every step."""
    prompt = [int(t) for t in _ids(9, seed=3)[0]]
    got = generate_greedy(model, prompt, 6)
    ids = list(prompt)
    for _ in range(6):
        ids.append(int(torch.argmax(model(torch.tensor([ids]))[0, -1])))
    assert got == ids[len(prompt):]


@torch.no_grad()
def test_greedy_stops_at_eos(model):
    prompt = [int(t) for t in _ids(9, seed=3)[0]]
    free = generate_greedy(model, prompt, 6)
    got = generate_greedy(model, prompt, 6, eos=(free[2],))
    assert got == free[:free.index(free[2]) + 1]
