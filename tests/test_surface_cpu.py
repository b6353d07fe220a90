"""Host-side behaviour of the drop-in Python surface that needs no GPU: constructor and factory
errors as in laguna_mlx/cache.py, the q8_decode_attention assertions of q8_attn.py:110-115, the
"no CPU path" rule, mask conventions, and the host NgramIndex against the brute force."""
import types

import numpy as np
import pytest
import torch

from lagunalab_amd import cache as C
from lagunalab_amd import lookup as LK
from lagunalab_amd import q8_attn as QA
from oracle import lookup as O


def test_fused_decode_needs_8bit():
    with pytest.raises(ValueError, match="8-bit"):
        C.DequantKVCache(bits=4, fused_decode=True)
    with pytest.raises(ValueError, match="8-bit"):
        C.DequantKVCache(group_size=32, fused_decode=True)
    C.DequantKVCache(bits=4)  # unfused 4-bit is fine


def _model(head_dim, layer_types=("full_attention", "sliding_attention")):
    return types.SimpleNamespace(args=types.SimpleNamespace(
        head_dim=head_dim, layer_types=list(layer_types), sliding_window=8))


def test_make_quantized_cache_layout_and_head_dim_check():
    cache = C.make_quantized_cache(_model(64), bits=4)
    assert isinstance(cache[0], C.DequantKVCache) and cache[0].kv_bits == 4
    assert cache[0].group_size == 64 and not hasattr(cache[0], "bits")
    assert isinstance(cache[1], C.RotatingKVCache) and cache[1].max_size == 8
    with pytest.raises(ValueError, match="head_dim"):
        C.make_quantized_cache(_model(16), 8)
    with pytest.raises(ValueError, match="8-bit"):
        C.make_quantized_cache(_model(128), 4, fused_decode=True)


def test_q8_decode_attention_assertions():
    kv = (torch.zeros(1, 8, 256, 128, dtype=torch.uint8), torch.zeros(1, 8, 256, 2, dtype=torch.bfloat16),
          torch.zeros(1, 8, 256, 2, dtype=torch.bfloat16))
    with pytest.raises(AssertionError, match="decode only"):
        QA.q8_decode_attention(torch.zeros(1, 32, 2, 128, dtype=torch.bfloat16), kv, kv, 10, 0.1)
    with pytest.raises(AssertionError, match="head_dim"):
        QA.q8_decode_attention(torch.zeros(1, 32, 1, 64, dtype=torch.bfloat16), kv, kv, 10, 0.1)
    kv4 = (torch.zeros(1, 8, 256, 64, dtype=torch.uint8),) + kv[1:]
    with pytest.raises(AssertionError, match="8-bit"):
        QA.q8_decode_attention(torch.zeros(1, 32, 1, 128, dtype=torch.bfloat16), kv4, kv4, 10, 0.1)
    with pytest.raises(AssertionError, match="too many"):
        QA.q8_decode_attention(torch.zeros(1, 136, 1, 128, dtype=torch.bfloat16), kv, kv, 10, 0.1)


def test_no_cpu_path():
    kv = (torch.zeros(1, 8, 256, 128, dtype=torch.uint8), torch.zeros(1, 8, 256, 2, dtype=torch.bfloat16),
          torch.zeros(1, 8, 256, 2, dtype=torch.bfloat16))
    q = torch.zeros(1, 32, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no CPU path"):
        QA.q8_decode_attention(q, kv, kv, 10, 0.1)
    with pytest.raises(ValueError, match="no CPU path"):
        LK.ngram_propose(torch.zeros(10, dtype=torch.int32))


def test_mask_convention():
    assert C.create_attention_mask(1, offset=5) is None
    assert C.create_attention_mask(3, offset=5) == "causal"
    m = C.create_attention_mask(3, offset=5, return_array=True)
    assert m.shape == (3, 8)
    assert m[0].tolist() == [True] * 6 + [False] * 2  # row 0 at position 5 sees keys 0..5


@pytest.mark.parametrize("g", [1, 3, 4])
def test_host_ngram_index_matches_brute_force(g):
    seq = [int(t) for t in np.random.default_rng(1).integers(0, 5, size=300)]
    idx = LK.NgramIndex(g)
    for t in range(len(seq) + 1):
        for n in (1, 7, 15):
            assert idx.propose(n) == O.lookup(seq, t, g, n)
        if t < len(seq):
            idx.extend(seq[t:t + 1])
