"""Prompt-cache files (``lagunalab_amd/prompt_cache.py``): every cache class's ``state`` and
``meta_state`` survive a save/load round trip bit for bit, and the file follows mlx-lm's
flattened layout (dotted tensor keys, string metadata ``0.<layer>.<j>``, ``1.<key>``,
``2.<layer>``). CPU tensors: the packed tuples are set through ``state``, no kernel runs."""
import numpy as np
import pytest
import torch

from lagunalab_amd import cache as C
from lagunalab_amd.prompt_cache import load_prompt_cache, save_prompt_cache


def _packed(rng, rows, bits=8, H=2):
    codes = torch.from_numpy(rng.integers(0, 256, (1, H, rows, 128 * bits // 8), dtype=np.uint8))
    sc = torch.from_numpy(rng.standard_normal((1, H, rows, 2)).astype(np.float32)).to(torch.bfloat16)
    bi = torch.from_numpy(rng.standard_normal((1, H, rows, 2)).astype(np.float32)).to(torch.bfloat16)
    return codes, sc, bi


def _bf16(rng, rows, H=2):
    return torch.from_numpy(rng.standard_normal((1, H, rows, 128)).astype(np.float32)).to(torch.bfloat16)


def _layers(rng):
    q = C.DequantKVCache(fused_decode=True)
    q.state = (_packed(rng, 300), _packed(rng, 300))
    q4 = C.DequantKVCache(bits=4)
    q4.state = (_packed(rng, 7, bits=4), _packed(rng, 7, bits=4))
    kv = C.KVCache()
    kv.state = (_bf16(rng, 5), _bf16(rng, 5))
    rot = C.RotatingKVCache(max_size=8)
    rot.state = (_bf16(rng, 8), _bf16(rng, 8))
    rot.meta_state = ("8", "40")
    tw = C.TrimmableWindowCache(window=8, slack=4)
    tw.state = (_bf16(rng, 12), _bf16(rng, 12))
    tw.meta_state = ("8", "4", "33")
    qp = C.DequantKVCache(fused_decode=True, fused_prefill=True)
    qp.state = (_packed(rng, 40), _packed(rng, 40))
    return [q, q4, kv, rot, tw, qp, C.DequantKVCache(), C.KVCache()]  # the last two empty


def _same(a, b):
    if a is None or b is None:
        return a is None and b is None
    if isinstance(a, tuple):
        return len(a) == len(b) and all(_same(x, y) for x, y in zip(a, b))
    return a.dtype == b.dtype and torch.equal(a.cpu(), b.cpu())


def test_round_trip_every_cache_class(tmp_path):
    caches = _layers(np.random.default_rng(0))
    f = tmp_path / "prompt.safetensors"
    save_prompt_cache(f, caches, {"model": "laguna-xs", "tokens": "300"})
    got, meta = load_prompt_cache(f, device="cpu", return_metadata=True)
    assert meta == {"model": "laguna-xs", "tokens": "300"}
    assert [type(c) for c in got] == [type(c) for c in caches]
    for a, b in zip(caches, got):
        assert _same(a.state, b.state), type(a).__name__
        assert a.meta_state == b.meta_state, type(a).__name__
    assert got[0].fused_decode and got[0].offset == 300 and got[0].kv_bits == 8
    assert not hasattr(got[0], "bits")  # the routing signal stays off after loading
    assert got[1].kv_bits == 4 and got[1].group_size == 64
    assert got[3].offset == 40 and got[4].offset == 33 and got[4].slack == 4
    assert got[5].fused_prefill and got[5].offset == 40 and not got[0].fused_prefill
    assert got[6].empty() and got[7].empty()


def test_file_layout_follows_mlx_lm(tmp_path):
    from safetensors import safe_open
    caches = _layers(np.random.default_rng(1))
    f = tmp_path / "p.safetensors"
    save_prompt_cache(f, caches)
    with safe_open(str(f), framework="pt") as h:
        keys, meta = set(h.keys()), h.metadata()
    assert {"0.0.0", "0.0.1", "0.0.2", "0.1.0", "0.1.1", "0.1.2", "2.0", "2.1"} <= keys
    assert "5.0.0" in keys and not any(k.startswith("6.") or k.startswith("7.") for k in keys)  # empty caches
    assert meta["2.0"] == "DequantKVCache" and meta["2.2"] == "KVCache"
    assert [meta[f"0.0.{j}"] for j in range(4)] == ["256", "300", "64", "8"]  # step, offset, g, bits
    assert meta["0.3.0"] == "8" and meta["0.3.1"] == "40"


def test_loaded_quantized_cache_keeps_growing(tmp_path):
    """A loaded cache's buffers hold exactly the saved rows; the next append reserves past them
    in 256-row steps (mlx-lm's growth), keeping the saved rows."""
    rng = np.random.default_rng(2)
    q = C.QuantizedKVCache()
    q.state = (_packed(rng, 300), _packed(rng, 300))
    f = tmp_path / "q.safetensors"
    save_prompt_cache(f, [q])
    (r,) = load_prompt_cache(f, device="cpu")
    row = r.reserve(torch.zeros(1, 2, 3, 128, dtype=torch.bfloat16),
                    torch.zeros(1, 2, 3, 128, dtype=torch.bfloat16))
    assert row == 300 and r.offset == 303 and r.keys[0].shape[2] == 300 + 256
    assert torch.equal(r.keys[0][:, :, :300], q.keys[0])


def test_meta_state_without_the_prefill_switch_loads(tmp_path):
    """A seven-entry meta_state (no fused_prefill entry) loads with fused_prefill off."""
    c = C.DequantKVCache()
    c.meta_state = ("256", "0", "64", "8", "0", "1", "1")
    assert c.fused_decode and c.fused_verify and not c.fused_prefill
    assert c.meta_state[-1] == "0" and len(c.meta_state) == 8


def test_fused_meta_state_checks_the_format(tmp_path):
    c = C.DequantKVCache(bits=4)
    with pytest.raises(ValueError, match="fused_decode"):
        c.meta_state = ("256", "0", "64", "4", "0", "1", "1")
