"""RoPE frequency tables of the attention block (``lagunalab_amd.attention.rope_frequencies``),
pinned by closed forms of the default and YaRN schedules (mlx-lm's ``initialize_rope`` is not in
this environment; the YaRN schedule follows the published method: frequencies of dims that
rotate more than ``beta_fast`` times over the original context are kept, those rotating fewer
than ``beta_slow`` times are divided by ``factor``, a linear ramp in between)."""
import math

import pytest
import torch

from lagunalab_amd.attention import rope_frequencies


def test_default_rope_is_theta_power():
    inv, dims, ms = rope_frequencies(128, {"rope_theta": 10000.0})
    assert dims == 128 and ms == 1.0 and inv.shape == (64,)
    assert torch.allclose(inv.double(), 10000.0 ** (-torch.arange(0, 128, 2).double() / 128))
    inv, dims, _ = rope_frequencies(128, {"rope_theta": 1e4, "partial_rotary_factor": 0.5})
    assert dims == 64 and inv.shape == (32,)
    assert inv[0] == 1.0 and inv[1].item() == pytest.approx(1e4 ** (-2 / 64), rel=1e-7)  # fp32


def test_yarn_limits_and_mscale():
    p = {"rope_type": "yarn", "rope_theta": 5e5, "factor": 32.0, "partial_rotary_factor": 0.5,
         "original_max_position_embeddings": 4096}
    inv, dims, ms = rope_frequencies(128, p)
    base, _, _ = rope_frequencies(128, {"rope_theta": 5e5, "partial_rotary_factor": 0.5})
    assert dims == 64
    assert ms == pytest.approx(0.1 * math.log(32.0) + 1.0)
    # correction range of the published method, in rotated-pair index
    cd = lambda r: dims * math.log(4096 / (r * 2 * math.pi)) / (2 * math.log(5e5))
    low, high = max(math.floor(cd(32)), 0), min(math.ceil(cd(1)), dims - 1)
    assert 0 < low < high < dims // 2
    assert torch.equal(inv[:low + 1], base[:low + 1])             # fast dims: unchanged
    assert torch.allclose(inv[high:], base[high:] / 32.0)         # slow dims: interpolated
    mid = (low + high) // 2
    t = (mid - low) / (high - low)
    assert inv[mid].item() == pytest.approx(base[mid].item() * ((1 - t) + t / 32.0), rel=1e-6)
    # factor 1: the default table, no scaling
    inv1, _, ms1 = rope_frequencies(128, dict(p, factor=1.0))
    assert torch.allclose(inv1, base) and ms1 == 1.0
    # mscale_all_dim equal to mscale cancels the attention factor
    _, _, ms2 = rope_frequencies(128, dict(p, mscale=0.7, mscale_all_dim=0.7))
    assert ms2 == pytest.approx(1.0)


def test_unknown_rope_type_rejected():
    with pytest.raises(ValueError, match="rope_type"):
        rope_frequencies(128, {"rope_type": "llama3", "rope_theta": 1e4})
