"""Pins oracle/attention.py: closed forms, a library routine (torch SDPA in float64), the
bottom-right causal alignment and the flash-decoding split/merge algebra."""
import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import quantize as Q


def test_zero_query_gives_mean_of_values():
    rng = np.random.default_rng(0)
    k = rng.standard_normal((1, 2, 37, 16))
    v = rng.standard_normal((1, 2, 37, 16))
    q = np.zeros((1, 4, 1, 16))
    out = A.sdpa(q, k, v, 0.25)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0].mean(0), atol=1e-12)
    np.testing.assert_allclose(out[0, 3, 0], v[0, 1].mean(0), atol=1e-12)  # head 3 -> kv head 1


def test_single_key_returns_its_value():
    rng = np.random.default_rng(1)
    k = rng.standard_normal((1, 1, 1, 8))
    v = rng.standard_normal((1, 1, 1, 8))
    q = rng.standard_normal((1, 3, 1, 8))
    np.testing.assert_allclose(A.sdpa(q, k, v, 1.0)[0, :, 0], np.repeat(v[0, :, 0], 3, 0))


def test_dominant_key_wins():
    k = np.zeros((1, 1, 5, 4))
    k[0, 0, 2] = [100, 0, 0, 0]
    v = np.arange(20, dtype=float).reshape(1, 1, 5, 4)
    q = np.array([1.0, 0, 0, 0]).reshape(1, 1, 1, 4)
    np.testing.assert_allclose(A.sdpa(q, k, v, 1.0)[0, 0, 0], v[0, 0, 2], atol=1e-12)


@pytest.mark.parametrize("L", [1, 5])
def test_matches_torch_sdpa_float64(L):
    rng = np.random.default_rng(2)
    B, Hq, Hkv, n, D = 2, 8, 2, 29, 16
    q = rng.standard_normal((B, Hq, L, D))
    k = rng.standard_normal((B, Hkv, n, D))
    v = rng.standard_normal((B, Hkv, n, D))
    got = A.sdpa(q, k, v, D ** -0.5, causal=True)
    G = Hq // Hkv
    K = torch.from_numpy(np.repeat(k, G, 1))
    V = torch.from_numpy(np.repeat(v, G, 1))
    mask = None
    if L > 1:  # bottom-right: row i sees keys 0 .. n-L+i
        mask = torch.ones(L, n, dtype=torch.bool).tril(diagonal=n - L)
    want = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q), K, V,
                                                            attn_mask=mask, scale=D ** -0.5)
    np.testing.assert_allclose(got, want.numpy(), atol=1e-12)


def test_causal_last_row_is_decode_and_first_row_skips_block():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 2, 4, 8))
    k = rng.standard_normal((1, 1, 10, 8))
    v = rng.standard_normal((1, 1, 10, 8))
    full = A.sdpa(q, k, v, 0.3, causal=True)
    last = A.sdpa(q[:, :, 3:], k, v, 0.3)
    first = A.sdpa(q[:, :, :1], k[:, :, :7], v[:, :, :7], 0.3)
    np.testing.assert_allclose(full[:, :, 3:], last, atol=1e-12)
    np.testing.assert_allclose(full[:, :, :1], first, atol=1e-12)


@pytest.mark.parametrize("n,block", [(1, 512), (7, 4), (513, 512), (1636, 512), (100, 7)])
def test_block_merge_equals_unsplit(n, block):
    rng = np.random.default_rng(4)
    Hkv, G, D = 2, 3, 128
    k = Q.randn_bf16(rng, (1, Hkv, n + 9, D))
    v = Q.randn_bf16(rng, (1, Hkv, n + 9, D))
    kq = Q.quantize_packed(k, 64, 8)
    vq = Q.quantize_packed(v, 64, 8)
    q = Q.randn_bf16(rng, (1, Hkv * G, 1, D))
    m, l, acc = A.block_partials(q, kq, vq, n, D ** -0.5, block=block)
    merged = A.merge_partials(m, l, acc)
    kf = Q.dequantize_f32(*(t[:, :, :n] for t in kq))
    vf = Q.dequantize_f32(*(t[:, :, :n] for t in vq))
    want = A.sdpa(q, kf, vf, D ** -0.5)
    np.testing.assert_allclose(merged, want, atol=1e-10)


def test_unfused_uses_bf16_dequantized_cache():
    rng = np.random.default_rng(5)
    k = Q.randn_bf16(rng, (1, 1, 40, 128))
    v = Q.randn_bf16(rng, (1, 1, 40, 128))
    kq, vq = Q.quantize_packed(k), Q.quantize_packed(v)
    q = Q.randn_bf16(rng, (1, 2, 1, 128))
    got = A.unfused_attention(q, kq, vq, 33, 128 ** -0.5)
    want = A.sdpa(q, Q.dequantize(*(t[:, :, :33] for t in kq)),
                  Q.dequantize(*(t[:, :, :33] for t in vq)), 128 ** -0.5)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
    # rows beyond n do not matter
    kq2 = tuple(t.copy() for t in kq)
    kq2[0][:, :, 33:] = 255
    np.testing.assert_array_equal(A.unfused_attention(q, kq2, vq, 33, 128 ** -0.5), got)


def test_planted_wrong_head_mapping_is_caught():
    # mapping query head h to kv head h % Hkv (instead of h // G) must change the result
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 4, 1, 8))
    k = rng.standard_normal((1, 2, 9, 8))
    v = rng.standard_normal((1, 2, 9, 8))
    good = A.sdpa(q, k, v, 0.5)
    bad = A.sdpa(q[:, [0, 2, 1, 3]], k, v, 0.5)[:, [0, 2, 1, 3]]
    assert not np.allclose(good, bad)
