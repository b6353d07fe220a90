"""Oracle: attention over the quantized KV cache (decode, ragged decode, causal verify).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

What it restates.

* :func:`unfused_attention` -- the reference's correctness oracle and default path: dequantize the
  cache to bf16 (``laguna_mlx/cache.py:99-100``) and run scaled-dot-product attention
  (``laguna_mlx/laguna.py:107``; the kernel test compares against exactly this,
  ``tests/test_q8_attn.py:27-31``). Query head ``h`` reads KV head ``h // G`` with
  ``G = Hq // Hkv`` (``q8_attn.py:31``). With ``L > 1`` query rows the mask is the causal mask
  aligned to the bottom-right: row ``i`` sits at absolute position ``n - L + i`` and sees keys
  ``0 .. n - L + i`` (``laguna.py:183-186``; pinned by ``tests/test_cache.py:23-28``). The math
  runs in float64; the result is returned as fp32 (callers round to bf16 when comparing a bf16
  output).
* :func:`fused_attention` -- the same attention with the fused kernel's dequantization (fp32
  ``scale * code + bias``, no bf16 rounding; ``q8_attn.py:46-55``). The two paths differ by the
  bf16 rounding of K/V: negligible once thousands of keys are averaged, up to ~1e-2 with a handful
  of keys (the reference's own fused-vs-unfused test allows 2e-2, ``tests/test_q8_attn.py:31``).
* :func:`block_partials` / :func:`merge_partials` -- the fused kernel's flash-decoding split:
  per block of keys the running max ``m``, the sum ``l`` of ``exp(s - m)`` and the unnormalised
  ``acc = sum exp(s - m) v`` (``q8_attn.py:44-91``), then the log-sum-exp merge
  (``q8_attn.py:126-130``). Used to pin the split/merge algebra, independent of any kernel.

Parity status: pinned. :func:`unfused_attention` is checked against closed forms (uniform
scores give the mean of V, a single key returns its value row, a dominant key wins) and against
``torch.nn.functional.scaled_dot_product_attention`` in float64; :func:`merge_partials` is
checked against the unsplit softmax for every split size.
"""
from __future__ import annotations

import numpy as np

from .quantize import dequantize, dequantize_f32


def sdpa(q, k, v, scale, causal=False, dtype=np.float64):
    """Textbook attention. q [B,Hq,L,D]; k,v [B,Hkv,n,D]; query head h reads KV head h // G.

    Computed per KV head with its G*L query rows stacked (no K/V expansion). ``dtype`` is the
    arithmetic type (float64 for the oracle, float32 for the timed CPU baseline)."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    B, Hq, L, D = q.shape
    Hkv, n = k.shape[1], k.shape[2]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    G = Hq // Hkv
    qg = q.reshape(B, Hkv, G * L, D)
    s = np.matmul(qg, np.swapaxes(k, -1, -2)) * dtype(scale)
    if causal and L > 1:
        pos = np.arange(n)[None, :]
        row = (n - L + np.arange(G * L) % L)[:, None]
        s = np.where(pos <= row, s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v).reshape(B, Hq, L, D)


def unfused_attention(q, kcache, vcache, n, scale, bits=8, group_size=64, causal=True):
    """Dequantize-to-bf16 + SDPA over the first ``n`` rows of a full-capacity cache.

    q: fp32 values [B, Hq, L, D]; kcache/vcache: (codes [B,Hkv,cap,Dc] uint8,
    scales [B,Hkv,cap,D/gs] uint16 bf16 bits, biases likewise). Returns fp32 [B,Hq,L,D].
    """
    kc, ks, kb = (a[:, :, :n] for a in kcache)
    vc, vs, vb = (a[:, :, :n] for a in vcache)
    k = dequantize(kc, ks, kb, group_size, bits)
    v = dequantize(vc, vs, vb, group_size, bits)
    return sdpa(q, k, v, scale, causal=causal).astype(np.float32)


def fused_attention(q, kcache, vcache, n, scale, bits=8, group_size=64, causal=True):
    """The reference's fused-kernel arithmetic: K/V dequantized as ``scale * code + bias`` in fp32
    without rounding to bf16 (``q8_attn.py:46-55``), then exact softmax attention (float64).
    Same arguments as :func:`unfused_attention`."""
    kc, ks, kb = (a[:, :, :n] for a in kcache)
    vc, vs, vb = (a[:, :, :n] for a in vcache)
    k = dequantize_f32(kc, ks, kb, group_size, bits)
    v = dequantize_f32(vc, vs, vb, group_size, bits)
    return sdpa(q, k, v, scale, causal=causal).astype(np.float32)


def bf16_attention(q, k, v, n, scale, causal=True):
    """Plain bf16 cache (values already bf16-exact fp32 [B,Hkv,cap,D])."""
    return sdpa(q, k[:, :, :n], v[:, :, :n], scale, causal=causal).astype(np.float32)


def ragged_unfused_attention(q, kcache, vcache, lens, scale, bits=8, group_size=64, fused=False):
    """One call per sequence, as the reference must do (``q8_attn.py:102`` takes one ``n``).

    q [B, Hq, 1, D]; caches [B, Hkv, cap, .]; lens: B valid lengths. ``fused`` selects the
    fp32-dequantize arithmetic of :func:`fused_attention`."""
    fn = fused_attention if fused else unfused_attention
    out = []
    for b, n in enumerate(lens):
        qb = q[b:b + 1]
        kb = tuple(a[b:b + 1] for a in kcache)
        vb = tuple(a[b:b + 1] for a in vcache)
        out.append(fn(qb, kb, vb, int(n), scale, bits, group_size))
    return np.concatenate(out, axis=0)


# ----------------------------------------------------------------------------------------------
# flash-decoding split + merge (restating the fused kernel's algebra)
# ----------------------------------------------------------------------------------------------

def block_partials(q, kcache, vcache, n, scale, block=512, bits=8, group_size=64):
    """Per-block (m, l, acc) of single-token attention with fp32 dequantized K/V.

    Follows ``q8_attn.py``: q pre-scaled (``:117``), K/V dequantized in fp32 (``:46-55``),
    per block the max ``m``, ``l = sum exp(s - m)`` and ``acc = sum exp(s - m) v``.
    Returns m, l [B,Hq,nblk] and acc [B,Hq,nblk,D] in float64."""
    kc, ks, kb = (a[:, :, :n] for a in kcache)
    vc, vs, vb = (a[:, :, :n] for a in vcache)
    k = dequantize_f32(kc, ks, kb, group_size, bits).astype(np.float64)
    v = dequantize_f32(vc, vs, vb, group_size, bits).astype(np.float64)
    B, Hq, L, D = q.shape
    assert L == 1
    Hkv = k.shape[1]
    G = Hq // Hkv
    qs = np.asarray(q, dtype=np.float64).reshape(B, Hkv, G, D) * scale
    s = np.matmul(qs, np.swapaxes(k, -1, -2)).reshape(B, Hq, n)
    nblk = max(1, -(-n // block))
    m = np.full((B, Hq, nblk), -np.inf)
    l = np.zeros((B, Hq, nblk))
    acc = np.zeros((B, Hq, nblk, D))
    for i in range(nblk):
        a, e = i * block, min((i + 1) * block, n)
        if a >= e:
            continue
        sb = s[:, :, a:e]
        m[:, :, i] = sb.max(axis=-1)
        p = np.exp(sb - m[:, :, i:i + 1])
        l[:, :, i] = p.sum(axis=-1)
        acc[:, :, i] = np.matmul(p.reshape(B, Hkv, G, e - a), v[:, :, a:e]).reshape(B, Hq, D)
    return m, l, acc


def merge_partials(m, l, acc):
    """Log-sum-exp merge of block partials (``q8_attn.py:126-130``); empty blocks (m=-inf)
    get weight 0. Returns [B, Hq, 1, D] float64."""
    M = m.max(axis=-1, keepdims=True)
    w = np.where(np.isneginf(m), 0.0, np.exp(m - M))
    out = (w[..., None] * acc).sum(axis=2) / (w * l).sum(axis=-1)[..., None]
    return out[:, :, None, :]
