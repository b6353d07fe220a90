"""Tiny random decoder for the generation tests: the attention protocol of
``laguna_mlx/laguna.py:94-111`` (q/k RMSNorm, RoPE at ``cache.offset``, ``update_and_fetch``,
``fused_step`` -> ``cache.attend``, ``bits`` -> quantized attention over the packed K/V, else SDPA
with the cache's mask, per-head softplus gate),
full-attention and sliding-window layers, head_dim 128 so that the HIP decode and verify kernels
take the full-attention layers. Weights and the residual stream are float32; the attention
operands (q, k, v after RoPE) and its output are rounded to ``attn_dtype`` (bf16 by default, what
the cache and the kernels take), so the fused and unfused paths see identical operands and differ
only inside attention. Logits are float32; the random ``lm_head`` is scaled as in
``tests/test_dflash.py:23-26`` of the reference.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from lagunalab_amd.cache import make_trimmable_cache


@dataclass
class TinyArgs:
    vocab_size: int = 1024
    hidden_size: int = 256
    intermediate_size: int = 512
    num_attention_heads: int = 8
    num_key_value_heads: int = 2
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    sliding_window: int = 8
    layer_types: list = field(default_factory=lambda: ["full_attention", "sliding_attention",
                                                       "full_attention"])


def _rms(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(x.dtype)


def _rope(x, offset, theta):
    """Non-interleaved rotary embedding on [B, H, L, D] at positions offset .. offset+L-1."""
    D = x.shape[-1]
    inv = theta ** (-torch.arange(0, D, 2, dtype=torch.float32, device=x.device) / D)
    pos = torch.arange(offset, offset + x.shape[2], dtype=torch.float32, device=x.device)
    ang = pos[:, None] * inv[None, :]
    cos, sin = ang.cos(), ang.sin()
    xf = x.float()
    a, b = xf[..., : D // 2], xf[..., D // 2:]
    return torch.cat([a * cos - b * sin, a * sin + b * cos], dim=-1).to(x.dtype)


def sdpa(q, k, v, mask, scale):
    """Float32 attention; ``mask`` is None, "causal" (bottom-right) or a boolean [Lq, Lk] array."""
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qf = q.float().reshape(B, Hkv, G * Lq, D)
    s = torch.matmul(qf, k.float().transpose(-1, -2).contiguous()) * scale
    s = s.reshape(B, Hkv, G, Lq, Lk)
    if isinstance(mask, str):
        mask = (torch.arange(Lk)[None, :] <= torch.arange(Lk - Lq, Lk)[:, None])
    if mask is not None:
        s = s.masked_fill(~mask.to(s.device), float("-inf"))
    p = torch.softmax(s, dim=-1).reshape(B, Hkv, G * Lq, Lk)
    return torch.matmul(p, v.float()).reshape(B, Hq, Lq, D).to(q.dtype)


def _mask(cache, N, window=None):
    if cache is None:
        return None if N == 1 else "causal"
    return cache.make_mask(N, window_size=window)


class TinyLM(torch.nn.Module):
    def __init__(self, args: TinyArgs | None = None, seed=0, dtype=torch.float32, device="cpu",
                 lm_head_scale=50.0, attn_dtype=torch.bfloat16):
        super().__init__()
        self.args = a = args or TinyArgs()
        self.attn_dtype = attn_dtype
        g = torch.Generator().manual_seed(seed)
        H, Hkv, D, C = a.num_attention_heads, a.num_key_value_heads, a.head_dim, a.hidden_size

        def w(*shape, s=0.05):
            return torch.nn.Parameter((s * torch.randn(*shape, generator=g)).to(dtype))

        def norm(n):
            return torch.nn.Parameter((1 + 0.1 * torch.randn(n, generator=g)).to(dtype))

        self.embed = w(a.vocab_size, C, s=1.0)
        self.layers = torch.nn.ModuleList()
        for _ in a.layer_types:
            m = torch.nn.Module()
            m.attn_norm, m.mlp_norm = norm(C), norm(C)
            m.q_proj, m.k_proj, m.v_proj = w(H * D, C), w(Hkv * D, C), w(Hkv * D, C)
            m.o_proj, m.g_proj = w(C, H * D), w(H, C)
            m.q_norm, m.k_norm = norm(D), norm(D)
            m.gate_proj, m.up_proj = w(a.intermediate_size, C), w(a.intermediate_size, C)
            m.down_proj = w(C, a.intermediate_size)
            self.layers.append(m)
        self.norm = norm(C)
        self.lm_head = torch.nn.Parameter((w(a.vocab_size, C).float() * lm_head_scale).to(dtype))
        self.to(device)

    def make_cache(self):
        return make_trimmable_cache(self)

    def _attention(self, m, x, mask, cache):
        a = self.args
        B, L, _ = x.shape
        H, Hkv, D = a.num_attention_heads, a.num_key_value_heads, a.head_dim
        q = _rms((x @ m.q_proj.T).reshape(B, L, H, D), m.q_norm, a.rms_norm_eps).transpose(1, 2)
        k = _rms((x @ m.k_proj.T).reshape(B, L, Hkv, D), m.k_norm, a.rms_norm_eps).transpose(1, 2)
        v = (x @ m.v_proj.T).reshape(B, L, Hkv, D).transpose(1, 2)
        offset = cache.offset if cache is not None else 0
        q, k = _rope(q, offset, a.rope_theta), _rope(k, offset, a.rope_theta)
        ad = self.attn_dtype
        q, k, v = q.to(ad).contiguous(), k.to(ad).contiguous(), v.to(ad).contiguous()
        if cache is not None:
            k, v = cache.update_and_fetch(k, v)
        scale = 1.0 / math.sqrt(D)
        if getattr(cache, "fused_step", False):
            out = cache.attend(q, scale)
        elif hasattr(cache, "bits"):  # quantized_decode step: packed K/V (mlx-lm's SDPA routing)
            from lagunalab_amd.q8_attn import quantized_scaled_dot_product_attention
            out = quantized_scaled_dot_product_attention(q, k, v, scale, mask, cache.group_size,
                                                         cache.bits)
        else:
            out = sdpa(q, k, v, mask, scale)
        out = out.to(x.dtype).transpose(1, 2)  # B, L, H, D
        gate = F.softplus((x @ m.g_proj.T).float()).to(out.dtype)[..., None]
        return (out * gate).reshape(B, L, H * D) @ m.o_proj.T

    def forward(self, ids, cache=None):
        a = self.args
        h = self.embed[ids]
        N = ids.shape[1]
        for i, (m, lt) in enumerate(zip(self.layers, a.layer_types)):
            c = cache[i] if cache is not None else None
            win = a.sliding_window if lt == "sliding_attention" else None
            mask = _mask(c, N, win)
            if c is None and win is not None:
                mask = (torch.arange(N)[None, :] <= torch.arange(N)[:, None]) & \
                       (torch.arange(N)[None, :] > torch.arange(N)[:, None] - win)
            h = h + self._attention(m, _rms(h, m.attn_norm, a.rms_norm_eps), mask, c)
            x = _rms(h, m.mlp_norm, a.rms_norm_eps)
            h = h + (F.silu(x @ m.gate_proj.T) * (x @ m.up_proj.T)) @ m.down_proj.T
        return (_rms(h, self.norm, a.rms_norm_eps) @ self.lm_head.T).float()
