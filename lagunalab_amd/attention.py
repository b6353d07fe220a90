"""The attention block of a full-attention decoder layer over the quantized cache
(``laguna_mlx/laguna.py:75-111``), MI355X side.

``Attention.__call__`` keeps the reference's protocol: projections, q/k RMSNorm, RoPE at
``cache.offset``, ``update_and_fetch``, then ``cache.attend`` on fused steps, quantized attention
over the returned packed K/V when the cache exposes ``bits`` (a ``quantized_decode`` step, as
mlx-lm's SDPA routes it), SDPA over the returned K/V otherwise, then the softplus output gate and
``o_proj``. The pieces:

* one GEMM for q, k, v and the gate logits (the four projection weights concatenated), one for
  ``o_proj``: ``lq_gemv_bf16`` for a single row (a decode step), hipBLASLt through torch for
  more rows;
* ``lq_qk_norm_rope``: the q and k RMSNorms and the rotary embedding of both in one launch
  (frequencies from :func:`rope_frequencies`: mlx-lm's default or YaRN RoPE, partial rotary);
* the cache: the fused decode / verify kernels, or dequantized K/V for the unfused path;
* ``lq_gate_heads``: softplus gate times the attention output, written in ``o_proj``'s layout.

Activations and weights are bf16, as in the reference's MLX model.
"""
from __future__ import annotations

import math

import torch

from . import _lib


def rope_frequencies(head_dim: int, params: dict):
    """``(inv_freq fp32 [rot_dims / 2], rot_dims, mscale)`` of mlx-lm's ``initialize_rope`` for a
    rope config (``laguna.py:69-72``): ``rope_theta``, ``partial_rotary_factor`` (rotated dims =
    head_dim x factor), ``rope_type`` "default" or "yarn" (``factor``,
    ``original_max_position_embeddings`` 4096, ``beta_fast`` 32, ``beta_slow`` 1, ``mscale`` 1,
    ``mscale_all_dim`` 0). YaRN (Peng et al. 2023, "YaRN: Efficient Context Window Extension of
    Large Language Models"): dims rotating more than ``beta_fast`` times over the original context
    keep their frequency, those rotating fewer than ``beta_slow`` times are divided by ``factor``,
    a linear ramp in between; the rotated dims are scaled by ``0.1 mscale ln(factor) + 1`` over the
    same with ``mscale_all_dim``."""
    dims = int(head_dim * params.get("partial_rotary_factor", 1.0))
    base = float(params["rope_theta"])
    rtype = params.get("rope_type", params.get("type", "default"))
    idx = torch.arange(0, dims, 2, dtype=torch.float64)
    inv_extra = base ** (-idx / dims)
    if rtype == "default":
        return inv_extra.float(), dims, 1.0
    if rtype != "yarn":
        raise ValueError(f"rope_type {rtype!r} is not supported")
    factor = float(params["factor"])
    orig = float(params.get("original_max_position_embeddings", 4096))
    beta_fast = float(params.get("beta_fast", 32))
    beta_slow = float(params.get("beta_slow", 1))

    def corr_dim(rotations):
        return dims * math.log(orig / (rotations * 2 * math.pi)) / (2 * math.log(base))

    low = max(math.floor(corr_dim(beta_fast)), 0)
    high = min(math.ceil(corr_dim(beta_slow)), dims - 1)
    if low == high:
        high += 0.001
    ramp = ((torch.arange(dims // 2, dtype=torch.float64) - low) / (high - low)).clamp(0, 1)
    keep = 1.0 - ramp  # 1: extrapolate (original frequency), 0: interpolate (divided by factor)
    inv = inv_extra * keep + inv_extra / factor * (1.0 - keep)

    def get_mscale(scale, m):
        return 1.0 if scale <= 1 else 0.1 * m * math.log(scale) + 1.0

    mscale = get_mscale(factor, float(params.get("mscale", 1))) / \
        get_mscale(factor, float(params.get("mscale_all_dim", 0)))
    return inv.float(), dims, mscale


def _sdpa(q, k, v, mask, scale):
    """Attention over the returned K/V for steps the fused kernels do not take: float32, GQA by
    grouping query heads, ``mask`` None, "causal" (bottom-right) or a boolean [Lq, Lk] array."""
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qf = q.float().reshape(B, Hkv, G * Lq, D)
    s = torch.matmul(qf, k.float().transpose(-1, -2).contiguous()) * scale
    s = s.reshape(B, Hkv, G, Lq, Lk)
    if isinstance(mask, str):
        mask = torch.arange(Lk)[None, :] <= torch.arange(Lk - Lq, Lk)[:, None]
    if mask is not None:
        s = s.masked_fill(~mask.to(s.device), float("-inf"))
    p = torch.softmax(s, dim=-1).reshape(B, Hkv, G * Lq, Lk)
    return torch.matmul(p, v.float()).reshape(B, Hq, Lq, D).to(q.dtype)


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``x @ w.T`` for bf16 ``x [..., K]`` and ``w [N, K]``: one row (a decode step) runs
    ``lq_gemv_bf16`` (weight-streaming, HBM-bound), more rows the library GEMM."""
    K = x.shape[-1]
    if x.numel() != K:
        return torch.matmul(x, w.t())
    lib = _lib.load()
    dev = _lib.require_device(x, w)
    x = x.contiguous()
    y = torch.empty((*x.shape[:-1], w.shape[0]), dtype=torch.bfloat16, device=dev)
    _lib.check(lib.lq_gemv_bf16(w.data_ptr(), x.data_ptr(), y.data_ptr(), w.shape[0], K,
                                _lib.stream_ptr(dev)), "lq_gemv_bf16")
    return y


class Attention:
    """``laguna_mlx.laguna.Attention`` for a full-attention layer, head_dim 128.

    Weights (bf16, on the GPU): ``wq [Hq*128, C]``, ``wk``/``wv [Hkv*128, C]``, ``wo [C, Hq*128]``,
    ``wg [Hq, C]`` (per-head gate) or ``[Hq*128, C]``, ``q_norm``/``k_norm [128]``."""

    def __init__(self, wq, wk, wv, wo, wg, q_norm, k_norm, n_heads, n_kv_heads, rope: dict,
                 eps: float = 1e-6, head_dim: int = 128):
        if head_dim != 128:
            raise ValueError("head_dim must be 128")
        self.n_heads, self.n_kv_heads, self.head_dim, self.eps = n_heads, n_kv_heads, head_dim, eps
        self.scale = head_dim ** -0.5
        self.per_head_gate = wg.shape[0] == n_heads
        dev = wq.device
        self.w_in = torch.cat([wq, wk, wv, wg], dim=0).to(torch.bfloat16).contiguous()
        self.wo = wo.to(torch.bfloat16).contiguous()
        self.q_norm = q_norm.to(device=dev, dtype=torch.bfloat16).contiguous()
        self.k_norm = k_norm.to(device=dev, dtype=torch.bfloat16).contiguous()
        inv, self.rot_dims, self.mscale = rope_frequencies(head_dim, rope)
        self.inv_freq = inv.to(dev)
        H, Hkv, D = n_heads, n_kv_heads, head_dim
        self._splits = [H * D, Hkv * D, Hkv * D, wg.shape[0]]

    def __call__(self, x: torch.Tensor, mask=None, cache=None) -> torch.Tensor:
        lib = _lib.load()
        dev = _lib.require_device(x)
        B, L, _ = x.shape
        H, Hkv, D = self.n_heads, self.n_kv_heads, self.head_dim
        x = x.to(torch.bfloat16)
        proj = linear(x, self.w_in)  # [B, L, (H + 2 Hkv) D + gate]
        qp, kp, vp, gp = torch.split(proj, self._splits, dim=-1)
        q = qp.reshape(B, L, H, D).transpose(1, 2).contiguous()
        k = kp.reshape(B, L, Hkv, D).transpose(1, 2).contiguous()
        v = vp.reshape(B, L, Hkv, D).transpose(1, 2).contiguous()
        g = gp.contiguous()
        offset = cache.offset if cache is not None else 0
        _lib.check(lib.lq_qk_norm_rope(q.data_ptr(), k.data_ptr(), q.data_ptr(), k.data_ptr(),
                                       self.q_norm.data_ptr(), self.k_norm.data_ptr(), B, H, Hkv,
                                       L, D, self.eps, self.inv_freq.data_ptr(), self.rot_dims,
                                       self.mscale, int(offset), None, _lib.stream_ptr(dev)),
                   "lq_qk_norm_rope")
        if cache is not None:
            k, v = cache.update_and_fetch(k, v)
        if getattr(cache, "fused_step", False):
            out = cache.attend(q, self.scale)
        elif hasattr(cache, "bits"):  # quantized_decode step: packed K/V, quantized attention
            from .q8_attn import quantized_scaled_dot_product_attention
            out = quantized_scaled_dot_product_attention(q, k, v, self.scale, mask,
                                                         cache.group_size, cache.bits)
        else:
            out = _sdpa(q, k, v, mask, self.scale)
        out = out.to(torch.bfloat16).contiguous()
        y = torch.empty((B, L, H, D), dtype=torch.bfloat16, device=dev)
        _lib.check(lib.lq_gate_heads(out.data_ptr(), g.data_ptr(), y.data_ptr(), B, H, L, D,
                                     0 if self.per_head_gate else 1, _lib.stream_ptr(dev)),
                   "lq_gate_heads")
        return linear(y.reshape(B, L, H * D), self.wo)
