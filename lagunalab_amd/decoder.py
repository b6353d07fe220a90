"""One decoded token through the attention blocks of a stack of full-attention layers, eager or as
one HIP graph per token.

Per layer (``laguna_mlx/laguna.py:94-111`` and the decoder layer around it): the residual add of
the previous block's output fused with this layer's input RMSNorm (``lq_add_rms_norm``), then the
attention block (:class:`lagunalab_amd.attention.Attention`: projection GEMM, ``lq_qk_norm_rope``,
the fused decode step over the layer's 8-bit cache, ``lq_gate_heads``, ``o_proj`` GEMM). The MLP /
MoE half of the layer is not part of this path.

A decode step is ~7 launches per layer and the host (Python, ctypes) takes longer to issue them
than the GPU to run them. :meth:`DecodeStack.capture` records the whole step once into a HIP graph
(``torch.cuda.CUDAGraph``) whose launches read the token position from device memory: the RoPE
offsets and the fused decode step's append row (``lq_q8_decode_append_attn_pos``) come from one
int32 counter that the graph's last launch increments, so each replay decodes the next token. The
caches' buffers are reserved for the replays beforehand (a replay never grows them) and their host
offsets advance after each replay.
"""
from __future__ import annotations

import torch

from . import _lib
from .attention import Attention, linear
from .cache import DequantKVCache


def add_rms_norm(h: torch.Tensor, d: torch.Tensor | None, w: torch.Tensor, eps: float = 1e-6):
    """``h + d`` (bf16, written into ``h``) and RMSNorm of it times ``w`` (new bf16 tensor); rows of
    the last dimension."""
    lib = _lib.load()
    dev = _lib.require_device(h, d, w)
    y = torch.empty_like(h)
    C = h.shape[-1]
    _lib.check(lib.lq_add_rms_norm(h.data_ptr(), d.data_ptr() if d is not None else None,
                                   w.data_ptr(), h.data_ptr(), y.data_ptr(), h.numel() // C, C,
                                   float(eps), _lib.stream_ptr(dev)), "lq_add_rms_norm")
    return y


class DecodeStack:
    """``blocks`` (:class:`Attention`), ``norms`` (input RMSNorm weights, bf16 [C]) and ``caches``
    (``DequantKVCache(fused_decode=True)``, one sequence, equal offsets) of the layers in order."""

    def __init__(self, blocks: list[Attention], norms: list[torch.Tensor],
                 caches: list[DequantKVCache], eps: float = 1e-6):
        if not (len(blocks) == len(norms) == len(caches)):
            raise ValueError("one block, norm and cache per layer")
        for c in caches:
            if not (isinstance(c, DequantKVCache) and c.fused_decode):
                raise ValueError("the layers need fused 8-bit caches")
        self.blocks, self.norms, self.caches, self.eps = blocks, norms, caches, eps
        self.graph = None

    def step(self, x: torch.Tensor) -> torch.Tensor:
        """Eager decode of one token: ``x`` [1, 1, C] bf16, the residual stream in; returns it out."""
        h, d = x.clone(), None
        for blk, wn, c in zip(self.blocks, self.norms, self.caches):
            y = add_rms_norm(h, d, wn, self.eps)
            d = blk(y, None, c)
        return h + d

    # ---- graph path
    def _block_pos(self, blk: Attention, y, cache, ws, n_plan):
        lib = _lib.load()
        dev = y.device
        sp = _lib.stream_ptr(dev)
        H, Hkv, D = blk.n_heads, blk.n_kv_heads, blk.head_dim
        proj = linear(y, blk.w_in)  # [1, 1, (H + 2 Hkv) D + gate]
        q, k, v, g = torch.split(proj, blk._splits, dim=-1)  # contiguous pieces of one row
        _lib.check(lib.lq_qk_norm_rope(q.data_ptr(), k.data_ptr(), q.data_ptr(), k.data_ptr(),
                                       blk.q_norm.data_ptr(), blk.k_norm.data_ptr(), 1, H, Hkv, 1,
                                       D, blk.eps, blk.inv_freq.data_ptr(), blk.rot_dims,
                                       blk.mscale, 0, self.pos.data_ptr(), sp), "lq_qk_norm_rope")
        (kc, ks, kb), (vc, vs, vb) = cache.q.keys, cache.q.values
        cap = kc.shape[2]
        out = torch.empty((1, H, 1, D), dtype=torch.bfloat16, device=dev)
        _lib.check(lib.lq_q8_decode_append_attn_pos(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
            vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), 1, H, Hkv, D, cap, n_plan,
            self.pos.data_ptr(), float(blk.scale), out.data_ptr(), ws.data_ptr(), ws.numel(), sp),
            "lq_q8_decode_append_attn_pos")
        gated = torch.empty((1, 1, H, D), dtype=torch.bfloat16, device=dev)
        _lib.check(lib.lq_gate_heads(out.data_ptr(), g.data_ptr(), gated.data_ptr(), 1, H, 1, D,
                                     0 if blk.per_head_gate else 1, sp), "lq_gate_heads")
        return linear(gated.reshape(1, 1, H * D), blk.wo)

    def _step_pos(self):
        h, d = self.x_in.clone(), None
        for i, (blk, wn, c) in enumerate(zip(self.blocks, self.norms, self.caches)):
            y = add_rms_norm(h, d, wn, self.eps)
            d = self._block_pos(blk, y, c, self.ws[i], self.n_plan)
        self.x_out.copy_(h + d)
        self.pos.add_(1)  # the next replay decodes the next token

    def capture(self, steps: int):
        """Records one decode step into a HIP graph; :meth:`replay` then decodes up to ``steps``
        tokens. Reserves ``steps`` rows in every cache first (without writing them)."""
        lib = _lib.load()
        c0 = self.caches[0]
        n0 = c0.offset
        if any(c.offset != n0 for c in self.caches):
            raise ValueError("the caches must be at one offset")
        dev = c0.q.keys[0].device
        for c in self.caches:  # room for `steps` appends, then back to n0
            c._flush()
            k = torch.empty((1, self.blocks[0].n_kv_heads, steps, 128), dtype=torch.bfloat16,
                            device=dev)
            c.q.reserve(k, k)
            c.q.offset = n0
        self.n_plan, self.steps_left = n0, steps
        self.pos = torch.tensor([n0], dtype=torch.int32, device=dev)
        C = self.norms[0].shape[0]
        self.x_in = torch.zeros((1, 1, C), dtype=torch.bfloat16, device=dev)
        self.x_out = torch.zeros_like(self.x_in)
        self.ws = []
        for blk in self.blocks:
            nb = lib.lq_decode_workspace_bytes(_lib.LQ_KV_Q8, 1, blk.n_heads, blk.n_kv_heads, 128,
                                               n0 + 1, None)
            if nb < 0:
                raise ValueError(lib.lq_last_error().decode())
            self.ws.append(torch.zeros(nb, dtype=torch.uint8, device=dev))  # counters start at 0
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step_pos()
        torch.cuda.synchronize(dev)

    def replay(self, x: torch.Tensor) -> torch.Tensor:
        """Decodes one token with the recorded graph; returns the residual stream out (a view of
        the graph's output buffer, overwritten by the next replay)."""
        if self.graph is None or self.steps_left <= 0:
            raise RuntimeError("capture() first; the reserved steps are used up")
        self.x_in.copy_(x)
        self.graph.replay()
        for c in self.caches:
            c.q.offset += 1
        self.steps_left -= 1
        return self.x_out
