"""One decoded token through the attention blocks of a stack of full-attention layers, eager or as
one HIP graph per token.

Per layer (``laguna_mlx/laguna.py:94-111`` and the decoder layer around it): the layer's input
RMSNorm, the attention block of :class:`lagunalab_amd.attention.Attention` (projections,
q/k RMSNorm + RoPE, the fused decode step over the layer's 8-bit cache, softplus gate, o_proj)
and the residual add, in three launches (:class:`DecodeStack`). The MLP / MoE half of the layer is
not part of this path.

The host (Python, ctypes) takes longer to issue a step's launches than the GPU to run them.
:meth:`DecodeStack.capture` records the whole step once into a HIP graph
(``torch.cuda.CUDAGraph``) whose launches read the token position from device memory: the RoPE
position and the fused decode step's append row (``lq_q8_decode_norm_append_attn``) come from one
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


def _gemv_fused(w, x, aux, res, y, mode, eps, per_dim=0):
    lib = _lib.load()
    dev = x.device
    _lib.check(lib.lq_gemv_fused(w.data_ptr(), x.data_ptr(), aux.data_ptr(),
                                 res.data_ptr() if res is not None else None, y.data_ptr(),
                                 w.shape[0], w.shape[1], mode, float(eps), per_dim,
                                 _lib.stream_ptr(dev)), "lq_gemv_fused")
    return y


class DecodeStack:
    """``blocks`` (:class:`Attention`), ``norms`` (input RMSNorm weights, bf16 [C]) and ``caches``
    (``DequantKVCache(fused_decode=True)``, one sequence, equal offsets) of the layers in order.

    A layer of a step is three launches: the input projection with the layer's input RMSNorm in
    its prologue (``lq_gemv_fused`` mode 1), the fused decode step from the raw q and new K rows
    (``lq_q8_decode_norm_append_attn``: q/k RMSNorm + RoPE in the attention kernel's prologue,
    while its first tiles stream in), and the output projection with the softplus gate in its
    prologue and the residual add in its epilogue (``lq_gemv_fused`` mode 2). :meth:`step` issues them from
    the host; :meth:`capture` records them once into a HIP graph that :meth:`replay` runs per
    token."""

    def __init__(self, blocks: list[Attention], norms: list[torch.Tensor],
                 caches: list[DequantKVCache], eps: float = 1e-6):
        if not (len(blocks) == len(norms) == len(caches)):
            raise ValueError("one block, norm and cache per layer")
        for c in caches:
            if not (isinstance(c, DequantKVCache) and c.fused_decode):
                raise ValueError("the layers need fused 8-bit caches")
        self.blocks, self.norms, self.caches, self.eps = blocks, norms, caches, eps
        self.graph = None
        self.pos = None

    def _layer(self, blk: Attention, wn, cache, h, ws=None, n_plan=None, h_out=None):
        """One layer on the residual stream h [1, 1, C]: the stream out goes to ``h_out`` (h itself,
        updated in place, by default). Host mode (``ws`` None): the cache reserves the row and the
        fused step gets its length from the host; graph mode: positions from ``self.pos``,
        workspace ``ws`` and plan length ``n_plan``."""
        from .q8_attn import _workspace
        lib = _lib.load()
        dev = h.device
        sp = _lib.stream_ptr(dev)
        H, Hkv, D = blk.n_heads, blk.n_kv_heads, blk.head_dim
        proj = torch.empty((1, 1, blk.w_in.shape[0]), dtype=torch.bfloat16, device=dev)
        _gemv_fused(blk.w_in, h, wn, None, proj, 1, self.eps)
        q, k, v, g = torch.split(proj, blk._splits, dim=-1)  # contiguous pieces of one row
        host = ws is None
        if host:  # the cache reserves the row; the kernel writes it
            n_plan = cache.q.reserve(k.view(1, Hkv, 1, D), v.view(1, Hkv, 1, D))
            nb = lib.lq_decode_workspace_bytes(_lib.LQ_KV_Q8, 1, H, Hkv, D, n_plan + 1, None)
            if nb < 0:
                raise ValueError(lib.lq_last_error().decode())
            ws = _workspace(dev, nb)
        (kc, ks, kb), (vc, vs, vb) = cache.q.keys, cache.q.values
        out = torch.empty((1, H, 1, D), dtype=torch.bfloat16, device=dev)
        _lib.check(lib.lq_q8_decode_norm_append_attn(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
            vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), 1, H, Hkv, D, kc.shape[2], int(n_plan),
            None if host else self.pos.data_ptr(), blk.q_norm.data_ptr(), blk.k_norm.data_ptr(),
            float(blk.eps), blk.inv_freq.data_ptr(), blk.rot_dims, float(blk.mscale),
            float(blk.scale), out.data_ptr(), ws.data_ptr(), ws.numel(), sp),
            "lq_q8_decode_norm_append_attn")
        _gemv_fused(blk.wo, out, g, h, h if h_out is None else h_out, 2, self.eps,
                    0 if blk.per_head_gate else 1)

    def step(self, x: torch.Tensor) -> torch.Tensor:
        """Eager decode of one token: ``x`` [1, 1, C] bf16, the residual stream in; returns it out."""
        h = x.to(torch.bfloat16).clone()
        for blk, wn, c in zip(self.blocks, self.norms, self.caches):
            c._flush()
            self._layer(blk, wn, c, h)
        return h

    # ---- graph path
    def _step_pos(self):
        # The first layer reads the input buffer and its output projection writes the residual
        # stream into x_out, which the other layers update in place: no copy of the stream into or
        # out of the graph (each was a copy launch of ~4.7 us of GPU time per token).
        for i, (blk, wn, c) in enumerate(zip(self.blocks, self.norms, self.caches)):
            self._layer(blk, wn, c, self.x_in if i == 0 else self.x_out, self.ws[i], self.n_plan,
                        h_out=self.x_out)
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
        self.n_plan, self.steps_left, self.next_row = n0, steps, n0
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
        self.captured_ptrs = self._buffer_ptrs()
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step_pos()
        torch.cuda.synchronize(dev)

    def _buffer_ptrs(self):
        return [tuple(t.data_ptr() for t in (*c.q.keys, *c.q.values)) for c in self.caches]

    def replay(self, x: torch.Tensor) -> torch.Tensor:
        """Decodes one token with the recorded graph; returns the residual stream out (a view of
        the graph's output buffer, overwritten by the next replay). Raises if any cache's buffers
        are not the ones the graph was recorded with (a cache grown by an eager step or an
        append past the reserved rows, or a reloaded ``state``), or if a cache's offset moved other
        than by replays (its rows would then not be where the graph's device position appends)."""
        if self.graph is None or self.steps_left <= 0:
            raise RuntimeError("capture() first; the reserved steps are used up")
        if self._buffer_ptrs() != self.captured_ptrs:
            # the graph's kernels hold the buffers taken at capture: a cache that grew or was
            # reloaded since would have its rows written to memory it no longer owns
            raise RuntimeError("a cache's buffers changed since capture(): capture() again")
        if any(c._pending is not None or c.q.offset != self.next_row for c in self.caches):
            # the graph appends at its device position, which only replays advance
            raise RuntimeError("a cache was appended to or trimmed since capture(): capture() again")
        self.x_in.copy_(x)
        self.graph.replay()
        for c in self.caches:
            c.q.offset += 1
        self.steps_left -= 1
        self.next_row += 1
        return self.x_out
