"""GPU parity of the attention block around the cache (``lagunalab_amd/attention.py``,
``csrc/layer.hip``) against a float32 torch restatement of ``laguna_mlx/laguna.py:94-111`` with
the reference's bf16 rounding points (norm output, rope output, gate, gated output).

* ``lq_qk_norm_rope`` and ``lq_gate_heads``: within one bf16 rounding step of the restatement
  (the two sides' rsqrt / sin / cos / exp / log1p may differ in the last fp32 bit).
* The whole block over a quantized cache: prefill through the unfused path, decode steps and a
  verify block through the fused kernels, against the restatement over the same cache with the
  unfused path throughout; the gap is the fused-vs-unfused attention difference carried through
  the gate and o_proj.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

BF16_ULP = 2.0 ** -7  # relative spacing of bf16 around 1


def _bf16(rng, shape, s=1.0, dev="cuda"):
    return torch.from_numpy((s * rng.standard_normal(shape)).astype(np.float32)).to(dev).to(torch.bfloat16)


def ref_norm_rope(x, w, eps, inv, rot, mscale, pos0):
    """x bf16 [B, H, L, D]; pos0: int or int tensor [B]."""
    B, H, L, D = x.shape
    xf = x.float()
    y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(torch.bfloat16).float()
    if rot:
        h = rot // 2
        p0 = torch.as_tensor(pos0, device=x.device).reshape(-1, 1, 1).float()
        pos = (p0 + torch.arange(L, device=x.device).float()[None, :, None]).expand(B, L, 1)
        ang = (pos * inv.to(x.device)[None, None, :])[:, None]  # [B, 1, L, h]
        c, s = ang.cos(), ang.sin()
        a, b = y[..., :h] * mscale, y[..., h:rot] * mscale
        y = torch.cat([a * c - b * s, a * s + b * c, y[..., rot:]], dim=-1)
    return y.to(torch.bfloat16)


def assert_within_ulp(got, want, what):
    g, w = got.float(), want.float()
    bad = (g - w).abs() > BF16_ULP * w.abs() + 1e-30
    assert int(bad.sum()) == 0, f"{what}: {int(bad.sum())} elements beyond one bf16 step, max " \
                                f"{float((g - w).abs().max())}"


@pytest.mark.parametrize("case", ["full", "partial_yarn", "norm_only"])
def test_qk_norm_rope_matches_restatement(dev, case):
    from lagunalab_amd import _lib
    from lagunalab_amd.attention import rope_frequencies
    rng = np.random.default_rng({"full": 1, "partial_yarn": 2, "norm_only": 3}[case])
    if case == "full":
        B, Hq, Hkv, L, rope, offsets = 1, 32, 8, 1, {"rope_theta": 1e4}, 82671
    elif case == "partial_yarn":
        B, Hq, Hkv, L = 2, 48, 8, 5
        rope = {"rope_type": "yarn", "rope_theta": 5e5, "factor": 32.0, "partial_rotary_factor": 0.5,
                "original_max_position_embeddings": 4096}
        offsets = torch.tensor([100, 65536], dtype=torch.int32, device=dev)
    else:
        B, Hq, Hkv, L, rope, offsets = 1, 4, 1, 3, {"rope_theta": 1e4, "partial_rotary_factor": 0.0}, 7
    inv, rot, ms = rope_frequencies(128, rope)
    inv = inv.to(dev)
    q, k = _bf16(rng, (B, Hq, L, 128), 3.0), _bf16(rng, (B, Hkv, L, 128), 0.5)
    wq, wk = _bf16(rng, (128,), 0.2) + 1, _bf16(rng, (128,), 0.2) + 1
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    lib = _lib.load()
    off_t = offsets if torch.is_tensor(offsets) else None
    off_s = 0 if torch.is_tensor(offsets) else offsets
    st = lib.lq_qk_norm_rope(q.data_ptr(), k.data_ptr(), qo.data_ptr(), ko.data_ptr(), wq.data_ptr(),
                             wk.data_ptr(), B, Hq, Hkv, L, 128, 1e-6,
                             inv.data_ptr() if rot else None, rot, ms, off_s,
                             off_t.data_ptr() if off_t is not None else None,
                             _lib.stream_ptr(dev))
    _lib.check(st, "lq_qk_norm_rope")
    pos0 = offsets if torch.is_tensor(offsets) else offsets
    assert_within_ulp(qo, ref_norm_rope(q, wq, 1e-6, inv, rot, ms, pos0), f"q {case}")
    assert_within_ulp(ko, ref_norm_rope(k, wk, 1e-6, inv, rot, ms, pos0), f"k {case}")
    # in place gives the same bytes
    q2, k2 = q.clone(), k.clone()
    _lib.check(lib.lq_qk_norm_rope(q2.data_ptr(), k2.data_ptr(), q2.data_ptr(), k2.data_ptr(),
                                   wq.data_ptr(), wk.data_ptr(), B, Hq, Hkv, L, 128, 1e-6,
                                   inv.data_ptr() if rot else None, rot, ms, off_s,
                                   off_t.data_ptr() if off_t is not None else None,
                                   _lib.stream_ptr(dev)), "in place")
    assert torch.equal(q2, qo) and torch.equal(k2, ko)


@pytest.mark.parametrize("per_dim", [0, 1])
def test_gate_heads_matches_restatement(dev, per_dim):
    from lagunalab_amd import _lib
    rng = np.random.default_rng(3 + per_dim)
    B, H, L = 2, 32, 5
    attn = _bf16(rng, (B, H, L, 128))
    g = _bf16(rng, (B, L, H, 128) if per_dim else (B, L, H), 4.0)
    out = torch.empty((B, L, H, 128), dtype=torch.bfloat16, device=dev)
    _lib.check(_lib.load().lq_gate_heads(attn.data_ptr(), g.data_ptr(), out.data_ptr(), B, H, L, 128,
                                         per_dim, _lib.stream_ptr(dev)), "lq_gate_heads")
    gate = torch.nn.functional.softplus(g.float()).to(torch.bfloat16)
    gate = gate if per_dim else gate[..., None]
    want = (attn.transpose(1, 2).float() * gate.float()).to(torch.bfloat16)
    assert_within_ulp(out, want, f"gate per_dim={per_dim}")


class RefBlock:
    """laguna.py:94-111 in torch float32 with bf16 rounding points, unfused attention."""

    def __init__(self, blk, rope):
        from lagunalab_amd.attention import rope_frequencies
        self.b = blk
        self.inv, self.rot, self.ms = rope_frequencies(128, rope)

    def __call__(self, x, mask, cache):
        from lagunalab_amd.attention import _sdpa
        b = self.b
        B, L, _ = x.shape
        H, Hkv, D = b.n_heads, b.n_kv_heads, 128
        wq, wk, wv, wg = torch.split(b.w_in, b._splits, dim=0)
        q = torch.matmul(x, wq.t()).reshape(B, L, H, D).transpose(1, 2).contiguous()
        k = torch.matmul(x, wk.t()).reshape(B, L, Hkv, D).transpose(1, 2).contiguous()
        v = torch.matmul(x, wv.t()).reshape(B, L, Hkv, D).transpose(1, 2).contiguous()
        g = torch.matmul(x, wg.t())
        off = cache.offset
        q = ref_norm_rope(q, b.q_norm, b.eps, self.inv, self.rot, self.ms, off)
        k = ref_norm_rope(k, b.k_norm, b.eps, self.inv, self.rot, self.ms, off)
        k, v = cache.update_and_fetch(k, v)
        out = _sdpa(q, k, v, mask, b.scale).to(torch.bfloat16)
        gate = torch.nn.functional.softplus(g.float()).to(torch.bfloat16)[..., None]
        y = (out.transpose(1, 2).float() * gate.float()).to(torch.bfloat16)
        return torch.matmul(y.reshape(B, L, H * D), b.wo.t())


def test_attention_block_prefill_decode_verify(dev):
    from lagunalab_amd.attention import Attention
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(11)
    C, H, Hkv, D = 512, 8, 2, 128
    rope = {"rope_type": "yarn", "rope_theta": 5e5, "factor": 32.0, "partial_rotary_factor": 0.5,
            "original_max_position_embeddings": 4096}
    w = lambda *s: _bf16(rng, s, 0.05)
    blk = Attention(w(H * D, C), w(Hkv * D, C), w(Hkv * D, C), w(C, H * D), w(H, C),
                    _bf16(rng, (D,), 0.1) + 1, _bf16(rng, (D,), 0.1) + 1, H, Hkv, rope)
    ref = RefBlock(blk, rope)
    fused, plain = DequantKVCache(fused_decode=True), DequantKVCache()
    for L in (300, 1, 1, 1, 5, 1):
        x = _bf16(rng, (1, L, C))
        a = blk(x, fused.make_mask(L), fused)
        want = ref(x, plain.make_mask(L), plain)
        assert fused.fused_step == (L <= 16) and fused.offset == plain.offset
        err = float((a.float() - want.float()).abs().max())
        scale = float(want.float().abs().max())
        assert err <= 2e-2 * scale, (L, err, scale)


@pytest.mark.parametrize("N,K", [(6176, 2048), (2048, 4096), (4608, 4096), (5, 8), (1, 520),
                                 (4099, 64), (300, 8200), (2048, 6144), (129, 7000)])
def test_gemv_matches_float64(dev, N, K):
    """lq_gemv_bf16 against float64 products of the same bf16 values: within the fp32
    accumulation error plus one bf16 rounding of the result."""
    from lagunalab_amd.attention import linear
    rng = np.random.default_rng(N + K)
    w, x = _bf16(rng, (N, K), 0.05), _bf16(rng, (1, 1, K))
    y = linear(x, w)
    want = (w.double() @ x.double().reshape(K)).reshape(1, 1, N)
    bound = BF16_ULP * want.abs() + 1e-5 * (w.double().abs() @ x.double().abs().reshape(K)).reshape(1, 1, N)
    assert y.shape == (1, 1, N) and bool(((y.double() - want).abs() <= bound).all())


@pytest.mark.parametrize("mode,per_dim,H,C", [(1, 0, 8, 512), (1, 0, 32, 2048), (2, 0, 8, 512),
                                              (2, 1, 8, 512), (2, 0, 32, 2048), (2, 1, 32, 4608),
                                              (1, 0, 1, 40), (2, 0, 48, 2048), (2, 1, 56, 1024),
                                              (1, 0, 48, 6144), (1, 0, 8, 3000)])
def test_gemv_fused_matches_restatement(dev, mode, per_dim, H, C):
    """lq_gemv_fused: mode 1 = W (RMSNorm(h) w_norm), mode 2 = W (attn * softplus(gate)) plus the
    residual, each against float64 products of the restatement's bf16 input vector (one fp32
    accumulation and a bf16 rounding or two apart). Widths 2048, 4096 and 6144 (Laguna's 48-head
    o_proj) take the exact-width kernels, the others the bounds-checked ones (up to 2048, 4096,
    8192); one and two rows per wave both occur."""
    from lagunalab_amd import _lib
    rng = np.random.default_rng(50 + mode + per_dim + H + C)
    if mode == 1:
        N, K = 3 * H * 128 + H, C
        x, aux = _bf16(rng, (K,), 2.0), _bf16(rng, (K,), 0.1) + 1
        xf = x.float()
        xin = (xf * torch.rsqrt(xf.pow(2).mean() + 1e-6) * aux.float()).to(torch.bfloat16)
        res = None
    else:
        N, K = C, H * 128
        x = _bf16(rng, (K,))
        aux = _bf16(rng, (K,) if per_dim else (H,), 3.0)
        gate = torch.nn.functional.softplus(aux.float()).to(torch.bfloat16).float()
        gate = gate if per_dim else gate.repeat_interleave(128)
        xin = (x.float() * gate).to(torch.bfloat16)
        res = _bf16(rng, (N,))
    w = _bf16(rng, (N, K), 0.05)
    y = torch.empty(N, dtype=torch.bfloat16, device=dev) if res is None else res.clone()
    _lib.check(_lib.load().lq_gemv_fused(w.data_ptr(), x.data_ptr(), aux.data_ptr(),
                                         y.data_ptr() if res is not None else None, y.data_ptr(),
                                         N, K, mode, 1e-6, per_dim, _lib.stream_ptr(dev)), "fused")
    want = w.double() @ xin.double()
    mag = w.double().abs() @ xin.double().abs()
    if res is not None:
        want = want + res.double()
        mag = mag + res.double().abs()
    assert bool(((y.double() - want).abs() <= 2 * BF16_ULP * mag + 1e-4).all())


@pytest.mark.parametrize("H,Hkv,C,rot,device_pos", [(32, 8, 2048, 64, False), (32, 8, 2048, 128, True),
                                                    (4, 2, 520, 0, False), (48, 8, 2048, 64, True)])
def test_gemv_norm_rope_equals_two_launches(dev, H, Hkv, C, rot, device_pos):
    """lq_gemv_norm_rope = lq_gemv_fused mode 1 followed by lq_qk_norm_rope on the q and k heads,
    bit for bit (the same arithmetic in one launch); a second call with the same counters gives
    the same result (the counters were left at zero)."""
    from lagunalab_amd import _lib
    from lagunalab_amd.attention import rope_frequencies
    lib = _lib.load()
    rng = np.random.default_rng(H + C + rot)
    N = (H + 2 * Hkv) * 128 + H
    w, x = _bf16(rng, (N, C), 0.05), _bf16(rng, (C,), 2.0)
    wn, qn, kn = (_bf16(rng, (n,), 0.1) + 1 for n in (C, 128, 128))
    params = {"rope_theta": 1e6, "partial_rotary_factor": rot / 128}
    inv, rot_dims, mscale = rope_frequencies(128, params) if rot else (torch.ones(1), 0, 1.0)
    inv = inv.to(dev)
    pos = 81234
    offs = torch.tensor([pos], dtype=torch.int32, device=dev) if device_pos else None
    sp = _lib.stream_ptr(dev)
    want = torch.empty(N, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.lq_gemv_fused(w.data_ptr(), x.data_ptr(), wn.data_ptr(), None, want.data_ptr(),
                                 N, C, 1, 1e-6, 0, sp), "fused")
    q, k = want[:H * 128], want[H * 128:(H + Hkv) * 128]
    _lib.check(lib.lq_qk_norm_rope(q.data_ptr(), k.data_ptr(), q.data_ptr(), k.data_ptr(),
                                   qn.data_ptr(), kn.data_ptr(), 1, H, Hkv, 1, 128, 1e-5,
                                   inv.data_ptr(), rot_dims, mscale, pos, None, sp), "rope")
    cnt = torch.zeros(H + Hkv, dtype=torch.int32, device=dev)
    for _ in range(2):
        y = torch.full((N,), 7.0, dtype=torch.bfloat16, device=dev)
        _lib.check(lib.lq_gemv_norm_rope(
            w.data_ptr(), x.data_ptr(), wn.data_ptr(), y.data_ptr(), N, C, 1e-6, qn.data_ptr(),
            kn.data_ptr(), H, Hkv, 1e-5, inv.data_ptr(), rot_dims, mscale,
            0 if device_pos else pos, offs.data_ptr() if device_pos else None, cnt.data_ptr(),
            sp), "gemv_norm_rope")
        torch.cuda.synchronize()
        assert torch.equal(y, want)
        assert int(cnt.abs().sum()) == 0


@pytest.mark.parametrize("G,B,rot,device_pos,n", [(4, 1, 64, True, 3000), (4, 1, 128, False, 3000),
                                                  (2, 2, 0, True, 3000), (4, 2, 64, False, 3000),
                                                  (4, 1, 64, True, 7), (1, 1, 128, False, 70),
                                                  (6, 1, 64, True, 3000), (6, 2, 128, False, 3000),
                                                  (8, 1, 64, True, 70)])
def test_decode_norm_entry_equals_norm_then_decode(dev, G, B, rot, device_pos, n):
    """lq_q8_decode_norm_append_attn (q/k RMSNorm + RoPE inside the attention kernel, or for G > 4
    in a launch of its own before the dense kernel) equals lq_qk_norm_rope followed by the fused
    decode step, bit for bit: output and cache bytes; host append row or device positions,
    partial / full / no rotation, one and two sequences, G = 1, 2, 4, 6 (Laguna's 48q/8kv) and 8,
    and short caches where most waves have no super-tile."""
    from lagunalab_amd import _lib
    from lagunalab_amd.attention import rope_frequencies
    from lagunalab_amd.quant import quantize_kv_into
    lib = _lib.load()
    rng = np.random.default_rng(70 + G + B + rot + n)
    Hkv, cap = 8, 3072
    H = Hkv * G
    k0, v0 = _bf16(rng, (B, Hkv, n, 128)), _bf16(rng, (B, Hkv, n, 128))
    mk = lambda: tuple(torch.zeros(sh, dtype=dt, device=dev) for sh, dt in (
        ((B, Hkv, cap, 128), torch.uint8), ((B, Hkv, cap, 2), torch.bfloat16),
        ((B, Hkv, cap, 2), torch.bfloat16)))
    ka, va = mk(), mk()
    quantize_kv_into(k0, v0, ka, va, 0)
    kb_, vb_ = tuple(t.clone() for t in ka), tuple(t.clone() for t in va)
    params = {"rope_type": "yarn", "rope_theta": 5e5, "factor": 32.0,
              "original_max_position_embeddings": 4096, "partial_rotary_factor": rot / 128}
    inv, rot_dims, mscale = rope_frequencies(128, params) if rot else (torch.ones(1), 0, 1.0)
    inv = inv.to(dev)
    qn, kn = _bf16(rng, (128,), 0.1) + 1, _bf16(rng, (128,), 0.1) + 1
    nb = lib.lq_decode_workspace_bytes(_lib.LQ_KV_Q8, B, H, Hkv, 128, n + 3, None)
    wa = torch.zeros(nb, dtype=torch.uint8, device=dev)
    wb = torch.zeros(nb, dtype=torch.uint8, device=dev)
    sp = _lib.stream_ptr(dev)
    pos = torch.full((B,), n, dtype=torch.int32, device=dev)
    for step in range(3):
        q = _bf16(rng, (B, H, 1, 128), 3.0)
        k1, v1 = _bf16(rng, (B, Hkv, 1, 128), 3.0), _bf16(rng, (B, Hkv, 1, 128))
        # reference: separate norm + rope launch, then the fused decode step
        qr, kr = q.clone(), k1.clone()
        _lib.check(lib.lq_qk_norm_rope(qr.data_ptr(), kr.data_ptr(), qr.data_ptr(), kr.data_ptr(),
                                       qn.data_ptr(), kn.data_ptr(), B, H, Hkv, 1, 128, 1e-6,
                                       inv.data_ptr(), rot_dims, mscale, n + step, None, sp), "rope")
        want = torch.empty((B, H, 1, 128), dtype=torch.bfloat16, device=dev)
        (kc, ks, kb), (vc, vs, vb) = ka, va
        _lib.check(lib.lq_q8_decode_append_attn_pos(
            qr.data_ptr(), kr.data_ptr(), v1.data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
            vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), B, H, Hkv, 128, cap, n + step,
            pos.data_ptr(), 0.09, want.data_ptr(), wa.data_ptr(), wa.numel(), sp), "decode")
        got = torch.empty_like(want)
        (kc, ks, kb), (vc, vs, vb) = kb_, vb_
        _lib.check(lib.lq_q8_decode_norm_append_attn(
            q.data_ptr(), k1.data_ptr(), v1.data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
            vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), B, H, Hkv, 128, cap,
            n if device_pos else n + step, pos.data_ptr() if device_pos else None, qn.data_ptr(),
            kn.data_ptr(), 1e-6, inv.data_ptr(), rot_dims, mscale, 0.09, got.data_ptr(),
            wb.data_ptr(), wb.numel(), sp), "norm decode")
        pos.add_(1)
        torch.cuda.synchronize()
        assert torch.equal(got, want), step
        for x, y in zip(ka + va, kb_ + vb_):
            assert torch.equal(x, y), step


def test_add_rms_norm_matches_restatement(dev):
    from lagunalab_amd.decoder import add_rms_norm
    rng = np.random.default_rng(21)
    for rows, C in ((1, 2048), (3, 512), (2, 8)):
        h, d, w = _bf16(rng, (rows, C)), _bf16(rng, (rows, C)), _bf16(rng, (C,), 0.2) + 1
        h0 = h.clone()
        y = add_rms_norm(h, d, w, 1e-6)
        s = (h0.float() + d.float()).to(torch.bfloat16)
        assert torch.equal(h, s), (rows, C)  # the residual sum, one bf16 rounding
        sf = s.float()
        want = (sf * torch.rsqrt(sf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()).to(torch.bfloat16)
        assert_within_ulp(y, want, f"rms {rows}x{C}")
        y2 = add_rms_norm(s.clone(), None, w, 1e-6)  # no residual
        assert torch.equal(y2, y)


def _stack(dev, seed, n0, layers=3, C=512, H=8, Hkv=2):
    from lagunalab_amd.decoder import DecodeStack
    return DecodeStack(*_layers(dev, seed, n0, layers, C, H, Hkv))


def _layers(dev, seed, n0, layers=3, C=512, H=8, Hkv=2, fused=True):
    """Blocks, input-norm weights and caches (n0 random prefill rows) of a layer stack; the same
    seed gives the same weights and cache rows."""
    from lagunalab_amd.attention import Attention
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(seed)
    rope = {"rope_type": "yarn", "rope_theta": 5e5, "factor": 32.0, "partial_rotary_factor": 0.5,
            "original_max_position_embeddings": 4096}
    w = lambda *s: _bf16(rng, s, 0.05)
    blocks, norms, caches = [], [], []
    for _ in range(layers):
        blocks.append(Attention(w(H * 128, C), w(Hkv * 128, C), w(Hkv * 128, C), w(C, H * 128),
                                w(H, C), _bf16(rng, (128,), 0.1) + 1, _bf16(rng, (128,), 0.1) + 1,
                                H, Hkv, rope))
        norms.append(_bf16(rng, (C,), 0.1) + 1)
        c = DequantKVCache(fused_decode=fused)
        c.q.update_and_fetch(_bf16(rng, (1, Hkv, n0, 128)), _bf16(rng, (1, Hkv, n0, 128)))
        caches.append(c)
    return blocks, norms, caches


@pytest.mark.parametrize("C,H,Hkv", [(512, 8, 2), (2048, 32, 8), (2048, 48, 8)])
def test_stack_step_matches_restatement(dev, C, H, Hkv):
    """DecodeStack.step (three fused launches per layer) against the float32 restatement of
    each layer: h + o_proj(block(RMSNorm(h) w_norm)) with the reference's bf16 rounding points and
    unfused attention over an unfused cache of the same rows; four tokens through three layers.
    The gap allowed is the fused-vs-unfused attention difference carried through o_proj, plus a
    bf16 rounding of the residual stream per layer."""
    from lagunalab_amd.decoder import DecodeStack
    stack = DecodeStack(*_layers(dev, 61, 4100, 3, C, H, Hkv))
    blocks, norms, caches = _layers(dev, 61, 4100, 3, C, H, Hkv, fused=False)
    rope = {"rope_type": "yarn", "rope_theta": 5e5, "factor": 32.0, "partial_rotary_factor": 0.5,
            "original_max_position_embeddings": 4096}
    refs = [RefBlock(b, rope) for b in blocks]
    rng = np.random.default_rng(62)
    for t in range(4):
        x = _bf16(rng, (1, 1, C))
        got = stack.step(x)
        h = x.clone()
        delta = 0.0
        for ref, wn, c in zip(refs, norms, caches):
            hf = h.float()
            xn = (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-6) * wn.float()).to(torch.bfloat16)
            a = ref(xn, None, c)
            delta = max(delta, float(a.float().abs().max()))
            h = (h.float() + a.float()).to(torch.bfloat16)
        err = (got.float() - h.float()).abs()
        bound = 2e-2 * delta + 3 * BF16_ULP * h.float().abs()
        assert bool((err <= bound).all()), (t, float(err.max()), delta)
        assert all(c.offset == 4101 + t for c in stack.caches)


def test_decode_pos_entry_matches_host_length(dev):
    """lq_q8_decode_append_attn_pos (append row read on the device) equals
    lq_q8_decode_append_attn (host n) bit for bit: output and cache bytes."""
    from lagunalab_amd import _lib
    from lagunalab_amd.q8_attn import decode_append_attention
    from lagunalab_amd.quant import quantize_kv_into
    rng = np.random.default_rng(31)
    n, cap, Hkv = 5000, 5376, 8
    k = _bf16(rng, (1, Hkv, n, 128))
    v = _bf16(rng, (1, Hkv, n, 128))
    mk = lambda: tuple(torch.zeros(s, dtype=dt, device=dev) for s, dt in (
        ((1, Hkv, cap, 128), torch.uint8), ((1, Hkv, cap, 2), torch.bfloat16), ((1, Hkv, cap, 2), torch.bfloat16)))
    ka, va = mk(), mk()
    quantize_kv_into(k, v, ka, va, 0)
    kb_, vb_ = tuple(t.clone() for t in ka), tuple(t.clone() for t in va)
    lib = _lib.load()
    pos = torch.tensor([n], dtype=torch.int32, device=dev)
    nb = lib.lq_decode_workspace_bytes(8, 1, 32, Hkv, 128, n + 1, None)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    for step in range(3):
        q = _bf16(rng, (1, 32, 1, 128))
        k1, v1 = _bf16(rng, (1, Hkv, 1, 128)), _bf16(rng, (1, Hkv, 1, 128))
        want = decode_append_attention(q, k1, v1, ka, va, n=n + step, scale=0.09)
        got = torch.empty_like(want)
        (kc, ks, kb), (vc, vs, vb) = kb_, vb_
        _lib.check(lib.lq_q8_decode_append_attn_pos(
            q.data_ptr(), k1.data_ptr(), v1.data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
            vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), 1, 32, Hkv, 128, cap, n, pos.data_ptr(),
            0.09, got.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev)), "pos entry")
        pos.add_(1)
        assert torch.equal(got, want), step
        for x, y in zip(ka + va, kb_ + vb_):
            assert torch.equal(x, y), step


@pytest.mark.parametrize("H,Hkv", [(8, 2), (12, 2)])
def test_graph_step_matches_eager(dev, H, Hkv):
    """The decode step recorded in a HIP graph (positions on the device) gives the eager step's
    residual stream bit for bit on every replay, with eager GPU work and synchronizations between
    the replays, and leaves the caches with the same bytes; G = 4 (packed kernel) and G = 6 (norm
    launch + dense kernel + merge launch)."""
    a, b = _stack(dev, 41, 4200, H=H, Hkv=Hkv), _stack(dev, 41, 4200, H=H, Hkv=Hkv)
    b.capture(steps=6)
    rng = np.random.default_rng(42)
    for t in range(6):
        x = _bf16(rng, (1, 1, 512))
        want = a.step(x)
        got = b.replay(x).clone()
        assert torch.equal(got, want), t
        torch.matmul(_bf16(rng, (64, 64)), _bf16(rng, (64, 64)))  # unrelated eager work
        torch.cuda.synchronize()
    for ca, cb in zip(a.caches, b.caches):
        assert ca.offset == cb.offset == 4206
        for x, y in zip(ca.state[0] + ca.state[1], cb.state[0] + cb.state[1]):
            assert torch.equal(x, y)
    with pytest.raises(RuntimeError, match="used up"):
        b.replay(x)


def test_graph_replay_refuses_changed_caches(dev):
    """A replay after a cache's buffers moved (an eager step past the reserved rows regrows them)
    or after its offset moved outside the replays raises instead of writing freed memory."""
    s = _stack(dev, 43, 1000)
    s.capture(steps=2)
    rng = np.random.default_rng(44)
    s.replay(_bf16(rng, (1, 1, 512)))
    s.caches[0].q.offset += 1  # an append the graph does not know about
    with pytest.raises(RuntimeError, match="appended to or trimmed"):
        s.replay(_bf16(rng, (1, 1, 512)))
    s.caches[0].q.offset -= 1
    c = s.caches[1]
    k = torch.zeros((1, c.q.keys[0].shape[1], 300, 128), dtype=torch.bfloat16, device=dev)
    c.q.reserve(k, k)  # grows past the capacity reserved at capture: new buffers
    c.q.offset -= 300
    with pytest.raises(RuntimeError, match="buffers changed"):
        s.replay(_bf16(rng, (1, 1, 512)))


@pytest.mark.parametrize("bits", [8, 4])
def test_attention_block_quantized_decode_routes_packed_kv(dev, bits):
    """``quantized_decode``: on single-token steps the cache returns the packed (codes, scales,
    biases) views and exposes ``bits``; the block routes them to the quantized decode kernels (as
    mlx-lm's SDPA routes them on ``hasattr(cache, "bits")``). Against the dequantizing cache's
    block output: within the fused-vs-unfused attention difference carried through the gate and
    o_proj."""
    from lagunalab_amd.attention import Attention
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(12 + bits)
    C, H, Hkv, D = 512, 8, 2, 128
    rope = {"rope_theta": 1e4}
    w = lambda *s: _bf16(rng, s, 0.05)
    blk = Attention(w(H * D, C), w(Hkv * D, C), w(Hkv * D, C), w(C, H * D), w(H, C),
                    _bf16(rng, (D,), 0.1) + 1, _bf16(rng, (D,), 0.1) + 1, H, Hkv, rope)
    qd, plain = DequantKVCache(bits=bits, quantized_decode=True), DequantKVCache(bits=bits)
    for L in (700, 1, 1, 3, 1):
        x = _bf16(rng, (1, L, C))
        a = blk(x, qd.make_mask(L), qd)
        assert hasattr(qd, "bits") == (L == 1)
        want = blk(x, plain.make_mask(L), plain)
        err = float((a.float() - want.float()).abs().max())
        scale = float(want.float().abs().max())
        assert err <= 2e-2 * scale, (L, err, scale)
        if L > 1:
            assert torch.equal(a, want)  # multi-row steps take the dequantize path in both
