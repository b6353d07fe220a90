"""Operand ranges of the MFMA attention kernels. Their operands are fp16 (normal from 2^-14 to
65504) while the reference computes in fp32 (``laguna_mlx/q8_attn.py:117``): the kernels scale q
and the P.V operand (softmax weight times V scale) by powers of two chosen from the data, so
queries far outside fp16's range and V groups with tiny or huge scales keep fp32-level accuracy.

Each case against the fused-arithmetic oracle (fp32 dequantize, float64 softmax) at the parity
bar scaled to the inputs: max-abs 2e-3 x (V std) + rel 1e-2. Peaked scores (large q) make the
output rest on a handful of keys, where a coarse P.V operand shows most.
"""
import numpy as np
import pytest
import torch

from gpu_util import RTOL, assert_attn_close, cache_np, make_cache, to_dev_bf16
from oracle import attention as A
from oracle import quantize as Q

pytestmark = pytest.mark.gpu

# (q std, V std): huge and tiny queries, V groups with tiny and huge scales, peaked softmax
RANGES = [(1e4, 1.0), (2e5, 1.0), (1e-4, 1.0), (1.0, 0.01), (3.0, 0.005), (3.0, 1e-4),
          (1.0, 1e3), (3.0, 1e5), (30.0, 0.02)]


def _case(dev, seed, B, Hkv, n, bits, qstd, vstd, G, L):
    rng = np.random.default_rng(seed)
    cap = (n + 255) // 256 * 256 + 256
    kq, vq = make_cache(rng, B, Hkv, n, cap, dev, bits=bits, vstd=vstd)
    q = Q.round_bf16(Q.randn_bf16(rng, (B, Hkv * G, L, 128)) * np.float32(qstd))
    return kq, vq, q


# (bits, G, B) -> the kernel that runs: one 8-bit sequence of at most 65,536 rows takes the
# dense kernel (attn_dense.hip) whatever G; a batch of 8-bit sequences with G <= 4 takes the
# packed kernel (qattn.hip); the 4-bit cache always takes its packed kernel (attn_q4.hip)
DECODE_KERNELS = {(8, 4, 1): "dense", (8, 1, 1): "dense", (8, 6, 1): "dense",
                  (8, 4, 2): "8-bit packed", (8, 1, 2): "8-bit packed", (4, 4, 1): "4-bit packed"}


@pytest.mark.parametrize("qstd,vstd", RANGES)
@pytest.mark.parametrize("bits,G,B", list(DECODE_KERNELS))
def test_decode_operand_range(dev, qstd, vstd, bits, G, B):
    """Decode on each kernel (DECODE_KERNELS); a batch of two sequences of 9,000 and 7,777 rows
    for the packed 8-bit kernel, each sequence checked."""
    from lagunalab_amd.q8_attn import decode_attention
    n = 9000
    lens = [n, 7777][:B]
    kq, vq, q = _case(dev, int(qstd * 7 + vstd * 13) % 1000 + G + bits + 100 * B, B, 8, n, bits,
                      qstd, vstd, G, 1)
    got = decode_attention(to_dev_bf16(q, dev), kq, vq, lens=lens, scale=128 ** -0.5)
    assert torch.isfinite(got.float()).all()
    for b in range(B):
        sl = slice(b, b + 1)
        want = A.fused_attention(q[sl], cache_np(tuple(t[sl] for t in kq)),
                                 cache_np(tuple(t[sl] for t in vq)), lens[b], 128 ** -0.5,
                                 bits=bits)
        assert_attn_close(got[sl], want, f"{DECODE_KERNELS[bits, G, B]} {bits}-bit G={G} "
                          f"sequence {b} q std {qstd} V std {vstd}", 2e-3 * vstd, RTOL)


@pytest.mark.parametrize("qstd,vstd", RANGES)
def test_verify_operand_range(dev, qstd, vstd):
    """The 5-row causal verify block (dense kernel, 20 rows per KV head)."""
    from lagunalab_amd.q8_attn import q8_verify_attention
    n = 6001
    kq, vq, q = _case(dev, int(qstd * 3 + vstd * 5) % 1000, 1, 8, n, 8, qstd, vstd, 4, 5)
    got = q8_verify_attention(to_dev_bf16(q, dev), kq, vq, n, 128 ** -0.5)
    assert torch.isfinite(got.float()).all()
    want = A.fused_attention(q, cache_np(kq), cache_np(vq), n, 128 ** -0.5, causal=True)
    assert_attn_close(got, want, f"verify q std {qstd} V std {vstd}", 2e-3 * vstd, RTOL)


@pytest.mark.parametrize("B", [1, 2], ids=["dense", "packed"])
def test_v_scales_changing_across_the_cache(dev, B):
    """V groups whose scales jump by 2^10 and 2^20 between 700-row regions of the cache: the P.V
    factor is re-chosen up and down as a wave's super-tiles cross the regions (rescaling what it
    accumulated). The keys of the smallest-scale region get the largest scores, so the output
    rests on the values that are 2^20 below the others. One sequence runs the dense kernel; a
    batch of two (the same cache contents, 12,000 and 10,650 rows) the packed 8-bit kernel."""
    from lagunalab_amd.q8_attn import decode_attention
    from lagunalab_amd.quant import quantize_into
    rng = np.random.default_rng(77)
    n, cap, Hkv, G = 12000, 12288, 8, 4
    lens = [n, 10650][:B]
    region = (np.arange(n) // 700) % 3  # V std 1, 2^-20, 2^-10
    # the G query heads of a KV head: one direction plus a little noise
    q = Q.randn_bf16(rng, (1, Hkv, 1, 1, 128)) * np.float32(4.0)
    q = Q.round_bf16(q + 0.3 * Q.randn_bf16(rng, (1, Hkv, G, 1, 128))).reshape(1, Hkv * G, 1, 128)
    qdir = q[0, ::G, 0] / np.linalg.norm(q[0, ::G, 0], axis=-1, keepdims=True)  # [Hkv, 128]
    shift = np.where(region == 1, 6.0, -6.0).astype(np.float32)
    k = Q.randn_bf16(rng, (1, Hkv, n, 128)) + shift[None, None, :, None] * qdir[None, :, None, :]
    v = Q.randn_bf16(rng, (1, Hkv, n, 128)) * (np.float32(2.0) ** np.array([0, -20, -10])[region]
                                                 ).astype(np.float32)[None, None, :, None]
    caches = []
    for x in (k, v):
        c = (torch.zeros((B, Hkv, cap, 128), dtype=torch.uint8, device=dev),
             torch.zeros((B, Hkv, cap, 2), dtype=torch.bfloat16, device=dev),
             torch.zeros((B, Hkv, cap, 2), dtype=torch.bfloat16, device=dev))
        xb = np.repeat(Q.round_bf16(x), B, axis=0)
        quantize_into(to_dev_bf16(xb, dev), *c, 0, 64, 8)
        caches.append(c)
    qb = np.repeat(q, B, axis=0)
    got = decode_attention(to_dev_bf16(qb, dev), caches[0], caches[1], lens=lens,
                           scale=128 ** -0.5)
    for b in range(B):
        sl = slice(b, b + 1)
        want = A.fused_attention(q, cache_np(tuple(t[sl] for t in caches[0])),
                                 cache_np(tuple(t[sl] for t in caches[1])), lens[b], 128 ** -0.5)
        mag = float(np.abs(want).max())
        assert mag < 2.0 ** -14, mag  # the output is the small-scale region's
        assert_attn_close(got[sl], want, f"V scales jumping by 2^10 and 2^20, sequence {b}",
                          2e-3 * mag, RTOL)
