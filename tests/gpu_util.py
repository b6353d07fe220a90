"""Helpers shared by the GPU parity tests: seeded inputs, caches quantized on the GPU, the
attention tolerance of the parity bar."""
import numpy as np
import torch

from oracle import quantize as Q

ATOL, RTOL = 2e-3, 1e-2  # attention tolerance (fp32 accumulate, bf16 output)
REF_SMALL_N_ATOL = 2e-2  # reference's fused-vs-unfused tolerance (tests/test_q8_attn.py:31)
TIGHT_TOL_MIN_N = 4096


def unfused_tol(n):
    return (ATOL, RTOL) if n >= TIGHT_TOL_MIN_N else (REF_SMALL_N_ATOL, 0.0)


def to_dev_bf16(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev).to(torch.bfloat16)


def bits16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def special_rows(D=128):
    """Groups that stress the quantizer: zeros, constant, ramps, exact halves, tiny values,
    all-negative, a single outlier."""
    rows = [np.zeros(D), np.full(D, 0.5), np.arange(D) % 64, -(np.arange(D) % 64),
            np.tile(np.r_[0, 255, 0.5, 2.5, np.zeros(60)], D // 64),
            np.tile(np.r_[1.0, -0.3125, np.zeros(62)], D // 64),
            np.full(D, 3e-8) * np.sign(np.arange(D) % 3 - 1),
            -np.abs(np.linspace(0.1, 5, D)),
            np.r_[np.zeros(D - 1), 1000.0]]
    return Q.round_bf16(np.stack(rows).astype(np.float32))


def make_cache(rng, B, Hkv, n, cap, dev, bits=8, D=128, kstd=1.0, vstd=1.0):
    """Random N(0,1) bf16 K/V quantized on the GPU into full-capacity buffers (rows >= n hold
    garbage codes so a kernel that reads past n is caught)."""
    out = []
    for std in (kstd, vstd):
        x = Q.round_bf16(Q.randn_bf16(rng, (B, Hkv, n, D)) * np.float32(std))
        codes = torch.randint(0, 256, (B, Hkv, cap, D * bits // 8), dtype=torch.uint8, device=dev)
        sc = to_dev_bf16(rng.standard_normal((B, Hkv, cap, D // 64)) * 100, dev)
        bi = to_dev_bf16(rng.standard_normal((B, Hkv, cap, D // 64)) * 100, dev)
        from lagunalab_amd.quant import quantize_into
        quantize_into(to_dev_bf16(x, dev), codes, sc, bi, 0, 64, bits)
        out.append((codes, sc, bi))
    return out


def cache_np(c):
    return tuple(t.cpu().numpy() if t.dtype == torch.uint8 else bits16(t) for t in c)


def assert_attn_close(got, want, what="", atol=ATOL, rtol=RTOL):
    got = got.float().cpu().numpy() if torch.is_tensor(got) else got
    err = np.abs(got - want)
    lim = atol + rtol * np.abs(want)
    assert np.all(err <= lim), f"{what} max-abs {err.max():.3e} (worst excess {(err - lim).max():.3e})"
