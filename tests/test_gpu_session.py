"""Parity at the session lengths the benchmarks run, on N(0,1) K/V quantized to the cache (the
reference's synthetic inputs, ``scripts/micro_kv_decode.py:30-40``), against the oracle:

* the fused decode step (``lq_q8_decode_append_attn``, the benchmarked kernel) over 256
  consecutive steps from 82,671 cached rows (n = 82,672 ... 82,927 after each append): every
  appended K/V row bit-exact against the oracle's quantizer, and the outputs of the first, a
  middle and the last step within 2e-3 + 1e-2 of the reference's unfused path (dequantize to
  bf16 + SDPA) over the cache as it stood at that step;
* a ragged batch at the eight lengths of ``default_rng(1).integers(42771, 82672, 8)``: the
  80,695-row sequence against the unfused path, the 44,161-row one against the fused-arithmetic
  oracle;
* the 4-bit decode at 82,671 rows against the unfused 4-bit path;
* Laguna's own 48q/8kv shape (6 query heads per KV head: the dense kernel with the append inside,
  then the merge launch) over 16 consecutive fused steps from 82,671 cached rows, every appended
  row bit-exact and three sampled outputs against the unfused path, and single fused steps at
  8,192 and 32,768 rows (the reference micro-benchmark's other contexts,
  ``scripts/micro_kv_decode.py:19,33``).

Inputs are drawn on the GPU (torch generator, fixed seeds) and copied to the host for the oracle.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_attn_close, cache_np
from oracle import attention as A
from oracle import quantize as Q

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

N0, CAP, STEPS = 82671, 82944, 256
SAMPLES = (0, 131, 255)
SCALE = 128 ** -0.5


def _gpu_cache(dev, g, B, Hkv, n, cap, bits=8):
    """Full-capacity cache whose first n rows (per sequence) are N(0,1) bf16 quantized on the GPU;
    rows past n hold random codes and large scales, so a kernel that reads them is caught."""
    from lagunalab_amd.quant import quantize_into
    out = []
    for _ in range(2):
        codes = torch.randint(0, 256, (B, Hkv, cap, 128 * bits // 8), dtype=torch.uint8,
                              device=dev, generator=g)
        sc = (torch.randn((B, Hkv, cap, 2), device=dev, generator=g) * 100).to(torch.bfloat16)
        bi = (torch.randn((B, Hkv, cap, 2), device=dev, generator=g) * 100).to(torch.bfloat16)
        x = torch.randn((B, Hkv, n, 128), device=dev, generator=g).to(torch.bfloat16)
        quantize_into(x, codes, sc, bi, 0, 64, bits)
        del x
        out.append((codes, sc, bi))
    return out


@pytest.fixture(scope="module")
def c2_session():
    from lagunalab_amd.q8_attn import decode_append_attention
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(2024)
    kq, vq = _gpu_cache(dev, g, 1, 8, N0, CAP)
    knew = torch.randn((STEPS, 1, 8, 1, 128), device=dev, generator=g).to(torch.bfloat16)
    vnew = torch.randn((STEPS, 1, 8, 1, 128), device=dev, generator=g).to(torch.bfloat16)
    qs = torch.randn((STEPS, 1, 32, 1, 128), device=dev, generator=g).to(torch.bfloat16)
    outs = {}
    for j in range(STEPS):
        o = decode_append_attention(qs[j], knew[j], vnew[j], kq, vq, n=N0 + j, scale=SCALE)
        if j in SAMPLES:
            outs[j] = o
    torch.cuda.synchronize()
    return {"k": cache_np(kq), "v": cache_np(vq), "knew": knew.float().cpu().numpy(),
            "vnew": vnew.float().cpu().numpy(), "q": qs.float().cpu().numpy(),
            "out": {j: o.float().cpu().numpy() for j, o in outs.items()}}


def test_fused_steps_append_bit_exact_rows(c2_session):
    s = c2_session
    for name, new in (("k", s["knew"]), ("v", s["vnew"])):
        codes, scales, biases = s[name]
        rows = new[:, 0, :, 0, :].transpose(1, 0, 2)  # [Hkv, STEPS, D]
        wc, ws, wb = Q.quantize_packed(rows, 64, 8)
        np.testing.assert_array_equal(codes[0, :, N0:N0 + STEPS], wc, err_msg=f"{name} codes")
        np.testing.assert_array_equal(scales[0, :, N0:N0 + STEPS], ws, err_msg=f"{name} scales")
        np.testing.assert_array_equal(biases[0, :, N0:N0 + STEPS], wb, err_msg=f"{name} biases")


@pytest.mark.parametrize("j", SAMPLES)
def test_fused_step_output_matches_unfused_oracle(c2_session, j):
    s = c2_session
    n = N0 + j + 1
    want = A.unfused_attention(s["q"][j], s["k"], s["v"], n, SCALE)
    assert_attn_close(s["out"][j], want, f"fused step {j} at n={n}")


def test_ragged_session_lengths_against_oracle(dev):
    from lagunalab_amd.q8_attn import decode_attention
    lens = [int(x) for x in np.random.default_rng(1).integers(42771, 82672, size=8)]
    assert lens[3] == 80695 and lens[4] == 44161
    g = torch.Generator(device=dev).manual_seed(7)
    kq, vq = _gpu_cache(dev, g, 8, 8, max(lens), CAP)
    q = torch.randn((8, 32, 1, 128), device=dev, generator=g).to(torch.bfloat16)
    got = decode_attention(q, kq, vq, lens=lens, scale=SCALE).float().cpu().numpy()
    for b, fn in ((3, A.unfused_attention), (4, A.fused_attention)):
        kb = cache_np(tuple(t[b:b + 1] for t in kq))
        vb = cache_np(tuple(t[b:b + 1] for t in vq))
        want = fn(q[b:b + 1].float().cpu().numpy(), kb, vb, lens[b], SCALE)
        assert_attn_close(got[b:b + 1], want, f"ragged sequence {b} ({lens[b]} rows)")


def test_q4_session_length_against_oracle(dev):
    from lagunalab_amd.q8_attn import decode_attention
    g = torch.Generator(device=dev).manual_seed(8)
    kq, vq = _gpu_cache(dev, g, 1, 8, N0, CAP, bits=4)
    q = torch.randn((1, 32, 1, 128), device=dev, generator=g).to(torch.bfloat16)
    got = decode_attention(q, kq, vq, n=N0, scale=SCALE)
    want = A.unfused_attention(q.float().cpu().numpy(), cache_np(kq), cache_np(vq), N0, SCALE,
                               bits=4)
    assert_attn_close(got, want, "4-bit decode at 82,671 rows")



STEPS48, SAMPLES48 = 16, (0, 7, 15)


def _fused_steps(dev, g, n0, steps, hq, samples):
    """`steps` consecutive fused decode steps of hq query heads over 8 KV heads from n0 cached
    rows; returns the host copies of the final cache, the appended rows, q and sampled outputs."""
    from lagunalab_amd.q8_attn import decode_append_attention
    cap = (n0 + steps + 255) // 256 * 256
    kq, vq = _gpu_cache(dev, g, 1, 8, n0, cap)
    knew = torch.randn((steps, 1, 8, 1, 128), device=dev, generator=g).to(torch.bfloat16)
    vnew = torch.randn((steps, 1, 8, 1, 128), device=dev, generator=g).to(torch.bfloat16)
    qs = torch.randn((steps, 1, hq, 1, 128), device=dev, generator=g).to(torch.bfloat16)
    outs = {}
    for j in range(steps):
        o = decode_append_attention(qs[j], knew[j], vnew[j], kq, vq, n=n0 + j, scale=SCALE)
        if j in samples:
            outs[j] = o
    torch.cuda.synchronize()
    return {"n0": n0, "k": cache_np(kq), "v": cache_np(vq), "knew": knew.float().cpu().numpy(),
            "vnew": vnew.float().cpu().numpy(), "q": qs.float().cpu().numpy(),
            "out": {j: o.float().cpu().numpy() for j, o in outs.items()}}


def _check_appended(s, steps):
    n0 = s["n0"]
    for name, new in (("k", s["knew"]), ("v", s["vnew"])):
        codes, scales, biases = s[name]
        rows = new[:, 0, :, 0, :].transpose(1, 0, 2)  # [Hkv, steps, D]
        wc, ws, wb = Q.quantize_packed(rows, 64, 8)
        np.testing.assert_array_equal(codes[0, :, n0:n0 + steps], wc, err_msg=f"{name} codes")
        np.testing.assert_array_equal(scales[0, :, n0:n0 + steps], ws, err_msg=f"{name} scales")
        np.testing.assert_array_equal(biases[0, :, n0:n0 + steps], wb, err_msg=f"{name} biases")


@pytest.fixture(scope="module")
def laguna_session():
    dev = torch.device("cuda", 0)
    return _fused_steps(dev, torch.Generator(device=dev).manual_seed(4848), N0, STEPS48, 48,
                        SAMPLES48)


def test_laguna_shape_steps_append_bit_exact_rows(laguna_session):
    _check_appended(laguna_session, STEPS48)


@pytest.mark.parametrize("j", SAMPLES48)
def test_laguna_shape_step_output_matches_unfused_oracle(laguna_session, j):
    s = laguna_session
    n = N0 + j + 1
    want = A.unfused_attention(s["q"][j], s["k"], s["v"], n, SCALE)
    assert_attn_close(s["out"][j], want, f"48q/8kv fused step {j} at n={n}")


@pytest.mark.parametrize("n0", [8191, 32767])
def test_laguna_shape_single_step_at_reference_contexts(dev, n0):
    """One 48q/8kv fused step that leaves 8,192 / 32,768 rows in the cache."""
    s = _fused_steps(dev, torch.Generator(device=dev).manual_seed(n0), n0, 1, 48, (0,))
    _check_appended(s, 1)
    want = A.unfused_attention(s["q"][0], s["k"], s["v"], n0 + 1, SCALE)
    assert_attn_close(s["out"][0], want, f"48q/8kv fused step at n={n0 + 1}")
