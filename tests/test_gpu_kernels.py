"""GPU parity of liblaguna_hip.so against the CPU oracle, through the Python surface that calls
the C ABI. Bit-exact for codes, scales, biases, dequantized values, draft ids and accept results.

Attention is checked twice: (1) against the fused-kernel arithmetic (fp32 dequantize, as the
reference's Metal kernel does, q8_attn.py:46-55) within max-abs 2e-3 + rel 1e-2 at every size;
(2) against the reference's unfused path (dequantize to bf16, then SDPA) within the same
2e-3 + 1e-2 from 4,096 keys up (the benchmarked context lengths), and within the reference's own
fused-vs-unfused tolerance of 2e-2 (tests/test_q8_attn.py:31) below that, where the bf16 rounding
of a handful of V rows is not averaged away."""
import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import lookup as O
from oracle import quantize as Q
from gpu_util import (ATOL, REF_SMALL_N_ATOL, RTOL, assert_attn_close, bits16, cache_np,  # noqa: F401
                      make_cache, special_rows, to_dev_bf16, unfused_tol)

pytestmark = pytest.mark.gpu

# ---------------------------------------------------------------------------------------------
# quantize / dequantize: bit-exact
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_bit_exact(dev, bits, gs):
    from lagunalab_amd.quant import quantize
    rng = np.random.default_rng(10 + bits + gs)
    x = np.concatenate([Q.randn_bf16(rng, (300, 128)) * np.float32(4), special_rows()])
    c, s, b = quantize(to_dev_bf16(x, dev), gs, bits)
    torch.cuda.synchronize()
    wc, ws, wb = Q.quantize_packed(x, gs, bits)
    np.testing.assert_array_equal(c.cpu().numpy(), wc)
    np.testing.assert_array_equal(bits16(s), ws)
    np.testing.assert_array_equal(bits16(b), wb)


def tie_rows(D, gs, rng, rows=64):
    """Groups whose quotients (x - bias) / scale sit exactly on, or one bf16 step beside, the
    half-integer rounding edges: ends -128 and 127 give scale 1 and bias -128, so x = -128 + k + 0.5
    divides to k + 0.5 exactly (round half away from zero decides the code)."""
    out = np.empty((rows, D), np.float32)
    for r in range(rows):
        g = []
        for _ in range(D // gs):
            v = -128.0 + rng.integers(0, 255, gs).astype(np.float32) + 0.5
            if r % 2:  # neighbours of the edges: one bf16 step up or down
                v = Q.round_bf16(v + np.where(rng.random(gs) < 0.5, -1, 1) * np.abs(v) * 2.0 ** -8)
            v[0], v[1] = -128.0, 127.0
            g.append(v)
        out[r] = np.concatenate(g)
    return Q.round_bf16(out)


@pytest.mark.parametrize("bits,gs,D", [(8, 64, 128), (4, 64, 128), (8, 32, 96), (4, 32, 160),
                                       (8, 128, 256), (4, 128, 128)])
def test_quantize_ties_and_shapes(dev, bits, gs, D):
    """Exact rounding ties and their neighbours, head dims whose 8-value chunks per row are not a
    power of two, and B, H, L, offset that make every index of the row and cache-row arithmetic
    matter: codes, scales and biases bit-exact against the oracle."""
    from lagunalab_amd.quant import quantize_into
    rng = np.random.default_rng(40 + bits + gs + D)
    B, H, L, cap, off = 2, 3, 37, 50, 11
    x = np.concatenate([tie_rows(D, gs, rng, B * H * L // 2),
                        Q.round_bf16(Q.randn_bf16(rng, (B * H * L - B * H * L // 2, D)) * 3)])
    x = x[rng.permutation(len(x))].reshape(B, H, L, D)
    codes = torch.full((B, H, cap, D * bits // 8), 9, dtype=torch.uint8, device=dev)
    sc = torch.full((B, H, cap, D // gs), 1.5, dtype=torch.bfloat16, device=dev)
    bi = torch.full((B, H, cap, D // gs), -2.0, dtype=torch.bfloat16, device=dev)
    quantize_into(to_dev_bf16(x, dev), codes, sc, bi, off, gs, bits)
    wc, ws, wb = Q.quantize_packed(x, gs, bits)
    c = codes.cpu().numpy()
    np.testing.assert_array_equal(c[:, :, off:off + L], wc)
    np.testing.assert_array_equal(bits16(sc)[:, :, off:off + L], ws)
    np.testing.assert_array_equal(bits16(bi)[:, :, off:off + L], wb)
    assert (c[:, :, :off] == 9).all() and (c[:, :, off + L:] == 9).all()


def test_quantize_prefill_size_bit_exact(dev):
    """A prefill-sized append (8 heads x 20,000 rows x 128, K and V in one launch: several
    grid-stride passes per wave) bit-exact against the oracle."""
    from lagunalab_amd.quant import quantize_kv_into
    g = torch.Generator(device=dev).manual_seed(5)
    H, L, cap = 8, 20000, 20224
    k = torch.randn((1, H, L, 128), device=dev, generator=g).to(torch.bfloat16)
    v = (torch.randn((1, H, L, 128), device=dev, generator=g) * 7).to(torch.bfloat16)

    def bufs():
        return (torch.zeros((1, H, cap, 128), dtype=torch.uint8, device=dev),
                torch.zeros((1, H, cap, 2), dtype=torch.bfloat16, device=dev),
                torch.zeros((1, H, cap, 2), dtype=torch.bfloat16, device=dev))
    kq, vq = bufs(), bufs()
    quantize_kv_into(k, v, kq, vq, 0, 64, 8)
    for src, (c, s, b) in ((k, kq), (v, vq)):
        wc, ws, wb = Q.quantize_packed(src.float().cpu().numpy(), 64, 8)
        np.testing.assert_array_equal(c.cpu().numpy()[:, :, :L], wc)
        np.testing.assert_array_equal(bits16(s)[:, :, :L], ws)
        np.testing.assert_array_equal(bits16(b)[:, :, :L], wb)


def test_quantize_append_writes_only_its_rows(dev):
    from lagunalab_amd.quant import quantize_into
    rng = np.random.default_rng(1)
    B, H, cap, L, off = 2, 3, 64, 5, 17
    codes = torch.full((B, H, cap, 128), 7, dtype=torch.uint8, device=dev)
    sc = torch.full((B, H, cap, 2), 1.5, dtype=torch.bfloat16, device=dev)
    bi = torch.full((B, H, cap, 2), -2.0, dtype=torch.bfloat16, device=dev)
    x = Q.randn_bf16(rng, (B, H, L, 128))
    quantize_into(to_dev_bf16(x, dev), codes, sc, bi, off, 64, 8)
    wc, ws, wb = Q.quantize_packed(x, 64, 8)
    c = codes.cpu().numpy()
    np.testing.assert_array_equal(c[:, :, off:off + L], wc)
    np.testing.assert_array_equal(bits16(sc)[:, :, off:off + L], ws)
    np.testing.assert_array_equal(bits16(bi)[:, :, off:off + L], wb)
    assert (c[:, :, :off] == 7).all() and (c[:, :, off + L:] == 7).all()
    assert (sc[:, :, :off] == 1.5).all() and (bi[:, :, off + L:] == -2.0).all()


@pytest.mark.parametrize("bits,gs", [(8, 64), (4, 64), (8, 128)])
def test_quantize_kv_one_launch_equals_two(dev, bits, gs):
    from lagunalab_amd.quant import quantize_into, quantize_kv_into
    rng = np.random.default_rng(3)
    B, H, cap, L, off = 2, 4, 96, 7, 33
    k = to_dev_bf16(Q.randn_bf16(rng, (B, H, L, 128)), dev)
    v = to_dev_bf16(Q.randn_bf16(rng, (B, H, L, 128)), dev)

    def bufs():
        return (torch.full((B, H, cap, 128 * bits // 8), 3, dtype=torch.uint8, device=dev),
                torch.full((B, H, cap, 128 // gs), 0.5, dtype=torch.bfloat16, device=dev),
                torch.full((B, H, cap, 128 // gs), 0.25, dtype=torch.bfloat16, device=dev))
    ka, va, kb_, vb_ = bufs(), bufs(), bufs(), bufs()
    quantize_kv_into(k, v, ka, va, off, gs, bits)
    quantize_into(k, *kb_, off, gs, bits)
    quantize_into(v, *vb_, off, gs, bits)
    for x, y in zip(ka + va, kb_ + vb_):
        assert torch.equal(x, y)
    wc, ws, wb = Q.quantize_packed(v.float().cpu().numpy(), gs, bits)
    np.testing.assert_array_equal(va[0].cpu().numpy()[:, :, off:off + L], wc)
    np.testing.assert_array_equal(bits16(va[1])[:, :, off:off + L], ws)


@pytest.mark.parametrize("bits", [8, 4])
def test_dequantize_bit_exact(dev, bits):
    from lagunalab_amd.quant import dequantize
    rng = np.random.default_rng(2)
    x = Q.randn_bf16(rng, (2, 4, 70, 128))
    wc, ws, wb = Q.quantize_packed(x, 64, bits)
    c = torch.from_numpy(wc).to(dev)
    s = torch.from_numpy(ws.view(np.int16)).to(dev).view(torch.bfloat16)
    b = torch.from_numpy(wb.view(np.int16)).to(dev).view(torch.bfloat16)
    got = dequantize(c, s, b, 64, bits, n=61)
    want = Q.dequantize(wc[:, :, :61], ws[:, :, :61], wb[:, :, :61], 64, bits)
    np.testing.assert_array_equal(got.float().cpu().numpy(), want)


# ---------------------------------------------------------------------------------------------
# fused decode attention
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n,G,B", [(1, 6, 1), (7, 6, 1), (512, 6, 1), (513, 4, 1), (1636, 6, 1),
                                   (4096, 4, 1), (300, 1, 2), (777, 2, 1), (2000, 8, 1),
                                   (1000, 3, 2), (129, 5, 1), (3001, 7, 1)])
def test_decode_matches_unfused_oracle(dev, n, G, B):
    from lagunalab_amd.q8_attn import q8_decode_attention
    rng = np.random.default_rng(n * 10 + G)
    Hkv = 8
    cap = (n + 255) // 256 * 256 + (256 if n % 256 == 0 else 0)
    kq, vq = make_cache(rng, B, Hkv, n, cap, dev)
    q = Q.randn_bf16(rng, (B, Hkv * G, 1, 128))
    scale = 128 ** -0.5
    got = q8_decode_attention(to_dev_bf16(q, dev), kq, vq, n, scale)
    assert got.shape == (B, Hkv * G, 1, 128) and got.dtype == torch.bfloat16
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, scale), f"fused n={n} G={G}")
    at, rt = unfused_tol(n)
    assert_attn_close(got, A.unfused_attention(q, kn, vn, n, scale), f"unfused n={n} G={G}", at, rt)


@pytest.mark.parametrize("n", [65536, 65537])
def test_decode_at_the_dense_packed_boundary(dev, n):
    """One sequence, 32q/8kv: up to 65,536 rows decode runs the dense kernel and a merge launch,
    past it the packed kernel with its merge inside. Both sides of the boundary against the
    oracle, plain and fused (append row n - 1 inside the step)."""
    from lagunalab_amd.q8_attn import decode_append_attention, q8_decode_attention
    rng = np.random.default_rng(n)
    Hkv, G, B = 8, 4, 1
    cap = (n + 256) // 256 * 256
    kq, vq = make_cache(rng, B, Hkv, n, cap, dev)
    q = Q.randn_bf16(rng, (B, Hkv * G, 1, 128))
    got = q8_decode_attention(to_dev_bf16(q, dev), kq, vq, n, 0.09)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, 0.09), f"decode n={n}")
    k1 = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    v1 = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    got = decode_append_attention(to_dev_bf16(q, dev), k1, v1, kq, vq, n=n - 1, scale=0.09)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, 0.09), f"fused step n={n}")


@pytest.mark.parametrize("n", [8500, 11000, 13500])
def test_decode_two_static_super_tiles(dev, n):
    """The packed kernel (two sequences, so that short lengths take it too), 8 KV heads: each
    sequence's 16 workgroups give 64 waves; between about 8.2k and 13.6k keys each wave takes two
    super-tiles statically and its third from the tile counter (its first dynamic one), so the
    counter must be read already for that third super-tile."""
    from lagunalab_amd.q8_attn import decode_append_attention, q8_decode_attention
    rng = np.random.default_rng(n)
    Hkv, G, B = 8, 4, 2
    cap = (n + 256) // 256 * 256
    kq, vq = make_cache(rng, B, Hkv, n, cap, dev)
    q = Q.randn_bf16(rng, (B, Hkv * G, 1, 128))
    got = q8_decode_attention(to_dev_bf16(q, dev), kq, vq, n, 0.09)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, 0.09), f"decode n={n}")
    # the fused step at the same length: append row n - 1, attend over n rows
    k1 = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    v1 = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    got = decode_append_attention(to_dev_bf16(q, dev), k1, v1, kq, vq, n=n - 1, scale=0.09)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, 0.09), f"fused step n={n}")


def test_decode_accepts_mlx_word_view_and_other_q_dtypes(dev):
    from lagunalab_amd.q8_attn import q8_decode_attention
    rng = np.random.default_rng(3)
    kq, vq = make_cache(rng, 1, 8, 700, 768, dev)
    q = Q.randn_bf16(rng, (1, 32, 1, 128))
    a = q8_decode_attention(to_dev_bf16(q, dev), kq, vq, 700, 0.088)
    kw = (kq[0].view(torch.int32),) + kq[1:]
    vw = (vq[0].view(torch.int32),) + vq[1:]
    b = q8_decode_attention(to_dev_bf16(q, dev), kw, vw, 700, 0.088)
    torch.testing.assert_close(a, b, rtol=0, atol=0)
    c = q8_decode_attention(to_dev_bf16(q, dev).float(), kq, vq, 700, 0.088)
    assert c.dtype == torch.float32
    torch.testing.assert_close(c, a.float(), rtol=0, atol=0)


@pytest.mark.slow
def test_decode_full_session_length(dev):
    """Config 2's shape: 82,671 valid rows in an 82,944-row cache, 32q/8kv."""
    from lagunalab_amd.q8_attn import q8_decode_attention
    rng = np.random.default_rng(0)
    n, cap = 82671, 82944
    kq, vq = make_cache(rng, 1, 8, n, cap, dev)
    q = Q.randn_bf16(rng, (1, 32, 1, 128))
    got = q8_decode_attention(to_dev_bf16(q, dev), kq, vq, n, 128 ** -0.5)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.unfused_attention(q, kn, vn, n, 128 ** -0.5), "unfused n=82671")
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, 128 ** -0.5), "fused n=82671")


def test_ragged_matches_per_sequence_oracle(dev):
    from lagunalab_amd.q8_attn import decode_attention
    rng = np.random.default_rng(1)
    lens = [61, 1, 2048, 513, 3000, 256, 1000, 4095]
    B, cap = len(lens), 4096
    kq, vq = make_cache(rng, B, 8, cap, cap, dev)
    q = Q.randn_bf16(rng, (B, 32, 1, 128))
    got = decode_attention(to_dev_bf16(q, dev), kq, vq, lens=lens, scale=128 ** -0.5)
    kn, vn = cache_np(kq), cache_np(vq)
    want = A.ragged_unfused_attention(q, kn, vn, lens, 128 ** -0.5, fused=True)
    assert_attn_close(got, want, "ragged fused")
    want = A.ragged_unfused_attention(q, kn, vn, lens, 128 ** -0.5)
    assert_attn_close(got, want, "ragged unfused", REF_SMALL_N_ATOL, 0.0)


@pytest.mark.parametrize("G", [6, 8, 16])
def test_ragged_dense_kernel_matches_per_sequence_oracle(dev, G):
    """Batches with more than 4 query rows per KV head run the dense kernel: with 6 or 8 rows
    (48q/8kv, 64q/8kv) it merges each sequence's splits in its last workgroup, with 16 rows the
    split merge is a launch of its own. The lengths give sequences of one split up to sixteen
    (at least 256 keys per split), so that the per-sequence merge sees fewer splits than the
    merge's four lanes per dim group as well as many."""
    from lagunalab_amd.q8_attn import decode_attention
    rng = np.random.default_rng(60 + G)
    lens = [130, 1, 4097, 700, 255, 2049]
    B, cap = len(lens), 4352
    kq, vq = make_cache(rng, B, 8, cap, cap, dev)
    q = Q.randn_bf16(rng, (B, 8 * G, 1, 128))
    got = decode_attention(to_dev_bf16(q, dev), kq, vq, lens=lens, scale=128 ** -0.5)
    kn, vn = cache_np(kq), cache_np(vq)
    want = A.ragged_unfused_attention(q, kn, vn, lens, 128 ** -0.5, fused=True)
    assert_attn_close(got, want, f"ragged dense G={G} fused")
    want = A.ragged_unfused_attention(q, kn, vn, lens, 128 ** -0.5)
    assert_attn_close(got, want, f"ragged dense G={G} unfused", REF_SMALL_N_ATOL, 0.0)


def test_ragged_session_lengths_match_single_calls(dev):
    """Config 3's lengths (default_rng(1) in [42771, 82671]): the variable-length call equals one
    call per sequence (size-independent property; per-sequence calls are checked above)."""
    from lagunalab_amd.q8_attn import decode_attention
    lens = [int(x) for x in np.random.default_rng(1).integers(42771, 82672, size=8)]
    cap = 82944
    g = torch.Generator(device=dev).manual_seed(0)
    kq = (torch.randint(0, 256, (8, 8, cap, 128), dtype=torch.uint8, device=dev, generator=g),
          (torch.rand(8, 8, cap, 2, device=dev, generator=g) * 0.03).to(torch.bfloat16),
          (torch.rand(8, 8, cap, 2, device=dev, generator=g) * -3).to(torch.bfloat16))
    vq = (torch.randint(0, 256, (8, 8, cap, 128), dtype=torch.uint8, device=dev, generator=g),
          (torch.rand(8, 8, cap, 2, device=dev, generator=g) * 0.03).to(torch.bfloat16),
          (torch.rand(8, 8, cap, 2, device=dev, generator=g) * -3).to(torch.bfloat16))
    q = torch.randn(8, 32, 1, 128, device=dev, generator=g).to(torch.bfloat16)
    got = decode_attention(q, kq, vq, lens=lens, scale=128 ** -0.5)
    for b, n in enumerate(lens):
        one = decode_attention(q[b:b + 1], tuple(t[b:b + 1] for t in kq),
                               tuple(t[b:b + 1] for t in vq), n=n, scale=128 ** -0.5)
        torch.testing.assert_close(got[b:b + 1].float(), one.float(), atol=1e-3, rtol=1e-2)


def test_attention_workspace_counters_return_to_zero(dev):
    """The kernels that merge their own splits count workgroup arrivals in the workspace's leading
    LQ_WS_ZERO_BYTES bytes; every call must leave them at zero, whatever its shape, so that calls
    of any shape share one workspace. Repeating a call reproduces it bit for bit."""
    from lagunalab_amd import _lib
    from lagunalab_amd import q8_attn as QA
    rng = np.random.default_rng(21)
    for B, n, G, Hkv in [(1, 3000, 4, 8), (2, 700, 2, 4), (3, 129, 1, 16), (1, 5000, 4, 8),
                         (2, 4000, 16, 2)]:
        cap = (n + 255) // 256 * 256
        kq, vq = make_cache(rng, B, Hkv, n, cap, dev)
        q = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv * G, 1, 128)), dev)
        a = QA.decode_attention(q, kq, vq, n=n, scale=0.09)
        b = QA.decode_attention(q, kq, vq, n=n, scale=0.09)
        torch.cuda.synchronize()
        ws = QA._workspaces[(dev, torch.cuda.current_stream(dev).cuda_stream)]
        assert int(ws[:_lib.LQ_WS_ZERO_BYTES].count_nonzero()) == 0, (B, n, G, Hkv)
        assert torch.equal(a, b), (B, n, G, Hkv)
        kn, vn = cache_np(kq), cache_np(vq)
        qn = q.float().cpu().numpy()
        assert_attn_close(a, A.fused_attention(qn, kn, vn, n, 0.09), f"B={B} n={n} G={G}")


# ---------------------------------------------------------------------------------------------
# n-gram propose and greedy accept: bit-exact
# ---------------------------------------------------------------------------------------------

def planted_history(T=82671, seed=0):
    rng = np.random.default_rng(seed)
    h = rng.integers(0, 131072, size=T).astype(np.int32)
    for s in range(0, T - 600, 500):  # copy an 8-gram forward every ~500 tokens
        src = rng.integers(0, max(1, s - 8)) if s > 8 else 0
        h[s:s + 8] = h[src:src + 8]
    h[-3:] = h[T // 2:T // 2 + 3]  # make the final 3-gram occur earlier
    return h


@pytest.mark.parametrize("T,g,n", [(82671, 3, 4), (82671, 4, 7), (5000, 1, 15), (20, 3, 4),
                                   (3, 3, 4), (2, 3, 4), (0, 3, 4), (4, 3, 4)])
def test_ngram_propose_bit_exact(dev, T, g, n):
    from lagunalab_amd.lookup import ngram_propose
    h = planted_history(max(T, 1))[:T] if T >= 100 else np.random.default_rng(T).integers(0, 3, T).astype(np.int32)
    hist = torch.from_numpy(np.ascontiguousarray(h)).to(dev) if T else torch.zeros(1, dtype=torch.int32, device=dev)
    out = ngram_propose(hist, T, g, n).cpu().numpy()
    cnt, pos, ids = O.propose_scan(h, T, g, n)
    assert int(out[0]) == cnt and int(out[1]) == pos
    assert out[2:2 + cnt].tolist() == ids
    assert ids == O.lookup(h.tolist(), T, g, n)


def test_ngram_edge_cases(dev):
    from lagunalab_amd.lookup import ngram_propose
    cases = [
        [7] * 6,                                   # overlapping match at s = T-g-1
        [1, 2, 3, 10, 1, 2, 3, 20, 5, 1, 2, 3],    # most recent match wins
        [1, 2, 3, 4, 5, 6, 7],                     # no match
        [5, 6, 7, 8, 5, 6, 7],                     # continuation truncated at T
    ]
    for seq in cases:
        h = torch.tensor(seq, dtype=torch.int32, device=dev)
        for g in (1, 2, 3):
            out = ngram_propose(h, len(seq), g, 4).cpu().numpy()
            want = O.lookup(seq, len(seq), g, 4)
            assert out[0] == len(want) and out[2:2 + len(want)].tolist() == want, (seq, g)


def test_device_index_matches_host_index(dev):
    from lagunalab_amd.lookup import DeviceNgramIndex, NgramIndex
    seq = [int(t) for t in np.random.default_rng(1).integers(0, 5, size=120)]
    a, b = NgramIndex(3), DeviceNgramIndex(3, dev, capacity=16)
    for t in range(len(seq)):
        assert a.propose(7) == b.propose(7)
        a.extend(seq[t:t + 1])
        b.extend(seq[t:t + 1])


@pytest.mark.parametrize("m", [0, 1, 2, 3, 4])
def test_greedy_accept_bit_exact(dev, m):
    from lagunalab_amd.lookup import greedy_accept
    rng = np.random.default_rng(m)
    logits = rng.standard_normal((5, 131072)).astype(np.float32)
    pred = logits.argmax(-1)
    drafts = np.array(list(pred[:m]) + [int(pred[m]) ^ 1] * (4 - m), np.int32)
    out = greedy_accept(torch.from_numpy(logits).to(dev), torch.from_numpy(drafts).to(dev)).cpu().numpy()
    k, nxt = O.greedy_accept(logits, drafts)
    assert int(out[0]) == k == m and int(out[1]) == nxt
    assert out[2:].tolist() == pred.tolist()


def test_greedy_accept_ties_and_odd_vocab(dev):
    from lagunalab_amd.lookup import greedy_accept
    logits = np.zeros((3, 10007), np.float32)
    logits[0, [9000, 17, 5000]] = 3.0   # first index (17) wins
    logits[1, [10006, 4096]] = 1.0      # across chunk boundary: 4096
    logits[2, :] = -1.0
    logits[2, 10006] = 0.0
    drafts = np.array([17, 4096], np.int32)
    out = greedy_accept(torch.from_numpy(logits).to(dev), torch.from_numpy(drafts).to(dev)).cpu().numpy()
    assert out.tolist() == [2, 10006, 17, 4096, 10006]


# ---------------------------------------------------------------------------------------------
# cache semantics on the GPU
# ---------------------------------------------------------------------------------------------

def test_quantized_cache_chunked_matches_one_pass(dev):
    """tests/test_cache.py:117-123's split: 200 + 60 rows, then 40 single rows, across the
    256-row growth step; the valid rows are bit-identical to one 300-row append."""
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(5)
    k = to_dev_bf16(Q.randn_bf16(rng, (1, 2, 300, 64)), dev)
    v = to_dev_bf16(Q.randn_bf16(rng, (1, 2, 300, 64)), dev)
    one = DequantKVCache(bits=8)
    ko, vo = one.update_and_fetch(k, v)
    c = DequantKVCache(bits=8)
    caps = []
    for a, b in [(0, 200), (200, 260)] + [(i, i + 1) for i in range(260, 300)]:
        kc, vc = c.update_and_fetch(k[:, :, a:b], v[:, :, a:b])
        caps.append(c.q.keys[0].shape[2])
    assert caps[0] == 256 and caps[1] == 456  # trimmed to 200, then one 256-row step
    assert c.offset == one.offset == 300
    torch.testing.assert_close(kc, ko, rtol=0, atol=0)
    torch.testing.assert_close(vc, vo, rtol=0, atol=0)
    for x, y in zip(c.state[0], one.state[0]):
        torch.testing.assert_close(x, y, rtol=0, atol=0)


def test_dequant_cache_switches(dev):
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(6)
    kv = lambda L: to_dev_bf16(Q.randn_bf16(rng, (1, 2, L, 64)), dev)
    c = DequantKVCache(bits=8, quantized_decode=True)
    k, _ = c.update_and_fetch(kv(5), kv(5))
    assert torch.is_tensor(k) and not hasattr(c, "bits")
    k, _ = c.update_and_fetch(kv(1), kv(1))
    assert isinstance(k, tuple) and c.bits == 8
    off = DequantKVCache(bits=8)
    off.update_and_fetch(kv(1), kv(1))
    assert not hasattr(off, "bits")
    assert c.trim(3) == 3 and c.offset == 3 and c.nbytes > 0


def test_fused_step_matches_dequantized_path(dev):
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(7)
    kv = lambda L: to_dev_bf16(Q.randn_bf16(rng, (1, 8, L, 128)), dev)
    fused, plain = DequantKVCache(fused_decode=True), DequantKVCache()
    k0, v0 = kv(600), kv(600)
    fused.update_and_fetch(k0, v0)
    plain.update_and_fetch(k0, v0)
    k1, v1 = kv(1), kv(1)
    fused.update_and_fetch(k1, v1)
    K, V = plain.update_and_fetch(k1, v1)
    assert fused.fused_step and not plain.fused_step
    q = to_dev_bf16(Q.randn_bf16(rng, (1, 32, 1, 128)), dev)
    got = fused.attend(q, 128 ** -0.5)
    qn = q.float().cpu().numpy()
    want = A.sdpa(qn, K.float().cpu().numpy(), V.float().cpu().numpy(), 128 ** -0.5)
    assert_attn_close(got, want.astype(np.float32), "fused vs dequantized", REF_SMALL_N_ATOL, 0.0)


# ---------------------------------------------------------------------------------------------
# 4-bit cache decode
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n,G,B", [(1, 4, 1), (7, 4, 1), (129, 2, 1), (700, 4, 2), (4096, 4, 1),
                                   (5003, 1, 1), (9000, 3, 1)])
def test_q4_decode_matches_oracle(dev, n, G, B):
    from lagunalab_amd.q8_attn import decode_attention
    rng = np.random.default_rng(300 + n + G)
    Hkv = 8
    cap = (n + 255) // 256 * 256
    kq, vq = make_cache(rng, B, Hkv, n, cap, dev, bits=4)
    q = Q.randn_bf16(rng, (B, Hkv * G, 1, 128))
    got = decode_attention(to_dev_bf16(q, dev), kq, vq, n=n, scale=128 ** -0.5)
    assert got.shape == (B, Hkv * G, 1, 128)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, 128 ** -0.5, bits=4),
                      f"q4 fused n={n} G={G}")
    at, rt = unfused_tol(n)
    assert_attn_close(got, A.unfused_attention(q, kn, vn, n, 128 ** -0.5, bits=4),
                      f"q4 unfused n={n} G={G}", at, rt)


def test_q4_decode_ragged_session_lengths(dev):
    """Ragged 4-bit decode equals one call per sequence at session lengths."""
    from lagunalab_amd.q8_attn import decode_attention
    lens = [82671, 42771, 60001]
    B, cap = len(lens), 82944
    g = torch.Generator(device=dev).manual_seed(9)
    mk = lambda: (torch.randint(0, 256, (B, 8, cap, 64), dtype=torch.uint8, device=dev, generator=g),
                  (torch.rand(B, 8, cap, 2, device=dev, generator=g) * 0.4).to(torch.bfloat16),
                  (torch.rand(B, 8, cap, 2, device=dev, generator=g) * -3).to(torch.bfloat16))
    kq, vq = mk(), mk()
    q = torch.randn(B, 32, 1, 128, device=dev, generator=g).to(torch.bfloat16)
    got = decode_attention(q, kq, vq, lens=lens, scale=128 ** -0.5)
    for b, n in enumerate(lens):
        one = decode_attention(q[b:b + 1], tuple(t[b:b + 1] for t in kq),
                               tuple(t[b:b + 1] for t in vq), n=n, scale=128 ** -0.5)
        torch.testing.assert_close(got[b:b + 1].float(), one.float(), atol=1e-3, rtol=1e-2)
    kn = tuple(t[2:3].cpu().numpy() if t.dtype == torch.uint8 else bits16(t[2:3]) for t in kq)
    vn = tuple(t[2:3].cpu().numpy() if t.dtype == torch.uint8 else bits16(t[2:3]) for t in vq)
    assert_attn_close(got[2:3], A.fused_attention(q[2:3].float().cpu().numpy(), kn, vn, 60001,
                                                  128 ** -0.5, bits=4), "q4 n=60001")


# ---------------------------------------------------------------------------------------------
# plain bf16 cache decode (the bandwidth reference of the quantized paths)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n,G,B", [(1, 4, 1), (7, 2, 1), (300, 4, 2), (1000, 1, 1), (4096, 4, 1),
                                   (5003, 3, 1)])
def test_bf16_decode_matches_sdpa(dev, n, G, B):
    from lagunalab_amd.q8_attn import decode_attention
    rng = np.random.default_rng(200 + n + G)
    Hkv = 8
    cap = (n + 255) // 256 * 256
    k = Q.randn_bf16(rng, (B, Hkv, cap, 128))
    v = Q.randn_bf16(rng, (B, Hkv, cap, 128))
    q = Q.randn_bf16(rng, (B, Hkv * G, 1, 128))
    got = decode_attention(to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev), n=n,
                           scale=128 ** -0.5)
    assert got.shape == (B, Hkv * G, 1, 128) and got.dtype == torch.bfloat16
    want = A.sdpa(q, k[:, :, :n], v[:, :, :n], 128 ** -0.5)
    assert_attn_close(got, want.astype(np.float32), f"bf16 n={n} G={G}")


def test_bf16_decode_ragged_and_session_length(dev):
    from lagunalab_amd.q8_attn import decode_attention
    g = torch.Generator(device=dev).manual_seed(5)
    lens = [82671, 42771, 1, 60000]
    B, cap = len(lens), 82944
    k = torch.randn(B, 8, cap, 128, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, 8, cap, 128, device=dev, generator=g).to(torch.bfloat16)
    q = torch.randn(B, 32, 1, 128, device=dev, generator=g).to(torch.bfloat16)
    got = decode_attention(q, k, v, lens=lens, scale=128 ** -0.5)
    for b, n in enumerate(lens):
        qn = q[b:b + 1].float().cpu().numpy()
        want = A.sdpa(qn, k[b:b + 1, :, :n].float().cpu().numpy(),
                      v[b:b + 1, :, :n].float().cpu().numpy(), 128 ** -0.5)
        assert_attn_close(got[b:b + 1], want.astype(np.float32), f"bf16 ragged n={n}")


def test_bf16_decode_rejects_large_groups(dev):
    from lagunalab_amd.q8_attn import decode_attention
    k = torch.zeros(1, 2, 256, 128, dtype=torch.bfloat16, device=dev)
    q = torch.zeros(1, 16, 1, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        decode_attention(q, k, k, n=10)


# ---------------------------------------------------------------------------------------------
# fused decode step: quantize-append of the new row inside the attention launch
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n,G,B", [(0, 4, 1), (63, 4, 1), (64, 4, 1), (700, 4, 1), (2583, 4, 1),
                                   (5000, 2, 2), (4095, 1, 1), (1500, 8, 1), (130, 16, 2)])
def test_fused_decode_step_equals_append_then_attend(dev, n, G, B):
    """lq_q8_decode_append_attn == lq_quantize_append_kv + lq_decode_attn: the same cache bytes
    (bit-exact, and equal to the oracle's quantizer) and the same attention output."""
    from lagunalab_amd.q8_attn import decode_append_attention, decode_attention
    from lagunalab_amd.quant import quantize_kv_into
    rng = np.random.default_rng(100 + n + G)
    Hkv = 8
    cap = (n + 1 + 255) // 256 * 256
    kq, vq = make_cache(rng, B, Hkv, max(n, 1), cap, dev)
    k1 = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    v1 = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    q = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv * G, 1, 128)), dev)
    kf, vf = tuple(t.clone() for t in kq), tuple(t.clone() for t in vq)
    got = decode_append_attention(q, k1, v1, kf, vf, n=n, scale=0.09)
    quantize_kv_into(k1, v1, kq, vq, n)
    want = decode_attention(q, kq, vq, n=n + 1, scale=0.09)
    for x, y in zip(kf + vf, kq + vq):
        assert torch.equal(x, y), f"cache differs n={n} G={G}"
    wc, ws, wb = Q.quantize_packed(k1.float().cpu().numpy(), 64, 8)
    np.testing.assert_array_equal(kf[0].cpu().numpy()[:, :, n:n + 1], wc)
    np.testing.assert_array_equal(bits16(kf[2])[:, :, n:n + 1], wb)
    torch.testing.assert_close(got.float(), want.float(), atol=1e-3, rtol=1e-2)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q.float().cpu().numpy(), kn, vn, n + 1, 0.09),
                      f"fused step n={n} G={G}")


def test_fused_decode_step_ragged(dev):
    from lagunalab_amd.q8_attn import decode_append_attention, decode_attention
    from lagunalab_amd.quant import quantize_kv_into
    rng = np.random.default_rng(41)
    lens = [61, 0, 2047, 512, 3000]
    B, Hkv, cap = len(lens), 8, 3072
    kq, vq = make_cache(rng, B, Hkv, cap, cap, dev)
    k1 = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    v1 = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    q = to_dev_bf16(Q.randn_bf16(rng, (B, 32, 1, 128)), dev)
    kf, vf = tuple(t.clone() for t in kq), tuple(t.clone() for t in vq)
    got = decode_append_attention(q, k1, v1, kf, vf, lens=lens, scale=0.09)
    for b, n in enumerate(lens):
        quantize_kv_into(k1[b:b + 1], v1[b:b + 1], tuple(t[b:b + 1] for t in kq),
                         tuple(t[b:b + 1] for t in vq), n)
    # the slices above are views of contiguous per-sequence blocks: kq now holds every new row
    want = decode_attention(q, kq, vq, lens=[x + 1 for x in lens], scale=0.09)
    for x, y in zip(kf + vf, kq + vq):
        assert torch.equal(x, y)
    torch.testing.assert_close(got.float(), want.float(), atol=1e-3, rtol=1e-2)


def test_fused_step_cache_defers_and_flushes(dev):
    """DequantKVCache(fused_decode=True): the fused step's cache equals the unfused cache's bytes
    after attend(); reading the returned tuples before attend() completes the append first."""
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(8)
    kv = lambda L: to_dev_bf16(Q.randn_bf16(rng, (1, 8, L, 128)), dev)
    fused, plain = DequantKVCache(fused_decode=True), DequantKVCache(quantized_decode=True)
    k0, v0 = kv(255), kv(255)
    fused.update_and_fetch(k0, v0)
    plain.update_and_fetch(k0, v0)
    q = to_dev_bf16(Q.randn_bf16(rng, (1, 32, 1, 128)), dev)
    for step in range(3):  # crosses the 256-row growth step
        k1, v1 = kv(1), kv(1)
        fk, fv = fused.update_and_fetch(k1, v1)
        pk, pv = plain.update_and_fetch(k1, v1)
        assert fused.fused_step and fused.offset == plain.offset == 256 + step
        if step == 1:  # touching the returned tuple writes the row now
            for x, y in zip(fk, pk):
                assert torch.equal(x, y)
        a = fused.attend(q, 0.09)
        from lagunalab_amd.q8_attn import q8_decode_attention
        b = q8_decode_attention(q, plain.q.keys, plain.q.values, plain.offset, 0.09)
        torch.testing.assert_close(a.float(), b.float(), atol=1e-3, rtol=1e-2)
        for x, y in zip(fused.q.keys + fused.q.values, plain.q.keys + plain.q.values):
            assert torch.equal(x[:, :, :fused.offset], y[:, :, :plain.offset])
    assert fused.trim(2) == 2 and fused.offset == 256


def test_prompt_cache_round_trip_continues_decoding(dev, tmp_path):
    """A fused-decode cache saved mid-step (a fused append still pending) and loaded again: the
    file holds the appended row, and the next fused decode steps on the loaded cache give the
    original cache's outputs and bytes bit for bit."""
    from lagunalab_amd.cache import DequantKVCache
    from lagunalab_amd.prompt_cache import load_prompt_cache, save_prompt_cache
    rng = np.random.default_rng(12)
    kv = lambda L: to_dev_bf16(Q.randn_bf16(rng, (1, 8, L, 128)), dev)
    a = DequantKVCache(fused_decode=True)
    a.update_and_fetch(kv(700), kv(700))
    a.update_and_fetch(kv(1), kv(1))  # pending: save() must write it first
    f = tmp_path / "p.safetensors"
    save_prompt_cache(f, [a], {"tokens": "701"})
    (b,), meta = load_prompt_cache(f, device=dev, return_metadata=True)
    assert meta == {"tokens": "701"} and b.offset == a.offset == 701 and b.fused_decode
    q = to_dev_bf16(Q.randn_bf16(rng, (1, 32, 1, 128)), dev)
    for _ in range(3):
        k1, v1 = kv(1), kv(1)
        a.update_and_fetch(k1, v1)
        b.update_and_fetch(k1, v1)
        assert torch.equal(a.attend(q, 0.09), b.attend(q, 0.09))
    for x, y in zip(a.state[0] + a.state[1], b.state[0] + b.state[1]):
        assert torch.equal(x, y)


# ---------------------------------------------------------------------------------------------
# fused causal verify attention (speculative-decoding block)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n,L,G", [(4101, 5, 4), (600, 2, 6), (1000, 8, 2), (300, 16, 4),
                                   (37, 5, 4), (16, 16, 1), (5000, 3, 8), (900, 2, 2),
                                   (1500, 4, 1), (130, 3, 1), (6000, 2, 1)])
def test_verify_matches_causal_oracle(dev, n, L, G):
    from lagunalab_amd.q8_attn import q8_verify_attention
    rng = np.random.default_rng(n + 7 * L + G)
    Hkv = 8
    cap = (n + 255) // 256 * 256
    kq, vq = make_cache(rng, 1, Hkv, n, cap, dev)
    q = Q.randn_bf16(rng, (1, Hkv * G, L, 128))
    scale = 128 ** -0.5
    got = q8_verify_attention(to_dev_bf16(q, dev), kq, vq, n, scale)
    assert got.shape == (1, Hkv * G, L, 128) and got.dtype == torch.bfloat16
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, scale, causal=True),
                      f"fused verify n={n} L={L} G={G}")
    at, rt = unfused_tol(n)
    assert_attn_close(got, A.unfused_attention(q, kn, vn, n, scale, causal=True),
                      f"unfused verify n={n} L={L} G={G}", at, rt)


@pytest.mark.parametrize("kind,L,G", [("verify", 5, 4), ("decode", 1, 6), ("decode", 1, 16)])
def test_two_kv_heads_many_splits_match_oracle(dev, kind, L, G):
    """Two KV heads give each head 128 workgroups' worth of splits: the dense kernel's merge launch
    then takes up to 64 splits per sequence (verify, and decode with 16 rows per KV head: the
    merge with 16 splits per lane), while the in-kernel merge (decode with 6 rows) caps them at 32."""
    from lagunalab_amd.q8_attn import decode_attention, q8_verify_attention
    rng = np.random.default_rng(90 + G * L)
    Hkv, n = 2, 20000
    cap = (n + 255) // 256 * 256
    kq, vq = make_cache(rng, 1, Hkv, n, cap, dev)
    q = Q.randn_bf16(rng, (1, Hkv * G, L, 128))
    scale = 128 ** -0.5
    if kind == "verify":
        got = q8_verify_attention(to_dev_bf16(q, dev), kq, vq, n, scale)
    else:
        got = decode_attention(to_dev_bf16(q, dev), kq, vq, n=n, scale=scale)
    kn, vn = cache_np(kq), cache_np(vq)
    causal = kind == "verify"
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, scale, causal=causal),
                      f"{kind} Hkv=2 G={G} L={L} fused")
    assert_attn_close(got, A.unfused_attention(q, kn, vn, n, scale, causal=causal),
                      f"{kind} Hkv=2 G={G} L={L} unfused")


@pytest.mark.parametrize("n,L,G", [(1500, 4, 1), (900, 2, 2), (130, 3, 1), (70000, 2, 2)])
def test_verify_packed_kernel_matches_causal_oracle(dev, n, L, G):
    """G * L <= 4 rows per KV head over two sequences, or one of more than 65,536 rows: the
    packed kernel's causal variant (a single shorter sequence takes the dense kernel, which the
    test above covers)."""
    from lagunalab_amd.q8_attn import q8_verify_attention
    rng = np.random.default_rng(n + 3 * L + G)
    Hkv = 8
    B = 1 if n > 65536 else 2
    cap = (n + 255) // 256 * 256
    kq, vq = make_cache(rng, B, Hkv, n, cap, dev)
    q = Q.randn_bf16(rng, (B, Hkv * G, L, 128))
    scale = 128 ** -0.5
    got = q8_verify_attention(to_dev_bf16(q, dev), kq, vq, n, scale)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, scale, causal=True),
                      f"fused verify n={n} L={L} G={G} B={B}")


@pytest.mark.parametrize("n,L,G,B", [(0, 5, 4, 1), (100, 5, 4, 1), (4093, 5, 4, 1), (65536, 5, 4, 1),
                                     (1000, 16, 4, 1), (300, 3, 6, 2), (500, 2, 2, 1), (777, 3, 1, 2),
                                     (63, 8, 2, 1)])
def test_fused_verify_step_equals_append_then_verify(dev, n, L, G, B):
    """lq_q8_verify_append_attn == lq_quantize_append_kv of the block's rows + lq_q8_verify_attn:
    the same cache bytes (bit-exact) and the same output, for blocks on the dense kernel (G * L > 4,
    the append inside the kernel, including blocks that straddle two 64-row super-tiles) and on
    the packed kernel (G * L <= 4, append launch first)."""
    from lagunalab_amd.q8_attn import q8_verify_append_attention, q8_verify_attention
    from lagunalab_amd.quant import quantize_kv_into
    rng = np.random.default_rng(300 + n + L + G)
    Hkv = 8
    cap = (n + L + 255) // 256 * 256
    kq, vq = make_cache(rng, B, Hkv, max(n, 1), cap, dev)
    kn = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, L, 128)), dev)
    vn = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, L, 128)), dev)
    q = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv * G, L, 128)), dev)
    kf, vf = tuple(t.clone() for t in kq), tuple(t.clone() for t in vq)
    got = q8_verify_append_attention(q, kn, vn, kf, vf, n, 0.09)
    quantize_kv_into(kn, vn, kq, vq, n)
    want = q8_verify_attention(q, kq, vq, n + L, 0.09)
    for x, y in zip(kf + vf, kq + vq):
        assert torch.equal(x, y), f"cache differs n={n} L={L} G={G}"
    assert torch.equal(got, want), f"fused verify step differs n={n} L={L} G={G}"
    if n + L <= 8192:
        assert_attn_close(got, A.fused_attention(q.float().cpu().numpy(), cache_np(kq), cache_np(vq),
                                                 n + L, 0.09, causal=True),
                          f"fused verify step n={n} L={L} G={G}")


def test_verify_single_row_equals_decode(dev):
    from lagunalab_amd.q8_attn import q8_decode_attention, q8_verify_attention
    rng = np.random.default_rng(11)
    kq, vq = make_cache(rng, 1, 8, 2000, 2048, dev)
    q = to_dev_bf16(Q.randn_bf16(rng, (1, 32, 1, 128)), dev)
    a = q8_decode_attention(q, kq, vq, 2000, 0.09)
    b = q8_verify_attention(q, kq, vq, 2000, 0.09)
    torch.testing.assert_close(a.float(), b.float(), atol=2e-3, rtol=1e-2)


@pytest.mark.slow
def test_verify_session_shape(dev):
    """Config 4a's shape: 65,536 cached keys + a 5-row block (1 accepted + 4 drafts), 32q/8kv."""
    from lagunalab_amd.q8_attn import q8_verify_attention
    rng = np.random.default_rng(4)
    n, L = 65536 + 5, 5
    kq, vq = make_cache(rng, 1, 8, n, 65536 + 256, dev)
    q = Q.randn_bf16(rng, (1, 32, L, 128))
    got = q8_verify_attention(to_dev_bf16(q, dev), kq, vq, n, 128 ** -0.5)
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.unfused_attention(q, kn, vn, n, 128 ** -0.5, causal=True), "verify 65541")


def test_fused_verify_step_in_cache(dev):
    """DequantKVCache(fused_decode=True) takes a 5-row block through the fused verify kernel;
    the result matches attention over the dequantized path with the causal mask."""
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(12)
    kv = lambda L: to_dev_bf16(Q.randn_bf16(rng, (1, 8, L, 128)), dev)
    fused, plain = DequantKVCache(fused_decode=True), DequantKVCache()
    k0, v0 = kv(700), kv(700)
    fused.update_and_fetch(k0, v0)
    plain.update_and_fetch(k0, v0)
    k1, v1 = kv(5), kv(5)
    fused.update_and_fetch(k1, v1)
    K, V = plain.update_and_fetch(k1, v1)
    assert fused.fused_step and not plain.fused_step
    q = to_dev_bf16(Q.randn_bf16(rng, (1, 32, 5, 128)), dev)
    got = fused.attend(q, 128 ** -0.5)
    want = A.sdpa(q.float().cpu().numpy(), K.float().cpu().numpy(), V.float().cpu().numpy(),
                  128 ** -0.5, causal=True)
    assert_attn_close(got, want.astype(np.float32), "fused verify vs dequantized",
                      REF_SMALL_N_ATOL, 0.0)


# ---------------------------------------------------------------------------------------------
# prefill chunks straight off the 8-bit cache (no dequantized copy, no score matrix)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n,L,G,Hkv,B", [(3000, 100, 4, 2, 1), (700, 64, 8, 2, 1), (33, 33, 1, 4, 1),
                                         (5000, 300, 4, 8, 1), (1200, 260, 2, 2, 2),
                                         (513, 513, 4, 1, 1), (4200, 17, 8, 8, 1),
                                         (2000, 17, 16, 1, 1), (900, 40, 3, 2, 1),
                                         (1536, 1536, 4, 2, 1), (1000, 1000, 8, 1, 1),
                                         (900, 900, 2, 2, 2), (2500, 1500, 4, 2, 1)])
def test_prefill_matches_causal_oracle(dev, n, L, G, Hkv, B):
    """q8_prefill_attention over n rows whose last L are the chunk's own: against the causal
    fused-arithmetic and unfused oracles. G in {1, 2, 4, 8}: the prefill kernel (blocks of
    256 / G positions, ragged last block, two sequences, a chunk that is the whole cache at
    n = L so that most tiles are masked or skipped); G = 16 and 3: the blocked verify path."""
    from lagunalab_amd.q8_attn import q8_prefill_attention
    rng = np.random.default_rng(n + L + G + B)
    cap = (n + 255) // 256 * 256
    kq, vq = make_cache(rng, B, Hkv, n, cap, dev)
    q = Q.randn_bf16(rng, (B, Hkv * G, L, 128))
    got = q8_prefill_attention(to_dev_bf16(q, dev), kq, vq, n, 0.09)
    assert got.shape == (B, Hkv * G, L, 128) and got.dtype == torch.bfloat16
    kn, vn = cache_np(kq), cache_np(vq)
    assert_attn_close(got, A.fused_attention(q, kn, vn, n, 0.09, causal=True),
                      f"fused prefill n={n} L={L} G={G}")
    at, rt = unfused_tol(n)
    assert_attn_close(got, A.unfused_attention(q, kn, vn, n, 0.09, causal=True),
                      f"unfused prefill n={n} L={L} G={G}", at, rt)


def test_prefill_blocks_equal_verify_calls(dev):
    """The blocked path: every block of a chunk is the verify kernel's result for those rows, bit
    for bit (16-row blocks at G = 4; rows 0..3 form the ragged first block); and the prefill
    kernel agrees with it within the attention tolerance."""
    from lagunalab_amd.q8_attn import _prefill_blocked, q8_prefill_attention, q8_verify_attention
    rng = np.random.default_rng(5)
    n, L = 1500, 52
    kq, vq = make_cache(rng, 1, 8, n, 1536, dev)
    q = to_dev_bf16(Q.randn_bf16(rng, (1, 32, L, 128)), dev)
    got = _prefill_blocked(q, kq, vq, n, 0.09)
    for a, b in ((0, 4), (4, 20), (20, 36), (36, 52)):
        want = q8_verify_attention(q[:, :, a:b].contiguous(), kq, vq, n - L + b, 0.09)
        assert torch.equal(got[:, :, a:b], want), (a, b)
    assert_attn_close(q8_prefill_attention(q, kq, vq, n, 0.09), got.float().cpu().numpy(),
                      "prefill kernel vs blocked path")


def test_prefill_never_materializes_scores(dev):
    """A 2,048-row chunk over 10,240 rows (32q/8kv) allocates only the chunk-sized copies: the
    score matrix alone would be 32 x 2,048 x 10,240 x 4 B = 2.7 GB (the reference's guard,
    tests/test_cache.py:79-93: quantized prefill peak < plain + 100 MB)."""
    from lagunalab_amd.cache import DequantKVCache
    rng = np.random.default_rng(6)
    c = DequantKVCache(fused_decode=True, fused_prefill=True)
    kv = lambda L: to_dev_bf16(Q.randn_bf16(rng, (1, 8, L, 128)), dev)
    c.update_and_fetch(kv(8192), kv(8192))
    q = to_dev_bf16(Q.randn_bf16(rng, (1, 32, 2048, 128)), dev)
    k, v = kv(2048), kv(2048)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    c.update_and_fetch(k, v)
    assert c.fused_step
    out = c.attend(q, 0.09)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(dev) - base
    assert out.shape == (1, 32, 2048, 128)
    assert peak < 100e6, peak
    # rows 2040.. of the chunk against the oracle over the same cache
    kn, vn = cache_np(c.q.keys), cache_np(c.q.values)
    qs = q[:, :, 2040:].float().cpu().numpy()
    want = A.fused_attention(qs, kn, vn, 10240, 0.09, causal=True)
    assert_attn_close(out[:, :, 2040:], want, "prefill rows 2040..2047 at 10,240")
