"""The CPU baseline of bench.py (the reference's unfused path on all host cores, keys split in
chunks over worker threads) computes what the oracle computes."""
import numpy as np
import pytest

import bench
from oracle import attention as A
from oracle import quantize as Q


def _cache(rng, Hkv, n, bits):
    x = Q.randn_bf16(rng, (1, Hkv, n, 128))
    return tuple(Q.quantize_packed(x, 64, bits))


@pytest.mark.parametrize("bits,L,causal,n", [(8, 1, False, 9000), (4, 1, False, 5000),
                                             (8, 5, True, 4100), (8, 3, True, 10)])
def test_cpu_attention_matches_oracle(bits, L, causal, n):
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(n + bits)
    Hkv, Hq = 4, 12
    kc, vc = _cache(rng, Hkv, n, bits), _cache(rng, Hkv, n, bits)
    q = Q.randn_bf16(rng, (1, Hq, L, 128))
    with ThreadPoolExecutor(3) as pool:
        got = bench.cpu_attention(pool, q[0], tuple(t[0] for t in kc), tuple(t[0] for t in vc), n,
                                  0.09, bits=bits, causal=causal, chunk=1024)
    want = A.unfused_attention(q, kc, vc, n, 0.09, bits=bits, causal=causal)[0]
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-4)


def test_cpu_attention_plain_values():
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(5)
    k = Q.randn_bf16(rng, (2, 3000, 128))
    v = Q.randn_bf16(rng, (2, 3000, 128))
    q = Q.randn_bf16(rng, (8, 1, 128))
    with ThreadPoolExecutor(2) as pool:
        got = bench.cpu_attention(pool, q, k, v, 2999, 0.1, bits=None, chunk=700)
    want = A.sdpa(q[None], k[None, :, :2999], v[None, :, :2999], 0.1)[0]
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-4)


def test_cpu_threads_respects_share(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "2")
    threads, host = bench.cpu_threads()
    assert threads == min(2, host) and host >= 1
