"""lq_q8_decode_append_attn_noalloc -- the fused decode step with the library's static scratch in
place of a caller workspace -- against lq_q8_decode_append_attn with a workspace, through the C
ABI: outputs and appended cache rows identical (same kernels, same split plan), on two calls in a
row, the second with a smaller input; a shape whose workspace exceeds the scratch is refused before
any launch."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import make_cache, to_dev_bf16
from oracle import quantize as Q

pytestmark = pytest.mark.gpu


def _args(q, kn, vn, cache, B, Hq, Hkv, cap, n, lens):
    (kc, ks, kb), (vc, vs, vb) = cache
    lens_arr = None if lens is None else C.cast((C.c_int32 * B)(*lens), C.c_void_p)
    return [q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), ks.data_ptr(),
            kb.data_ptr(), vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), B, Hq, Hkv, 128, cap,
            0 if lens is not None else n, lens_arr, 128 ** -0.5]


@pytest.mark.parametrize("order", ["larger_first"])
def test_noalloc_equals_workspace_entry(dev, order):
    from lagunalab_amd import _lib
    lib = _lib.load()
    sp = _lib.stream_ptr(dev)
    # (B, Hkv, G, cap, n or lens): the second call is smaller in every dimension
    for seed, (B, Hkv, G, cap, n, lens) in enumerate([(2, 8, 4, 9216, None, [9000, 6100]),
                                                      (1, 4, 2, 1024, 700, None)]):
        rng = np.random.default_rng(100 + seed)
        rows = max(lens) if lens else n
        c0 = make_cache(np.random.default_rng(200 + seed), B, Hkv, rows, cap, dev)
        caches = [c0, tuple(tuple(t.clone() for t in kv) for kv in c0)]
        Hq = Hkv * G
        q = to_dev_bf16(Q.randn_bf16(rng, (B, Hq, 1, 128)), dev)
        kn = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
        vn = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
        outs = [torch.empty((B, Hq, 1, 128), dtype=torch.bfloat16, device=dev) for _ in range(2)]
        lens_after = None if lens is None else lens
        need = lib.lq_decode_workspace_bytes(
            8, B, Hq, Hkv, 128, 0 if lens else n + 1,
            None if lens is None else C.cast((C.c_int32 * B)(*[x + 1 for x in lens]), C.c_void_p))
        assert need > 0
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        st = lib.lq_q8_decode_append_attn(*_args(q, kn, vn, caches[0], B, Hq, Hkv, cap, n, lens_after),
                                          outs[0].data_ptr(), ws.data_ptr(), ws.numel(), sp)
        _lib.check(st, "lq_q8_decode_append_attn")
        st = lib.lq_q8_decode_append_attn_noalloc(*_args(q, kn, vn, caches[1], B, Hq, Hkv, cap, n,
                                                         lens_after), outs[1].data_ptr(), sp)
        _lib.check(st, "lq_q8_decode_append_attn_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), f"call {seed}: outputs differ"
        for a, b in zip(caches[0][0] + caches[0][1], caches[1][0] + caches[1][1]):
            assert torch.equal(a, b), f"call {seed}: cache bytes differ"
        assert torch.isfinite(outs[1].float()).all()


def test_noalloc_refuses_a_workspace_beyond_its_scratch(dev):
    """64 sequences with 16 query heads per KV head need about 4.4 MB of partials: refused with
    LQ_EWORKSPACE before any launch; the next call still runs."""
    from lagunalab_amd import _lib
    lib = _lib.load()
    sp = _lib.stream_ptr(dev)
    B, Hkv, G, cap = 64, 8, 16, 256
    lens = [100] * B
    cache = make_cache(np.random.default_rng(5), B, Hkv, 101, cap, dev)
    q = torch.zeros((B, Hkv * G, 1, 128), dtype=torch.bfloat16, device=dev)
    kn = torch.zeros((B, Hkv, 1, 128), dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(q)
    need = lib.lq_decode_workspace_bytes(8, B, Hkv * G, Hkv, 128, 0,
                                         C.cast((C.c_int32 * B)(*[x + 1 for x in lens]), C.c_void_p))
    assert need > 4 << 20
    st = lib.lq_q8_decode_append_attn_noalloc(*_args(q, kn, kn, cache, B, Hkv * G, Hkv, cap, 0,
                                                     lens), out.data_ptr(), sp)
    assert st == _lib.LQ_EWORKSPACE
    assert b"static scratch" in lib.lq_last_error()
    test_noalloc_equals_workspace_entry(dev, "larger_first")
