"""lq_q8_decode_append_attn_noalloc -- the fused decode step with the library's static scratch in
place of a caller workspace -- against lq_q8_decode_append_attn with a workspace, through the C
ABI: outputs and appended cache rows identical (same kernels, same split plan), on two calls in a
row, the second with a smaller input; inside HIP graphs (the first call of the process made during
a capture, and an eager call followed by a captured one), every replay checked; a shape whose
workspace exceeds the scratch is refused before any launch, and so is a call on another stream
than the one the device's scratch is bound to (its first call's).

Every call of this file runs on one stream per process (`_stream`): the scratch binds to the
stream of the first call on the device."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import make_cache, to_dev_bf16
from oracle import quantize as Q

pytestmark = pytest.mark.gpu

_STREAMS = {}


def _stream(dev):
    """The one stream every no-allocation call of this process is made on."""
    if dev not in _STREAMS:
        _STREAMS[dev] = torch.cuda.Stream(dev)
    return _STREAMS[dev]


def _args(q, kn, vn, cache, B, Hq, Hkv, cap, n, lens):
    (kc, ks, kb), (vc, vs, vb) = cache
    lens_arr = None if lens is None else C.cast((C.c_int32 * B)(*lens), C.c_void_p)
    return [q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), ks.data_ptr(),
            kb.data_ptr(), vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), B, Hq, Hkv, 128, cap,
            0 if lens is not None else n, lens_arr, 128 ** -0.5]


def _workspace_step(lib, q, kn, vn, cache, B, Hq, Hkv, cap, n, lens, out, sp):
    """The same fused step through the workspace entry (a fresh zeroed workspace)."""
    from lagunalab_amd import _lib
    need = lib.lq_decode_workspace_bytes(
        8, B, Hq, Hkv, 128, 0 if lens else n + 1,
        None if lens is None else C.cast((C.c_int32 * B)(*[x + 1 for x in lens]), C.c_void_p))
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=q.device)
    _lib.check(lib.lq_q8_decode_append_attn(*_args(q, kn, vn, cache, B, Hq, Hkv, cap, n, lens),
                                            out.data_ptr(), ws.data_ptr(), ws.numel(), sp),
               "lq_q8_decode_append_attn")
    torch.cuda.synchronize()


def _clone(cache):
    return tuple(tuple(t.clone() for t in kv) for kv in cache)


def _assert_same(out_a, out_b, cache_a, cache_b, what):
    assert torch.equal(out_a, out_b), f"{what}: outputs differ"
    for a, b in zip(cache_a[0] + cache_a[1], cache_b[0] + cache_b[1]):
        assert torch.equal(a, b), f"{what}: cache bytes differ"
    assert torch.isfinite(out_a.float()).all()


def _graph_case(dev, shape, seed, eager_first):
    """Captures the no-allocation step on `_stream` (after one eager call when `eager_first`)
    and replays it 4 times with new q, K and V rows copied into its input buffers between the
    replays; every replay's output and cache equal the workspace entry's on the same inputs."""
    from lagunalab_amd import _lib
    lib = _lib.load()
    S = _stream(dev)
    sp = S.cuda_stream
    B, Hkv, G, cap, n, lens = shape
    Hq = Hkv * G
    rng = np.random.default_rng(seed)
    rows = max(lens) if lens else n
    cache_g = make_cache(np.random.default_rng(seed + 1), B, Hkv, rows, cap, dev)
    cache_w = _clone(cache_g)
    q = torch.empty((B, Hq, 1, 128), dtype=torch.bfloat16, device=dev)
    kn = torch.empty((B, Hkv, 1, 128), dtype=torch.bfloat16, device=dev)
    vn = torch.empty_like(kn)
    out_g = torch.empty_like(q)
    out_w = torch.empty_like(q)

    def load_inputs():
        q.copy_(to_dev_bf16(Q.randn_bf16(rng, q.shape), dev))
        kn.copy_(to_dev_bf16(Q.randn_bf16(rng, kn.shape), dev))
        vn.copy_(to_dev_bf16(Q.randn_bf16(rng, vn.shape), dev))
        torch.cuda.synchronize()

    args = _args(q, kn, vn, cache_g, B, Hq, Hkv, cap, n, lens)
    if eager_first:
        load_inputs()
        with torch.cuda.stream(S):
            _lib.check(lib.lq_q8_decode_append_attn_noalloc(*args, out_g.data_ptr(), sp),
                       "eager lq_q8_decode_append_attn_noalloc")
        torch.cuda.synchronize()
        _workspace_step(lib, q, kn, vn, cache_w, B, Hq, Hkv, cap, n, lens, out_w, sp)
        _assert_same(out_g, out_w, cache_g, cache_w, "eager call")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=S):
        st = lib.lq_q8_decode_append_attn_noalloc(*args, out_g.data_ptr(), sp)
    _lib.check(st, "captured lq_q8_decode_append_attn_noalloc")
    for r in range(4):
        load_inputs()
        out_g.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _workspace_step(lib, q, kn, vn, cache_w, B, Hq, Hkv, cap, n, lens, out_w, sp)
        _assert_same(out_g, out_w, cache_g, cache_w, f"replay {r}")


def test_noalloc_first_call_inside_a_graph_capture(dev):
    """The file's first test: in a fresh process the first no-allocation call on the device (the
    scratch address lookup and its counter clear) happens while a graph is being captured. A
    batch of two sequences (the packed kernel, split merge in the kernel)."""
    _graph_case(dev, (2, 8, 4, 4352, None, [4200, 3001]), 300, eager_first=False)


@pytest.mark.parametrize("shape", [(1, 8, 4, 2048, 1500, None),      # dense kernel + merge launch
                                   (2, 4, 2, 1280, None, [1100, 700])],  # packed kernel
                         ids=["dense", "packed"])
def test_noalloc_eager_then_graph_replays(dev, shape):
    _graph_case(dev, shape, 400 + shape[1], eager_first=True)


@pytest.mark.parametrize("order", ["larger_first"])
def test_noalloc_equals_workspace_entry(dev, order):
    from lagunalab_amd import _lib
    lib = _lib.load()
    S = _stream(dev)
    sp = S.cuda_stream
    # (B, Hkv, G, cap, n or lens): the second call is smaller in every dimension
    for seed, (B, Hkv, G, cap, n, lens) in enumerate([(2, 8, 4, 9216, None, [9000, 6100]),
                                                      (1, 4, 2, 1024, 700, None)]):
        rng = np.random.default_rng(100 + seed)
        rows = max(lens) if lens else n
        c0 = make_cache(np.random.default_rng(200 + seed), B, Hkv, rows, cap, dev)
        caches = [c0, _clone(c0)]
        Hq = Hkv * G
        q = to_dev_bf16(Q.randn_bf16(rng, (B, Hq, 1, 128)), dev)
        kn = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
        vn = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
        outs = [torch.empty((B, Hq, 1, 128), dtype=torch.bfloat16, device=dev) for _ in range(2)]
        torch.cuda.synchronize()
        _workspace_step(lib, q, kn, vn, caches[0], B, Hq, Hkv, cap, n, lens, outs[0], sp)
        with torch.cuda.stream(S):
            st = lib.lq_q8_decode_append_attn_noalloc(*_args(q, kn, vn, caches[1], B, Hq, Hkv, cap,
                                                             n, lens), outs[1].data_ptr(), sp)
        _lib.check(st, "lq_q8_decode_append_attn_noalloc")
        torch.cuda.synchronize()
        _assert_same(outs[0], outs[1], caches[0], caches[1], f"call {seed}")


def test_noalloc_refuses_another_stream(dev):
    """A call on another stream than the device's first no-allocation call is refused with
    LQ_EINVAL before any launch (output and cache untouched); the bound stream still works."""
    from lagunalab_amd import _lib
    lib = _lib.load()
    S = _stream(dev)
    B, Hkv, G, cap, n = 1, 8, 4, 1024, 900
    cache = make_cache(np.random.default_rng(7), B, Hkv, n + 1, cap, dev)
    rng = np.random.default_rng(8)
    q = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv * G, 1, 128)), dev)
    kn = to_dev_bf16(Q.randn_bf16(rng, (B, Hkv, 1, 128)), dev)
    out = torch.empty_like(q)
    args = _args(q, kn, kn, cache, B, Hkv * G, Hkv, cap, n, None)
    torch.cuda.synchronize()
    with torch.cuda.stream(S):  # binds the scratch to S if no call of this process has yet
        _lib.check(lib.lq_q8_decode_append_attn_noalloc(*args, out.data_ptr(), S.cuda_stream),
                   "call on the bound stream")
    torch.cuda.synchronize()
    before = _clone(cache)
    first = out.clone()
    out.fill_(7.0)
    other = torch.cuda.Stream(dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(other):
        st = lib.lq_q8_decode_append_attn_noalloc(*args, out.data_ptr(), other.cuda_stream)
    torch.cuda.synchronize()
    assert st == _lib.LQ_EINVAL
    assert b"bound to stream" in lib.lq_last_error()
    assert torch.equal(out, torch.full_like(q, 7.0)), "a refused call wrote its output"
    _assert_same(first, first, cache, before, "refused call")
    with torch.cuda.stream(S):
        _lib.check(lib.lq_q8_decode_append_attn_noalloc(*args, out.data_ptr(), S.cuda_stream),
                   "call on the bound stream after a refusal")
    torch.cuda.synchronize()
    assert torch.equal(out, first), "the same step on the bound stream gave another output"


def test_noalloc_refuses_a_workspace_beyond_its_scratch(dev):
    """64 sequences with 16 query heads per KV head need about 4.4 MB of partials: refused with
    LQ_EWORKSPACE before any launch; the next call still runs."""
    from lagunalab_amd import _lib
    lib = _lib.load()
    S = _stream(dev)
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
                                                     lens), out.data_ptr(), S.cuda_stream)
    assert st == _lib.LQ_EWORKSPACE
    assert b"static scratch" in lib.lq_last_error()
    test_noalloc_equals_workspace_entry(dev, "larger_first")
