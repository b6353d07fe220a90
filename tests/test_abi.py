"""CPU checks of the C ABI: the library loads, exports every symbol include/laguna_hip.h declares,
and rejects bad arguments with LQ_EINVAL before touching the GPU."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "laguna_hip.h"


@pytest.fixture(scope="module")
def lib():
    from lagunalab_amd import _lib
    if not _lib.LIB_PATH.exists():
        from lagunalab_amd import build
        build.build()
    return _lib.load()


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lq_\w+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = header_functions()
    for want in ("lq_quantize_append", "lq_dequantize", "lq_decode_attn", "lq_q8_verify_attn",
                 "lq_ngram_propose", "lq_greedy_accept", "lq_version", "lq_last_error"):
        assert want in names


def test_library_exports_every_declared_symbol(lib):
    from lagunalab_amd import _lib
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(header_functions()) == set(_lib.SIGNATURES), "ctypes table out of sync with header"


def test_version(lib):
    assert lib.lq_version() >= 100


def test_quantize_rejects_bad_arguments(lib):
    from lagunalab_amd import _lib
    st = lib.lq_quantize_append(1, 1, 8, 1, 128, 1, 1, 1, 256, 0, 5, 64, None)
    assert st == _lib.LQ_EINVAL and b"bits" in lib.lq_last_error()
    st = lib.lq_quantize_append(1, 1, 8, 1, 96, 1, 1, 1, 256, 0, 8, 64, None)
    assert st == _lib.LQ_EINVAL and b"group_size" in lib.lq_last_error()
    st = lib.lq_quantize_append(1, 1, 8, 4, 128, 1, 1, 1, 256, 254, 8, 64, None)
    assert st == _lib.LQ_EINVAL and b"capacity" in lib.lq_last_error()
    st = lib.lq_quantize_append(None, 1, 8, 1, 128, 1, 1, 1, 256, 0, 8, 64, None)
    assert st == _lib.LQ_EINVAL


def test_decode_rejects_bad_arguments(lib):
    from lagunalab_amd import _lib
    args = dict(kind=8, q=1, kc=1, ks=1, kb=1, vc=1, vs=1, vb=1, B=1, Hq=32, Hkv=8, D=128,
                cap=256, n=10, lens=None, scale=0.1, out=1, ws=1, wsb=1 << 20, st=None)

    def call(**kw):
        a = {**args, **kw}
        return lib.lq_decode_attn(*a.values())

    assert call(D=64) == _lib.LQ_EINVAL
    assert call(Hq=30) == _lib.LQ_EINVAL
    assert call(Hq=136) == _lib.LQ_EINVAL  # 17 query heads per KV head
    assert call(B=0) == _lib.LQ_EINVAL
    assert call(B=65) == _lib.LQ_EINVAL
    assert call(q=None) == _lib.LQ_EINVAL
    assert call(kind=3) == _lib.LQ_EINVAL


def test_fused_step_rejects_bad_arguments(lib):
    from lagunalab_amd import _lib
    args = dict(q=1, kn=1, vn=1, kc=1, ks=1, kb=1, vc=1, vs=1, vb=1, B=1, Hq=32, Hkv=8, D=128,
                cap=256, n=10, lens=None, scale=0.1, out=1, ws=1, wsb=1 << 20, st=None)

    def call(**kw):
        a = {**args, **kw}
        return lib.lq_q8_decode_append_attn(*a.values())

    assert call(n=256) == _lib.LQ_EINVAL and b"room" in lib.lq_last_error()  # no free row
    assert call(kn=None) == _lib.LQ_EINVAL
    assert call(D=64) == _lib.LQ_EINVAL
    assert call(B=65) == _lib.LQ_EINVAL
    st = lib.lq_quantize_append_kv(1, 1, 1, 8, 4, 128, 1, 1, 1, 1, 1, 1, 256, 254, 8, 64, None)
    assert st == _lib.LQ_EINVAL and b"capacity" in lib.lq_last_error()


def test_lookup_ops_reject_bad_arguments(lib):
    from lagunalab_amd import _lib
    assert lib.lq_ngram_propose(1, 100, 0, 4, 1, 1, 64, None) == _lib.LQ_EINVAL
    assert lib.lq_ngram_propose(1, 100, 3, 0, 1, 1, 64, None) == _lib.LQ_EINVAL
    assert lib.lq_greedy_accept(1, 5, 100, 1, 5, 1, 1, 1 << 16, None) == _lib.LQ_EINVAL  # m > L-1
    assert lib.lq_greedy_accept(1, 0, 100, 1, 0, 1, 1, 1 << 16, None) == _lib.LQ_EINVAL


def test_workspace_queries(lib):
    assert lib.lq_ngram_workspace_bytes(82671) >= 4 * (82671 // 4096)
    assert lib.lq_accept_workspace_bytes(5, 131072) == 5 * 32 * 8


def test_python_constants_match_header():
    """The constants the Python side uses equal the header's #defines."""
    import re
    from pathlib import Path

    from lagunalab_amd import _lib
    hdr = (Path(__file__).resolve().parents[1] / "include" / "laguna_hip.h").read_text()
    defs = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define (LQ_\w+) (\d+)", hdr)}
    names = ("LQ_WS_ZERO_BYTES", "LQ_MAX_SEQS", "LQ_OK", "LQ_EINVAL", "LQ_EHIP", "LQ_EWORKSPACE",
             "LQ_KV_Q8", "LQ_KV_Q4", "LQ_KV_BF16")
    for name in names:
        assert getattr(_lib, name) == defs[name], name


def test_decode_split_plan_fills_one_wave(lib):
    """The 8-bit decode plan gives each KV head at most one wave of resident workgroups (256 CUs,
    one workgroup each, over 8 KV heads: 32 splits per head), apportioned over the sequences by
    keys per split. The split count is read back from the workspace size of batches (the packed
    kernel: the counter block plus one (m, l, acc[128]) fp32 partial per split, KV head and query
    row) and of single sequences of at most 65,536 rows (the dense kernel: the same, then the
    normalized q / k rows, 256-byte aligned). Without a GPU the host assumes 256 CUs and one
    resident workgroup per CU."""
    import ctypes as C

    import numpy as np

    from lagunalab_amd import _lib

    def splits(lens, Hq=32, Hkv=8):
        arr = (C.c_int32 * len(lens))(*lens)
        ws = lib.lq_decode_workspace_bytes(8, len(lens), Hq, Hkv, 128, 0, C.cast(arr, C.c_void_p))
        per = Hkv * (Hq // Hkv) * (128 * 4 + 8)
        if len(lens) == 1:
            assert lens[0] <= 65536
            ws -= (Hq + Hkv) * 128 * 2
            return (ws - _lib.LQ_WS_ZERO_BYTES) // per
        assert (ws - _lib.LQ_WS_ZERO_BYTES) % per == 0
        return (ws - _lib.LQ_WS_ZERO_BYTES) // per

    # config 3's lengths: a shared chunk would need 34 splits (a second, partial wave)
    c3 = [int(x) for x in np.random.default_rng(1).integers(42771, 82672, size=8)]
    assert splits(c3) == 32
    assert splits([82671, 82671]) == 32
    assert splits([65536]) == 32
    assert splits([1000]) == 4        # at least 256 keys per split
    assert splits([1, 1, 1]) == 3     # one split per sequence at least
    assert splits([5000] * 40) == 40  # more sequences than the budget: one split each


def _ws(lib, lens, Hq=32, Hkv=8, kind=8):
    import ctypes as C
    arr = (C.c_int32 * len(lens))(*lens)
    return lib.lq_decode_workspace_bytes(kind, len(lens), Hq, Hkv, 128, 0, C.cast(arr, C.c_void_p))


def test_decode_kernel_choice_at_the_length_boundary(lib):
    """One sequence of up to 65,536 rows (G L <= 4) takes the dense kernel and a merge launch:
    its workspace holds the normalized q / k rows behind the partials. From 65,537 rows the packed
    kernel merges inside and needs only counters + partials, but the size reported for one
    sequence also covers the dense kernel's need at 65,536 rows; batches take the packed kernel."""
    from lagunalab_amd import _lib
    per = 8 * 4 * (128 * 4 + 8)  # partial bytes per split, 32q/8kv
    partials = _lib.LQ_WS_ZERO_BYTES + 32 * per
    dense = _ws(lib, [65536])
    assert dense == (partials + 255) // 256 * 256 + (32 + 8) * 128 * 2
    assert _ws(lib, [65537]) == dense and _ws(lib, [82671]) == dense
    two = _ws(lib, [65536, 65536])
    assert two == partials  # a batch: packed, no norm rows
    # the 4-bit and bf16 kinds always run their packed kernels
    assert (_ws(lib, [4096], kind=4) - _lib.LQ_WS_ZERO_BYTES) % per == 0
    assert (_ws(lib, [4096], kind=16) - _lib.LQ_WS_ZERO_BYTES) % per == 0


@pytest.mark.parametrize("kind", [8, 4, 16])
@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (16, 4), (8, 2), (48, 8), (8, 8)])
def test_workspace_size_never_falls_as_the_length_grows(lib, kind, Hq, Hkv):
    """A workspace sized for a session's longest length serves every shorter call of the same
    shape: the reported size is non-decreasing in the length, across the dense/packed boundary
    at 65,536 rows (where, with 4 KV heads or fewer, the dense plan has up to 64 splits against
    the packed kernel's 32) and across the chunk rounding of the 4-bit and bf16 plans; the verify
    size likewise for every block length."""
    if kind != 8 and Hq // Hkv > 4:
        return
    lengths = sorted({1, 255, 256, 257, 1000, 4096, 16384, 16385, 20000, 32768, 65535, 65536,
                      65537, 70000, 82671, 100000, 262144, 1 << 20})
    sizes = [_ws(lib, [n], Hq, Hkv, kind) for n in lengths]
    assert min(sizes) > 0
    assert all(a <= b for a, b in zip(sizes, sizes[1:])), list(zip(lengths, sizes))
    for L in (1, 2, 5):
        if kind != 8 or (Hq // Hkv) * L > 64:
            continue
        vs = [lib.lq_verify_workspace_bytes(1, Hq, Hkv, L, 128, n) for n in lengths if n >= L]
        assert all(a <= b for a, b in zip(vs, vs[1:])), (L, vs)
