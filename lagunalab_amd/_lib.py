"""ctypes binding of liblaguna_hip.so (C ABI declared in include/laguna_hip.h).

The library is loaded after ``import torch`` so that it binds to the HIP runtime PyTorch has
already mapped (same soname). There is no CPU fallback: every op raises if the library is missing
or if it is called on tensors that are not on a ROCm device.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the library load: one HIP runtime per process)

LIB_PATH = Path(__file__).resolve().parent / "liblaguna_hip.so"

LQ_OK, LQ_EINVAL, LQ_EHIP, LQ_EWORKSPACE = 0, 1, 2, 3
LQ_KV_Q8, LQ_KV_Q4, LQ_KV_BF16 = 8, 4, 16
LQ_MAX_SEQS = 64
LQ_WS_ZERO_BYTES = 131072  # leading workspace bytes that attention calls keep at zero

i64, i32, f32, vp = C.c_int64, C.c_int, C.c_float, C.c_void_p

# name -> (restype, argtypes)
SIGNATURES = {
    "lq_version": (i32, []),
    "lq_last_error": (C.c_char_p, []),
    "lq_quantize_append": (i32, [vp, i64, i64, i64, i64, vp, vp, vp, i64, i64, i32, i32, vp]),
    "lq_quantize_append_kv": (i32, [vp, vp, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, i64, i64,
                                    i32, i32, vp]),
    "lq_dequantize": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, i32, i32, vp, vp]),
    "lq_decode_workspace_bytes": (i64, [i32, i64, i64, i64, i64, i64, vp]),
    "lq_decode_attn": (i32, [i32, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, vp,
                             f32, vp, vp, i64, vp]),
    "lq_q8_decode_append_attn": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64,
                                       i64, vp, f32, vp, vp, i64, vp]),
    "lq_verify_workspace_bytes": (i64, [i64, i64, i64, i64, i64, i64]),
    "lq_q8_verify_attn": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i64,
                                f32, vp, vp, i64, vp]),
    "lq_q8_verify_append_attn": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64,
                                       i64, i64, f32, vp, vp, i64, vp]),
    "lq_ngram_workspace_bytes": (i64, [i64]),
    "lq_ngram_propose": (i32, [vp, i64, i32, i32, vp, vp, i64, vp]),
    "lq_accept_workspace_bytes": (i64, [i64, i64]),
    "lq_greedy_accept": (i32, [vp, i64, i64, vp, i64, vp, vp, i64, vp]),
    "lq_qk_norm_rope": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, f32, vp, i64, f32,
                              i64, vp, vp]),
    "lq_gate_heads": (i32, [vp, vp, vp, i64, i64, i64, i64, i32, vp]),
    "lq_add_rms_norm": (i32, [vp, vp, vp, vp, vp, i64, i64, f32, vp]),
    "lq_gemv_bf16": (i32, [vp, vp, vp, i64, i64, vp]),
    "lq_gemv_fused": (i32, [vp, vp, vp, vp, vp, i64, i64, i32, f32, i32, vp]),
    "lq_q8_decode_norm_append_attn": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64,
                                            i64, i64, i64, vp, vp, vp, f32, vp, i64, f32, f32, vp,
                                            vp, i64, vp]),
    "lq_q8_prefill_attn": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i64,
                                 f32, vp, vp]),
    "lq_gemv_norm_rope": (i32, [vp, vp, vp, vp, i64, i64, f32, vp, vp, i64, i64, f32, vp, i64, f32,
                                i64, vp, vp, vp]),
    "lq_q8_decode_append_attn_pos": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64,
                                           i64, i64, vp, f32, vp, vp, i64, vp]),
    "lq_q8_decode_append_attn_noalloc": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64,
                                               i64, i64, i64, vp, f32, vp, vp]),
}

_lib = None


class LagunaHipError(RuntimeError):
    """A HIP-side failure reported by liblaguna_hip.so."""


def load():
    """Load (once) and return the ctypes library. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m lagunalab_amd.build` "
                "(there is no CPU fallback)")
        lib = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_symbols():
    """Names declared in the C header that the loaded library exports."""
    lib = load()
    return [n for n in SIGNATURES if hasattr(lib, n)]


def check(status: int, what: str):
    if status == LQ_OK:
        return
    msg = load().lq_last_error().decode(errors="replace")
    if status in (LQ_EINVAL, LQ_EWORKSPACE):
        raise ValueError(f"{what}: {msg}")
    raise LagunaHipError(f"{what}: {msg} (status {status})")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor):
    """All tensors on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("liblaguna_hip ops need tensors on a ROCm device "
                             f"(got one on {t.device}); there is no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
