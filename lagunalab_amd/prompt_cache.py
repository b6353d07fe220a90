"""Prompt-cache files: every layer's cache state in one safetensors file.

The layout follows mlx-lm 0.31.3's ``save_prompt_cache`` / ``load_prompt_cache`` (the protocol
the reference's caches plug into through ``state`` and ``meta_state``; mlx-lm itself is not in
this environment, so byte compatibility with its files is not checked): the tensors of
``[c.state for c in caches]`` flattened with dotted indices (``"3.0.1"`` = layer 3, keys, scales
of a quantized cache; ``"0.1"`` = layer 0, values of a plain cache), and string metadata holding
``[[c.meta_state ...], metadata, [class names]]`` flattened the same way (``"0.3.1"``,
``"1.<key>"``, ``"2.3"``). The reference's ``DequantKVCache`` has no ``state`` setter
(``docs/architecture.md:347-349``), so its prompt caches cannot be loaded; the caches here can.
"""
from __future__ import annotations

import torch
from safetensors.torch import load_file, save_file

from . import cache as C

_CLASSES = {k: getattr(C, k) for k in ("QuantizedKVCache", "DequantKVCache", "KVCache",
                                       "RotatingKVCache", "TrimmableWindowCache")}


def _flatten(tree, prefix, out):
    if isinstance(tree, (list, tuple)):
        for i, t in enumerate(tree):
            _flatten(t, f"{prefix}{i}.", out)
    elif isinstance(tree, dict):
        for k, t in tree.items():
            _flatten(t, f"{prefix}{k}.", out)
    elif tree is not None:
        out[prefix[:-1]] = tree
    return out


def _unflatten(flat):
    """Dotted numeric keys -> nested tuples (missing leaves: None)."""
    root = {}
    for key, v in flat.items():
        node = root
        parts = key.split(".")
        for p in parts[:-1]:
            node = node.setdefault(p, {})
        node[parts[-1]] = v

    def build(node):
        if not isinstance(node, dict):
            return node
        n = 1 + max(int(k) for k in node)
        return tuple(build(node.get(str(i))) for i in range(n))
    return build(root)


def _make(cls_name):
    cls = _CLASSES[cls_name]
    if cls is C.QuantizedKVCache or cls is C.KVCache:
        return cls()
    if cls is C.DequantKVCache:
        return cls()
    if cls is C.RotatingKVCache:
        return cls(max_size=1)
    return cls(window=1)


def save_prompt_cache(path, caches, metadata: dict[str, str] | None = None):
    """Writes the states of ``caches`` (one per layer) to ``path`` (safetensors). Pending fused
    appends are completed first (reading ``state`` does that)."""
    states = [c.state for c in caches]
    tensors = {k: v.detach().contiguous().cpu() for k, v in _flatten(states, "", {}).items()}
    info = [list(c.meta_state) for c in caches]
    classes = [type(c).__name__ for c in caches]
    for name in classes:
        if name not in _CLASSES:
            raise ValueError(f"cannot save a {name}")
    meta = _flatten([info, dict(metadata or {}), classes], "", {})
    save_file(tensors, str(path), metadata={k: str(v) for k, v in meta.items()})


def load_prompt_cache(path, device=None, return_metadata: bool = False):
    """Reads a file written by :func:`save_prompt_cache`; tensors go to ``device`` (default: the
    current CUDA device when there is one, else the CPU)."""
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else "cpu"
    from safetensors import safe_open
    with safe_open(str(path), framework="pt") as f:
        meta = f.metadata() or {}
    tensors = {k: v.to(device) for k, v in load_file(str(path)).items()}
    classes, info, user = {}, {}, {}
    for k, v in meta.items():
        top, _, rest = k.partition(".")
        if top == "2":
            classes[int(rest)] = v
        elif top == "0":
            i, _, j = rest.partition(".")
            info.setdefault(int(i), {})[int(j)] = v
        elif top == "1":
            user[rest] = v
    n = len(classes)
    states = _unflatten(tensors) if tensors else ()
    caches = []
    for i in range(n):
        c = _make(classes[i])
        st = states[i] if i < len(states) else None
        if st is None:
            st = (None, None)
        c.state = st
        ms = info.get(i, {})
        c.meta_state = tuple(ms[j] for j in range(len(ms)))
        caches.append(c)
    return (caches, user) if return_metadata else caches
