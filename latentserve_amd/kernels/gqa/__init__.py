"""Paged GQA decode attention: the reference's dispatch API (paged_decode.py)."""

from __future__ import annotations

import torch

# Persistent buffers, one per (name, shape, dtype, device) — the reference's
# `_scratch` (kernels/gqa/paged_decode.py:474-517). Keyed by shape so a
# captured graph's addresses stay valid when another shape is captured later;
# buffers are never replaced.
_SCRATCH: dict = {}


def _scratch(key, shape, dtype, device, fill=None, init=None):
    """Persistent scratch. `fill` is written on every call (the reference's
    semantics); `init` only when the buffer is first created."""
    full_key = (key, tuple(shape), dtype, str(device))
    buf = _SCRATCH.get(full_key)
    if buf is None:
        buf = torch.empty(shape, dtype=dtype, device=device)
        if init is not None:
            buf.fill_(init)
        _SCRATCH[full_key] = buf
    if fill is not None:
        buf.fill_(fill)
    return buf
