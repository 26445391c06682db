"""Block-table gather on a HIP kernel: the paged cache's read path.

Mirrors PagedKVCache.read (cache/paged_cache.py:486-506): every live token's
rows of a layer's pool, in logical order, as [B, H, L, D] (a permuted view of
a [B, L, H, D] buffer, as the reference returns).  Positions past a
sequence's length hold flat slot 0, as the reference's zero-padded slot
table (:305-323) reads; the caller masks them.
"""

from __future__ import annotations

from typing import Optional

import torch

from latentserve_amd import _lib

PAGE = 16


def gather(pool: torch.Tensor, block_tables: torch.Tensor, seq_lens: torch.Tensor,
           length: Optional[int] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """pool [nb, 16, H, D] (fp16 / int8 / fp32) -> [B, H, length, D] view.

    `length` defaults to the table's width in tokens; `out` (a [B, length, H,
    D] tensor) is written in place when given.  Bit-exact copy."""
    if pool.dim() != 4 or pool.shape[1] != PAGE or pool.stride(-1) != 1:
        raise ValueError("pool must be [num_blocks, 16, H, D] with unit channel stride")
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32 \
            or block_tables.stride(-1) != 1 or seq_lens.stride(-1) != 1:
        raise ValueError("block tables and sequence lengths must be unit-stride int32")
    nb, _, h, d = pool.shape
    b = block_tables.shape[0]
    length = block_tables.shape[1] * PAGE if length is None else int(length)
    if out is None:
        out = torch.empty(b, length, h, d, dtype=pool.dtype, device=pool.device)
    elif out.shape != (b, length, h, d) or out.dtype != pool.dtype or out.stride(-1) != 1:
        raise ValueError(f"out must be {pool.dtype} [{b}, {length}, {h}, {d}]")
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_paged_gather(
        P(pool), pool.element_size(), S(pool, 3), nb, P(block_tables), block_tables.stride(0),
        block_tables.shape[1], P(seq_lens), P(out), S(out, 3), b, h, d, PAGE, length,
        _lib.stream_of(pool.device))
    _lib.check(rc, "ls_paged_gather")
    return out.permute(0, 2, 1, 3)


def read(k_pool: torch.Tensor, v_pool: torch.Tensor, block_tables: torch.Tensor,
         seq_lens: torch.Tensor, length: Optional[int] = None):
    """(k, v) [B, H, L, D] for one layer: PagedKVCache.read's result."""
    return (gather(k_pool, block_tables, seq_lens, length),
            gather(v_pool, block_tables, seq_lens, length))
