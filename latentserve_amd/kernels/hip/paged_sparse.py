"""Sparse (page-subset) decode attention on the HIP kernels.

Mirrors the reference's kernels/cuda/paged_sparse.py: ``budget`` (:74-78),
``budgets`` (:171-182), ``select`` (:164-168), ``sparse_decode`` (:185-219)
and ``sparse_attention`` (:222-251), with ``page_scores`` / ``update_bounds``
/ ``rebuild_bounds`` on HIP kernels of their own.

Per layer per decode step the pipeline is index -> top-k -> attend, all on
the GPU and capturable in a HIP graph.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from latentserve_amd import _lib
from latentserve_amd.kernels.hip import paged_decode_hip as pdh

PAGE = pdh.PAGE


def budget(ratio: float, max_pages: int, recent: int = 2) -> int:
    """Pages kept per (sequence, KV head): at least the sink and recent ones."""
    if ratio >= 1.0:
        return max_pages
    return min(max_pages, max(recent + 1, math.ceil(ratio * max_pages)))


def budgets(seq_lens: torch.Tensor, ratio: float, recent: int = 2, page: int = 16) -> torch.Tensor:
    """Per-sequence budget for its current length — the rule the sparse kernel
    applies inline: max(recent + 1, ceil(ratio x pages)) in float32, capped at
    the pages it has. For tests and reference; the kernel does not use it."""
    pages = (seq_lens.to(torch.int64) + page - 1) // page
    if ratio >= 1.0:
        return pages.to(torch.int32)
    prod = torch.tensor(ratio, dtype=torch.float32, device=pages.device) * pages.to(torch.float32)
    n = torch.ceil(prod).to(torch.int64).clamp(min=recent + 1)
    return torch.minimum(n, pages).to(torch.int32)


def sparse_decode(q, k_pool, v_pool, block_tables, seq_lens, sel,
                  num_splits: Optional[int] = None,
                  softmax_scale: Optional[float] = None,
                  ratio: Optional[float] = None, recent: int = 2) -> torch.Tensor:
    """Attention over the pages in `sel` [B, H, K] only -> [B, H, n_rep, D].

    With `ratio`, each sequence attends the first max(recent+1,
    ceil(ratio*pages)) entries of its (score-sorted) list for its current
    length, counted on the device; entries past a sequence's end are skipped.
    """
    reason = pdh.ineligible_reason(q, k_pool)
    if reason is None and k_pool.dtype != torch.float16:
        reason = "the page-subset kernel reads fp16 pools"
    if reason is not None:
        raise ValueError(f"sparse_decode: {reason}")
    pdh._check_common(q, k_pool, v_pool, block_tables, seq_lens)
    if sel.dtype != torch.int32 or sel.dim() != 3 or sel.stride(-1) != 1:
        raise ValueError("sel must be an int32 [B, H, K] tensor with unit last stride")
    b, h, n_rep, d = q.shape
    num_sel = sel.shape[-1]
    splits = num_splits or pdh.choose_splits(b, h, num_sel, q.device)
    splits = max(1, min(splits, max(1, num_sel), pdh.MAX_SPLITS))
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    out, work, cnt = pdh._buffers("sparse", b, h, splits, n_rep, q.device)
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_paged_sparse_fp16(
        P(q), S(q, 3), P(k_pool), P(v_pool), S(k_pool, 3), k_pool.shape[0],
        P(block_tables), block_tables.stride(0), block_tables.shape[1], P(seq_lens),
        P(sel), S(sel, 2), num_sel, 0.0 if ratio is None else float(ratio), int(recent),
        P(out), S(out, 3), P(work), P(cnt), b, h, n_rep, d, k_pool.shape[1],
        splits, 0, float(scale), _lib.stream_of(q.device))
    _lib.check(rc, "ls_paged_sparse_fp16")
    return out[:, :, :n_rep]
