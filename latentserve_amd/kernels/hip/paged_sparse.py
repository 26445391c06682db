"""Sparse (page-subset) decode attention on the HIP kernels.

Mirrors the reference's kernels/cuda/paged_sparse.py: ``budget`` (:74-78),
``rebuild_bounds`` (:81-84), ``update_bounds`` (:86-101), ``page_scores``
(:104-123), ``select`` (:164-168), ``budgets`` (:171-182), ``sparse_decode``
(:185-219) and ``sparse_attention`` (:222-251), all on HIP kernels.

Per layer per decode step ``sparse_attention`` with bounds scoring is one
launch (ls_sparse_attention_bounds_fp16): the page-subset decode's
workgroups score their shares of their sequence's pages, exchange the
scores, and each selects its own list with the selection kernel's radix
select (the same lists and partition as index + select + sparse_decode).
Mass scoring, and bounds scoring of rows longer than COOP_MAX_PAGES or of
more than COOP_MAX_NREP query rows a KV head, are two launches (the scores,
then ls_sparse_attention_fp16);
``fused=False`` runs the three (index, select, decode).  Nothing syncs with
the host, so the step is capturable in a HIP graph.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from latentserve_amd import _lib
from latentserve_amd.kernels.gqa import _scratch as scratch
from latentserve_amd.kernels.hip import paged_decode_hip as pdh

PAGE = pdh.PAGE
SELECT_MAX_PAGES = 8192
_LINE_FLOATS = 32          # one 128-byte line of fp32 scores per index group


def _check_bounds(kmin: torch.Tensor, kmax: torch.Tensor, device) -> None:
    if kmin.dtype != torch.float16 or kmax.dtype != torch.float16:
        raise ValueError("kmin/kmax must be float16 [num_blocks, H_kv, head_dim]")
    if kmin.dim() != 3 or kmin.shape != kmax.shape or kmin.stride() != kmax.stride() \
            or kmin.stride(-1) != 1:
        raise ValueError("kmin/kmax must match, [num_blocks, H_kv, head_dim], unit last stride")
    if kmin.device != device or kmax.device != device:
        raise ValueError("kmin/kmax must be on q's device")


def _score_buffer(b: int, h: int, max_pages: int, device) -> torch.Tensor:
    """Persistent [B, H, max_pages] fp32 view whose rows start on 128-byte
    lines (the fused index+select kernel's requirement)."""
    width = -(-max(1, max_pages) // _LINE_FLOATS) * _LINE_FLOATS
    buf = scratch("sparse_scores", (b, h, width), torch.float32, device)
    return buf[:, :, :max_pages]


def kernel_resources(device: Optional[torch.device] = None, n_rep: int = 6,
                     kv_heads: int = 2) -> dict:
    """Registers, private (spill) memory and LDS of each loaded page-subset
    kernel, by name (kernels/cuda/paged_sparse.py:254-265; the reference's
    four names plus this build's selection and one-launch kernels)."""
    names = ("page_bounds_update", "page_index", "page_index_heads", "paged_sparse_fp16",
             "page_mass", "page_select", "page_bounds_rebuild", "sparse_attention_fp16",
             "sparse_attention_bounds_fp16")
    return {n: _lib.kernel_resources(n, device, kv_heads=kv_heads, n_rep=n_rep) for n in names}


def rebuild_bounds(k_pool: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor) -> None:
    """Every block's per-channel K bounds from the pool, over all PAGE rows."""
    _check_bounds(kmin, kmax, k_pool.device)
    if k_pool.dtype != torch.float16 or k_pool.stride(-1) != 1:
        raise ValueError("k_pool must be float16 with unit last stride")
    nb, page, h, d = k_pool.shape
    if kmin.shape != (nb, h, d):
        raise ValueError(f"kmin/kmax must be [{nb}, {h}, {d}]")
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_page_bounds_rebuild(P(k_pool), S(k_pool, 3), nb, P(kmin), P(kmax),
                                           S(kmin, 2), h, d, page, _lib.stream_of(k_pool.device))
    _lib.check(rc, "ls_page_bounds_rebuild")


def update_bounds(k_new: torch.Tensor, slots: torch.Tensor, kmin: torch.Tensor,
                  kmax: torch.Tensor, page: int = 16) -> None:
    """k_new [B, H, D] (or [B, H, 1, D]) just written at flat `slots` [B]."""
    k = k_new.reshape(k_new.shape[0], k_new.shape[1], k_new.shape[-1])
    _check_bounds(kmin, kmax, k.device)
    if k.dtype != torch.float16 or k.stride(-1) != 1:
        raise ValueError("k_new must be float16 with unit last stride")
    if slots.dtype != torch.int64 or slots.dim() != 1 or slots.shape[0] != k.shape[0] \
            or slots.stride(0) != 1:
        raise ValueError("slots must be a contiguous int64 [B] tensor")
    b, h, d = k.shape
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_page_bounds_update(P(k), S(k, 2), P(slots), P(kmin), P(kmax), S(kmin, 2),
                                          kmin.shape[0], b, h, d, page,
                                          _lib.stream_of(k.device))
    _lib.check(rc, "ls_page_bounds_update")


def _check_index_inputs(q, kmin, kmax, block_tables, seq_lens):
    if q.dtype != torch.float16 or q.dim() != 4 or q.stride(-1) != 1:
        raise ValueError("q must be float16 [B, H_kv, n_rep, D] with unit last stride")
    _check_bounds(kmin, kmax, q.device)
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32 \
            or block_tables.stride(-1) != 1 or seq_lens.stride(-1) != 1:
        raise ValueError("block tables and sequence lengths must be unit-stride int32")


def page_scores(q, kmin, kmax, block_tables, seq_lens, recent: int = 2) -> torch.Tensor:
    """-> [B, H, max_pages] fp32: bound per page, +inf forced, -inf past the end."""
    _check_index_inputs(q, kmin, kmax, block_tables, seq_lens)
    b, h, n_rep, d = q.shape
    max_pages = block_tables.shape[1]
    scores = _score_buffer(b, h, max_pages, q.device)
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_page_scores(
        P(q), S(q, 3), P(kmin), P(kmax), S(kmin, 2), kmin.shape[0], P(block_tables),
        block_tables.stride(0), max_pages, P(seq_lens), P(scores), S(scores, 2),
        b, h, n_rep, d, PAGE, int(recent), _lib.stream_of(q.device))
    _lib.check(rc, "ls_page_scores")
    return scores


def page_scores_mass(q, kmin, kmax, block_tables, seq_lens, recent: int = 2,
                     softmax_scale: Optional[float] = None, page: int = PAGE) -> torch.Tensor:
    """Summed-mass scores -> [B, H, max_pages] fp32 (kernels/cuda/
    paged_sparse.py:126-161): for each query head a softmax over the pages
    of bound * scale + log(tokens in the page), summed over the group; page
    0 and the last `recent` pages +inf, pages past the end -inf.  Two
    launches; the per-head logits go through a persistent workspace."""
    _check_index_inputs(q, kmin, kmax, block_tables, seq_lens)
    if page != PAGE:
        raise ValueError(f"the HIP indexer reads {PAGE}-token pages")
    b, h, n_rep, d = q.shape
    max_pages = block_tables.shape[1]
    scores = _score_buffer(b, h, max_pages, q.device)
    nbytes = _lib.lib().ls_page_mass_workspace_bytes(b, h, n_rep, max_pages)
    work = scratch("sparse_mass_heads", (max(1, nbytes // 4),), torch.float32, q.device)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_page_scores_mass(
        P(q), S(q, 3), P(kmin), P(kmax), S(kmin, 2), kmin.shape[0], P(block_tables),
        block_tables.stride(0), max_pages, P(seq_lens), P(work), P(scores), S(scores, 2),
        b, h, n_rep, d, PAGE, int(recent), float(scale), _lib.stream_of(q.device))
    _lib.check(rc, "ls_page_scores_mass")
    return scores


def select(scores: torch.Tensor, k: int, sorted: bool = False,
           seq_lens: Optional[torch.Tensor] = None, ratio: Optional[float] = None,
           recent: int = 2) -> torch.Tensor:
    """Top-k pages per (sequence, head) -> int32 [B, H, k].

    Ties between equal scores go to the lower page. ``sorted``: best first
    (forced +inf pages first, then by score). Unsorted, the pages come in
    page order; given ``seq_lens`` and ``ratio``, the first n_b entries of
    sequence b are then its own budget's best pages (what sparse_decode
    attends with that ratio) and the remaining k - n_b follow.
    """
    if scores.dtype != torch.float32 or scores.dim() != 3 or scores.stride(-1) != 1:
        raise ValueError("scores must be float32 [B, H, P] with unit last stride")
    b, h, p = scores.shape
    k = int(k)
    if not 0 <= k <= p:
        raise ValueError(f"k={k} out of range for {p} pages")
    if p > SELECT_MAX_PAGES:
        raise ValueError(f"select supports up to {SELECT_MAX_PAGES} pages, got {p}")
    use_ratio = ratio is not None and not sorted
    if use_ratio and (seq_lens is None or seq_lens.dtype != torch.int32):
        raise ValueError("a ratio needs int32 seq_lens")
    if k == 0 or b == 0:
        return torch.empty(b, h, k, dtype=torch.int32, device=scores.device)
    sel = scratch("sparse_select", (b, h, k), torch.int32, scores.device)
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_page_select(
        P(scores), S(scores, 2), P(seq_lens) if use_ratio else None, b, h, p, k,
        float(ratio) if use_ratio else 0.0, int(recent), 1 if sorted else 0, P(sel),
        (ctypes.c_int64 * 2)(*sel.stride()[:2]), _lib.stream_of(scores.device))
    _lib.check(rc, "ls_page_select")
    return sel


def index_select(q, kmin, kmax, block_tables, seq_lens, k: int, ratio: float,
                 recent: int = 2) -> torch.Tensor:
    """page_scores + select(ratio=...) -> int32 [B, H, k] (two launches)."""
    _check_index_inputs(q, kmin, kmax, block_tables, seq_lens)
    b, h, n_rep, d = q.shape
    max_pages = block_tables.shape[1]
    if max_pages > SELECT_MAX_PAGES:
        raise ValueError(f"selection supports up to {SELECT_MAX_PAGES} pages, got {max_pages}")
    k = int(k)
    if not 1 <= k <= max_pages:
        raise ValueError(f"k={k} out of range for {max_pages} pages")
    scores = _score_buffer(b, h, max_pages, q.device)
    sel = scratch("sparse_index_sel", (b, h, k), torch.int32, q.device)
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_sparse_index(
        P(q), S(q, 3), P(kmin), P(kmax), S(kmin, 2), kmin.shape[0], P(block_tables),
        block_tables.stride(0), max_pages, P(seq_lens), P(scores), S(scores, 2), None, k,
        float(ratio), int(recent), P(sel), S(sel, 2), b, h, n_rep, d, PAGE,
        _lib.stream_of(q.device))
    _lib.check(rc, "ls_sparse_index")
    return sel


def budget(ratio: float, max_pages: int, recent: int = 2) -> int:
    """List width for a context of max_pages pages: ceil(ratio x pages),
    never fewer than page 0 plus the `recent` forced pages, never more than
    the pages there are (paged_sparse.py:74-78)."""
    if ratio >= 1.0:
        return max_pages
    return min(max_pages, max(recent + 1, math.ceil(ratio * max_pages)))


def budgets(seq_lens: torch.Tensor, ratio: float, recent: int = 2, page: int = 16) -> torch.Tensor:
    """int32 [B]: how many pages each sequence attends at its present
    length (paged_sparse.py:171-182).  The same product the kernels form in
    fp32 with ceilf, so host and device agree on every length; raised to
    recent + 1, cut to the sequence's pages.  The kernels compute it
    themselves: this is for callers and tests."""
    pages = (seq_lens.to(torch.int64) + page - 1) // page
    if ratio >= 1.0:
        return pages.to(torch.int32)
    prod = torch.tensor(ratio, dtype=torch.float32, device=pages.device) * pages.to(torch.float32)
    n = torch.ceil(prod).to(torch.int64).clamp(min=recent + 1)
    return torch.minimum(n, pages).to(torch.int32)


def sparse_decode(q, k_pool, v_pool, block_tables, seq_lens, sel,
                  num_splits: Optional[int] = None,
                  softmax_scale: Optional[float] = None,
                  ratio: Optional[float] = None, recent: int = 2,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention over the pages in `sel` [B, H, K] only -> [B, H, n_rep, D]
    (into `out` when given, as paged_decode_hip).

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
    buf, work, cnt = pdh._buffers("sparse", b, h, splits, n_rep, q.device)
    target = buf if out is None else pdh.check_out(out, q)
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_paged_sparse_fp16(
        P(q), S(q, 3), P(k_pool), P(v_pool), S(k_pool, 3), k_pool.shape[0],
        P(block_tables), block_tables.stride(0), block_tables.shape[1], P(seq_lens),
        P(sel), S(sel, 2), num_sel, 0.0 if ratio is None else float(ratio), int(recent),
        P(target), S(target, 3), P(work), P(cnt), b, h, n_rep, d, k_pool.shape[1],
        splits, 0, float(scale), _lib.stream_of(q.device))
    _lib.check(rc, "ls_paged_sparse_fp16")
    return buf[:, :, :n_rep] if out is None else out


SELECT_SPLIT_ENTRIES = 1024    # list entries a selecting group keeps (a split's share)
# the one-launch bounds path: rows of at most this many pages, at most this
# many query rows a KV head (else the index kernel, then the selecting decode)
COOP_MAX_PAGES = 2048
COOP_MAX_NREP = 8


def sparse_attention(q, k_pool, v_pool, block_tables, seq_lens, kmin, kmax,
                     ratio: float = 0.25, recent: int = 2,
                     num_splits: Optional[int] = None, max_seq_len: Optional[int] = None,
                     softmax_scale: Optional[float] = None,
                     scoring: str = "bounds",
                     out: Optional[torch.Tensor] = None, fused: bool = True) -> torch.Tensor:
    """Index, select, attend. The list width k follows `max_seq_len` (the
    context) when given, else the table's width; each sequence then attends
    its own budget for its current length.  Fused, bounds scoring is one
    launch (the decode's workgroups score, select and attend) and mass
    scoring two (the scores, then a decode that selects); ``fused=False``
    runs index, select and decode as three."""
    if scoring not in ("bounds", "mass"):
        raise ValueError(f"unknown scoring {scoring!r} (bounds or mass)")
    page = k_pool.shape[1]
    pages = block_tables.shape[1] if max_seq_len is None else min(
        block_tables.shape[1], -(-int(max_seq_len) // page))
    k = budget(ratio, pages, recent)
    if not fused:
        if scoring == "mass":
            mass = page_scores_mass(q, kmin, kmax, block_tables, seq_lens, recent, softmax_scale)
            sel = select(mass, k, seq_lens=seq_lens, ratio=ratio, recent=recent)
        else:
            sel = index_select(q, kmin, kmax, block_tables, seq_lens, k, ratio, recent)
        return sparse_decode(q, k_pool, v_pool, block_tables, seq_lens, sel, num_splits,
                             softmax_scale, ratio=ratio, recent=recent, out=out)
    reason = pdh.ineligible_reason(q, k_pool)
    if reason is None and k_pool.dtype != torch.float16:
        reason = "the page-subset kernel reads fp16 pools"
    if reason is not None:
        raise ValueError(f"sparse_attention: {reason}")
    pdh._check_common(q, k_pool, v_pool, block_tables, seq_lens)
    if block_tables.shape[1] > SELECT_MAX_PAGES:
        raise ValueError(f"selection supports up to {SELECT_MAX_PAGES} pages, "
                         f"got {block_tables.shape[1]}")
    b, h, n_rep, d = q.shape
    splits = num_splits or pdh.choose_splits(b, h, k, q.device)
    splits = max(1, min(splits, max(1, k), pdh.MAX_SPLITS))
    splits = max(splits, -(-k // SELECT_SPLIT_ENTRIES))
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    buf, work, cnt = pdh._buffers("sparse", b, h, splits, n_rep, q.device)
    target = buf if out is None else pdh.check_out(out, q)
    P, S = _lib.ptr, _lib.strides
    if (scoring == "bounds" and block_tables.shape[1] <= COOP_MAX_PAGES
            and n_rep <= COOP_MAX_NREP):
        # one launch: the decode's workgroups score the pages themselves,
        # exchanging the scores through a buffer whose count words are all
        # ones at rest
        _check_bounds(kmin, kmax, q.device)
        # (each row is followed by one word: the count of its scored shares)
        # (rows padded to 16 bytes, so a row starts 16-byte aligned)
        ws = scratch("sparse_coop_scores", (b, h, (block_tables.shape[1] + 4) // 4 * 4),
                     torch.int32, q.device, init=-1)
        rc = _lib.lib().ls_sparse_attention_bounds_fp16(
            P(q), S(q, 3), P(k_pool), P(v_pool), S(k_pool, 3), k_pool.shape[0],
            P(block_tables), block_tables.stride(0), block_tables.shape[1], P(seq_lens),
            P(kmin), P(kmax), S(kmin, 2), P(ws), S(ws, 2), k, float(ratio), int(recent),
            P(target), S(target, 3), P(work), P(cnt), b, h, n_rep, d, page,
            splits, 0, float(scale), _lib.stream_of(q.device))
        _lib.check(rc, "ls_sparse_attention_bounds_fp16")
        return buf[:, :, :n_rep] if out is None else out
    if scoring == "mass":
        scores = page_scores_mass(q, kmin, kmax, block_tables, seq_lens, recent, softmax_scale)
    else:
        scores = page_scores(q, kmin, kmax, block_tables, seq_lens, recent)
    rc = _lib.lib().ls_sparse_attention_fp16(
        P(q), S(q, 3), P(k_pool), P(v_pool), S(k_pool, 3), k_pool.shape[0],
        P(block_tables), block_tables.stride(0), block_tables.shape[1], P(seq_lens),
        P(scores), S(scores, 2), scores.shape[2], k, float(ratio), int(recent),
        P(target), S(target, 3), P(work), P(cnt), b, h, n_rep, d, page,
        splits, 0, float(scale), _lib.stream_of(q.device))
    _lib.check(rc, "ls_sparse_attention_fp16")
    return buf[:, :, :n_rep] if out is None else out
