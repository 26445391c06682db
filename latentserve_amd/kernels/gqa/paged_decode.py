"""Paged GQA decode attention — the reference's dispatch API, HIP backend.

Same module surface as the reference's kernels/gqa/paged_decode.py:
``set_decode_backend`` / ``decode_backend`` (:488-498), ``_scratch``
(:501-517), ``choose_num_splits`` (:671-686), ``combine_splits`` (:689-706)
and ``paged_decode_attention`` (:709-829) with the identical signature, so a
caller (GQAAttention's decode branch, the graph runner, the tests) switches
by importing this module and selecting ``"hip"``.

Differences, each deliberate:

* The only backend is ``"hip"`` (hand-written gfx950 kernels). ``"triton"``
  and ``"cuda"`` name backends that do not exist on MI355X here, so
  selecting them raises, as any unknown name does in the reference.
* There is no silent fallback. The reference sends CPU tensors and
  ``force_reference=True`` to its torch loop and ineligible GPU inputs to
  Triton; here those raise ``ValueError`` with the reason. The torch-loop
  algorithm lives in the test oracle (oracle/), never on the product path.
* ``pages_per_iter``, ``num_warps`` and ``num_stages`` are Triton tunables.
  They stay in the signature as per-call keyword arguments (the reference's
  tests pin that, tests/test_phase11_kernel.py:419-434) and are ignored.
"""

from __future__ import annotations

import os
from typing import Optional

import torch

from latentserve_amd.kernels.gqa import _SCRATCH, _scratch  # noqa: F401  (re-exported)
from latentserve_amd.kernels.hip import paged_decode_hip as hip

_BACKENDS = ("hip",)
_BACKEND = {"decode": os.environ.get("LATENTSERVE_DECODE_BACKEND", "hip")}
if _BACKEND["decode"] not in _BACKENDS:
    _BACKEND["decode"] = "hip"


def set_decode_backend(name: str) -> None:
    if name not in _BACKENDS:
        raise ValueError(f"unknown decode backend {name!r} (this build provides 'hip')")
    _BACKEND["decode"] = name


def decode_backend() -> str:
    return _BACKEND["decode"]


def choose_num_splits(batch: int, kv_heads: int, max_seq_len: int, page: int,
                      device: torch.device, int8: bool = False) -> int:
    """The split rule ``paged_decode_attention`` applies when ``num_splits`` is
    None, callable before a launch so a graph runner can pin it per bucket
    (``int8``: for an INT8 pool)."""
    num_pages = (max_seq_len + page - 1) // page
    return hip.choose_splits(batch, kv_heads, num_pages, device, int8=int8)


def combine_splits(partial_acc: torch.Tensor, partial_m: torch.Tensor, partial_l: torch.Tensor,
                   out_dtype: torch.dtype) -> torch.Tensor:
    """Merge per-split partial softmaxes: partial_acc [B, H, S, N_REP, D],
    partial_m/l [B, H, S, N_REP] -> [B, H, N_REP, D] (one HIP launch)."""
    return hip.combine_splits_hip(partial_acc, partial_m, partial_l, out_dtype)


def paged_decode_attention(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    k_zero: Optional[torch.Tensor] = None,
    v_zero: Optional[torch.Tensor] = None,
    num_splits: Optional[int] = None,
    softmax_scale: Optional[float] = None,
    max_seq_len: Optional[int] = None,
    force_reference: bool = False,
    k_residual: Optional[torch.Tensor] = None,
    res_rows: Optional[torch.Tensor] = None,
    pages_per_iter: Optional[int] = None,
    num_warps: Optional[int] = None,
    num_stages: Optional[int] = None,
) -> torch.Tensor:
    """Paged decode attention, one query position per sequence.

    q [B, H_kv, N_REP, D] (query heads folded onto their KV head);
    k_pool/v_pool [num_blocks, PAGE, H_kv, D] fp16 or int8; block_tables
    [B, max_pages] int32; seq_lens [B] int32; INT8: k_scale [nb, H_kv, D],
    v_scale [nb, PAGE, H_kv] fp32 (+ zero points), k_residual
    [max_batch, PAGE, H_kv, D] fp16 with res_rows [B] int32.
    Returns [B, H_kv, N_REP, D] in q.dtype (a view of a persistent buffer).
    """
    del pages_per_iter, num_warps, num_stages          # Triton tunables: no meaning here
    if force_reference:
        raise ValueError("force_reference: the reference loop is test infrastructure "
                         "(oracle/), not a product path")
    if not q.is_cuda:
        raise ValueError("paged_decode_attention: the HIP backend needs GPU tensors")
    if max_seq_len is None:
        # As in the reference: one device sync. Callers should pass it.
        max_seq_len = int(seq_lens.max().item())
    return hip.paged_decode_hip(q, k_pool, v_pool, block_tables, seq_lens, max_seq_len,
                                num_splits=num_splits, softmax_scale=softmax_scale,
                                k_scale=k_scale, v_scale=v_scale, k_zero=k_zero, v_zero=v_zero,
                                k_residual=k_residual, res_rows=res_rows)
