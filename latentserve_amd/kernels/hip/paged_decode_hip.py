"""The MI355X paged decode backend: HIP kernels behind a C ABI.

Mirrors the reference's CUDA backend module (kernels/cuda/paged_decode_cuda.py):
``eligible`` (:112-141), ``choose_splits`` (:197-199) and the launcher
``paged_decode_cuda`` (:202-252), here ``paged_decode_hip``. The same
arguments, the same ValueErrors for non-unit strides / non-int32 tables, the
same return value (a ``[B, H_kv, n_rep, D]`` view of a persistent fp16 buffer).

What differs is underneath: one launch per call (the split combine is fused
into the decode kernel: the last workgroup of each (sequence, head) merges
the partials), MFMA tiles instead of scalar FMAs, and no runtime compilation —
the library is built ahead of time for gfx950.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from latentserve_amd import _lib
from latentserve_amd.kernels.gqa import _scratch as scratch

HEAD_DIM = 128
PAGE = 16
MAX_NREP = 16
MAX_SPLITS = 1024
# (sequence, KV head, split) units per 4 CUs the split count aims at.  A
# workgroup serves the splits of a KV-head pair (two units), one workgroup a
# CU fits, and more groups than CUs leave a second, partial round.  INT8: one
# group a CU (8 units a 4 CUs), the measured optimum (B16 x 16K: 14 splits
# 34.6 us, 15: 33.1, 16: 32.9).  fp16: 7 groups an 8 CUs (7 units a 4 CUs):
# fewer split records to combine, and the walk is bound by HBM as a whole,
# not by the CUs (B16 x 16K: 13-14 splits 46.4-46.5 us against 46.7-46.8 at
# 16; B8 x 32K: 28 splits 48.4 us against 48.8 at 32).
UNITS_PER_4_CUS = {"fp16": 7, "int8": 8}
# Fewest pages a split is given.
MIN_SPLIT_PAGES = 8

_CU_COUNT: dict = {}


def _cus(device: torch.device) -> int:
    dev = device.index if device.index is not None else torch.cuda.current_device()
    if dev not in _CU_COUNT:
        _CU_COUNT[dev] = torch.cuda.get_device_properties(dev).multi_processor_count
    return _CU_COUNT[dev]


def choose_splits(batch: int, kv_heads: int, num_pages: int,
                  device: Optional[torch.device] = None, int8: bool = False) -> int:
    """Splits per (sequence, KV head) for the MI355X kernel.

    Enough (sequence, head, split) units for UNITS_PER_4_CUS per 4 CUs (the
    fp16 or the INT8 walk's), never a split of fewer than MIN_SPLIT_PAGES
    pages.  Fixed by (batch, heads, pages, pool type) alone, so a captured
    graph can pin it per context bucket.
    """
    cus = _cus(device) if device is not None and torch.cuda.is_available() else 256
    units = UNITS_PER_4_CUS["int8" if int8 else "fp16"] * cus // 4
    by_cus = -(-units // max(1, batch * kv_heads))
    by_pages = max(1, num_pages // MIN_SPLIT_PAGES)
    return max(1, min(MAX_SPLITS, by_cus, by_pages))


def ineligible_reason(q: torch.Tensor, k_pool: torch.Tensor, k_scale=None, k_residual=None,
                      v_scale=None, k_zero=None, v_zero=None, res_rows=None) -> Optional[str]:
    """Why the HIP kernels cannot take these inputs, or None.

    The reference's rules (kernels/cuda/paged_decode_cuda.py:112-141) plus the
    tile shape: head_dim 128, 16-token pages, at most 16 query rows per KV head.
    """
    if not q.is_cuda or not k_pool.is_cuda:
        return "tensors are not on a GPU"
    if q.dtype != torch.float16:
        return f"q must be float16, got {q.dtype}"
    if q.dim() != 4 or q.shape[-1] != HEAD_DIM:
        return f"q must be [B, H_kv, n_rep, {HEAD_DIM}]"
    if not 1 <= q.shape[2] <= MAX_NREP:
        return f"n_rep must be in [1, {MAX_NREP}], got {q.shape[2]}"
    if k_pool.dim() != 4 or k_pool.shape[1] != PAGE or k_pool.shape[-1] != HEAD_DIM:
        return f"pools must be [num_blocks, {PAGE}, H_kv, {HEAD_DIM}]"
    if k_pool.shape[2] != q.shape[1]:
        return "q and the pools disagree on H_kv"
    if not _aligned(q, 16):
        return "q rows must be 16-byte aligned and unit-stride"
    if k_pool.dtype == torch.float16:
        if k_scale is not None or k_residual is not None:
            return "an fp16 pool takes no scales or residual"
        return None if _aligned(k_pool, 16) else "pool rows must be 16-byte aligned"
    if k_pool.dtype != torch.int8:
        return f"pools must be float16 or int8, got {k_pool.dtype}"
    if k_scale is None or v_scale is None:
        return "an INT8 pool needs k_scale and v_scale"
    if not _aligned(k_pool, 8):
        return "INT8 pool rows must be 8-byte aligned"
    if k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
        return "scales must be float32"
    if not _aligned(k_scale, 16):
        return "k_scale rows must be 16-byte aligned"
    if (k_zero is None) != (v_zero is None):
        return "k_zero and v_zero go together"
    if k_zero is not None and (k_zero.dtype != torch.float32 or k_zero.stride() != k_scale.stride()
                               or v_zero.stride() != v_scale.stride() or not _aligned(k_zero, 16)):
        return "zero points must be float32 with their scales' strides"
    if (k_residual is None) != (res_rows is None):
        return "k_residual and res_rows go together"
    if k_residual is not None and (k_residual.dtype != torch.float16 or not _aligned(k_residual, 16)
                                   or res_rows.dtype != torch.int32):
        return "k_residual must be aligned float16 and res_rows int32"
    return None


def eligible(q: torch.Tensor, k_pool: torch.Tensor, k_scale=None, k_residual=None,
             v_scale=None, k_zero=None, v_zero=None, res_rows=None) -> bool:
    """kernels/cuda/paged_decode_cuda.py:112-141, for the HIP kernels."""
    return ineligible_reason(q, k_pool, k_scale, k_residual, v_scale, k_zero, v_zero,
                             res_rows) is None


def _aligned(t: torch.Tensor, nbytes: int) -> bool:
    return (t.stride(-1) == 1 and t.data_ptr() % nbytes == 0
            and all((st * t.element_size()) % nbytes == 0 for st in t.stride()[:-1]))


def _buffers(tag: str, b: int, h: int, splits: int, n_rep: int, device):
    """Persistent output, split workspace and arrival counters for one shape
    (graph-address stable)."""
    out = scratch(f"{tag}_out", (b, h, MAX_NREP, HEAD_DIM), torch.float16, device)
    cnt = scratch(f"{tag}_cnt", (_lib.lib().ls_decode_counter_ints(b, h),), torch.int32, device,
                  init=0)
    if splits == 1:
        return out, None, cnt
    nbytes = _lib.lib().ls_decode_workspace_bytes(b, h, n_rep, splits)
    work = scratch(f"{tag}_work", (nbytes // 4,), torch.float32, device)
    return out, work, cnt


def check_out(out: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """A caller's output buffer for q [B, H_kv, n_rep, D]."""
    if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device \
            or not _aligned(out, 16):
        raise ValueError(f"out must be {q.dtype} {tuple(q.shape)} on {q.device} with 16-byte "
                         "aligned rows")
    return out


def _check_common(q, k_pool, v_pool, block_tables, seq_lens):
    if q.stride(-1) != 1 or k_pool.stride(-1) != 1 or v_pool.stride() != k_pool.stride():
        raise ValueError("the HIP kernel needs unit-stride head dims and matching K/V pools")
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("block tables and sequence lengths must be int32")
    if block_tables.stride(-1) != 1 or seq_lens.stride(-1) != 1:
        raise ValueError("block tables and sequence lengths must be unit-stride")
    if v_pool.dtype != k_pool.dtype or v_pool.shape != k_pool.shape:
        raise ValueError("K and V pools must match in dtype and shape")
    for t in (k_pool, v_pool, block_tables, seq_lens):
        if t.device != q.device:
            raise ValueError("all tensors must be on q's device")


def paged_decode_hip(q, k_pool, v_pool, block_tables, seq_lens, max_seq_len: int,
                     num_splits: Optional[int] = None,
                     softmax_scale: Optional[float] = None,
                     k_scale=None, v_scale=None, k_zero=None, v_zero=None,
                     k_residual=None, res_rows=None,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Paged decode on the HIP kernels -> [B, H_kv, n_rep, D] (q.dtype).

    kernels/cuda/paged_decode_cuda.py:202-252. The returned tensor is a view
    of a persistent buffer, overwritten by the next call of the same shape,
    or `out` when given ([B, H_kv, n_rep, D] fp16 with 16-byte aligned rows,
    e.g. a contiguous [B, H_kv * n_rep * D] buffer the output projection
    reads without a copy).
    """
    reason = ineligible_reason(q, k_pool, k_scale, k_residual, v_scale, k_zero, v_zero, res_rows)
    if reason is not None:
        raise ValueError(f"paged_decode_hip: {reason}")
    _check_common(q, k_pool, v_pool, block_tables, seq_lens)
    b, h_kv, n_rep, d = q.shape
    num_pages = -(-int(max_seq_len) // PAGE)
    splits = int(num_splits) if num_splits else choose_splits(b, h_kv, num_pages, q.device,
                                                              int8=k_pool.dtype == torch.int8)
    splits = max(1, min(MAX_SPLITS, splits))
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    is_int8 = k_pool.dtype == torch.int8
    buf, work, cnt = _buffers("hip_i8" if is_int8 else "hip", b, h_kv, splits, n_rep, q.device)
    target = buf if out is None else check_out(out, q)
    L = _lib.lib()
    P, S = _lib.ptr, _lib.strides
    common_tail = (P(target), S(target, 3), P(work), P(cnt), b, h_kv, n_rep, d, k_pool.shape[1],
                   splits, int(max_seq_len), float(scale), _lib.stream_of(q.device))
    if is_int8:
        rc = L.ls_paged_decode_int8(
            P(q), S(q, 3), P(k_pool), P(v_pool), S(k_pool, 3), k_pool.shape[0],
            P(k_scale), S(k_scale, 2), P(v_scale), S(v_scale, 3), P(k_zero), P(v_zero),
            P(k_residual), S(k_residual, 3), 0 if k_residual is None else k_residual.shape[0],
            P(res_rows), P(block_tables), block_tables.stride(0), block_tables.shape[1],
            P(seq_lens), *common_tail)
        _lib.check(rc, "ls_paged_decode_int8")
    else:
        rc = L.ls_paged_decode_fp16(
            P(q), S(q, 3), P(k_pool), P(v_pool), S(k_pool, 3), k_pool.shape[0],
            P(block_tables), block_tables.stride(0), block_tables.shape[1], P(seq_lens),
            *common_tail)
        _lib.check(rc, "ls_paged_decode_fp16")
    return buf[:, :, :n_rep] if out is None else out


def paged_decode_cuda(q, k_pool, v_pool, block_tables, seq_lens, max_seq_len: int,
                      num_splits: Optional[int] = None,
                      softmax_scale: Optional[float] = None,
                      k_scale=None, v_scale=None, k_zero=None, v_zero=None,
                      k_residual=None, res_rows=None,
                      min_blocks: Optional[int] = None) -> torch.Tensor:
    """The reference's launcher name and signature
    (kernels/cuda/paged_decode_cuda.py:202-207), on the HIP kernels.

    ``min_blocks`` is accepted and has no effect: the reference passes it to
    NVRTC as the INT8 kernel's minimum resident blocks (a register cap);
    these kernels are built ahead of time with fixed launch bounds (one
    workgroup of 8 waves a CU), reported by ``kernel_resources``.
    """
    del min_blocks
    return paged_decode_hip(q, k_pool, v_pool, block_tables, seq_lens, max_seq_len,
                            num_splits=num_splits, softmax_scale=softmax_scale,
                            k_scale=k_scale, v_scale=v_scale, k_zero=k_zero, v_zero=v_zero,
                            k_residual=k_residual, res_rows=res_rows)


def kernel_resources(device: Optional[torch.device] = None, head_dim: int = HEAD_DIM,
                     n_rep: int = 6, page: int = PAGE, variant: str = "fp16",
                     asym: bool = False, has_res: bool = False,
                     min_blocks: Optional[int] = None, kv_heads: int = 2) -> dict:
    """Registers, private (spill) memory and LDS of the loaded decode kernel
    that a launch with these properties runs, as the HIP runtime reports
    them (kernels/cuda/paged_decode_cuda.py:163-186, which asks the CUDA
    driver): ``regs`` (vector registers a lane), ``local_bytes`` (0: no
    spills), ``shared_bytes``, plus ``threads`` (a workgroup) and
    ``groups_per_cu`` (occupancy).  ``min_blocks`` has no effect here (see
    paged_decode_cuda); ``kv_heads`` chooses the paired-head kernel (even)
    or the one-head kernel (odd).
    """
    del min_blocks
    if head_dim != HEAD_DIM or page != PAGE or not 1 <= n_rep <= MAX_NREP:
        raise ValueError(f"the HIP kernels are built for head_dim {HEAD_DIM}, page {PAGE} and "
                         f"n_rep 1..{MAX_NREP}")
    names = {"fp16": "paged_decode_fp16", "int8": "paged_decode_int8"}
    if variant not in names:
        raise ValueError(f"variant must be 'fp16' or 'int8', got {variant!r}")
    return _lib.kernel_resources(names[variant], device, kv_heads=kv_heads, n_rep=n_rep,
                                 asym=asym, has_res=has_res)


def combine_splits_hip(partial_acc: torch.Tensor, partial_m: torch.Tensor,
                       partial_l: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """combine_splits (kernels/gqa/paged_decode.py:689-706) as one HIP launch.

    partial_acc [B, H, S, N_REP, D] fp32, partial_m/l [B, H, S, N_REP] fp32
    (natural-log maxima) -> [B, H, N_REP, D] in out_dtype (fp16 or fp32).
    """
    if out_dtype not in (torch.float16, torch.float32):
        raise ValueError("out_dtype must be float16 or float32")
    for t in (partial_acc, partial_m, partial_l):
        if t.dtype != torch.float32 or not t.is_cuda:
            raise ValueError("partials must be float32 GPU tensors")
    if partial_m.stride() != partial_l.stride() or partial_m.stride(-1) != 1 \
            or partial_acc.stride(-1) != 1:
        raise ValueError("m and l must share strides; rows and channels unit-stride")
    b, h, s, nr, d = partial_acc.shape
    out = torch.empty((b, h, nr, d), dtype=out_dtype, device=partial_acc.device)
    rc = _lib.lib().ls_combine_splits(
        _lib.ptr(partial_acc), _lib.strides(partial_acc, 4), _lib.ptr(partial_m),
        _lib.ptr(partial_l), _lib.strides(partial_m, 3), _lib.ptr(out),
        1 if out_dtype == torch.float32 else 0, _lib.strides(out, 3), b, h, s, nr, d,
        _lib.stream_of(partial_acc.device))
    _lib.check(rc, "ls_combine_splits")
    return out
