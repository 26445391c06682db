"""INT8 KV cache write side on HIP kernels.

Mirrors the reference's kernels/cuda/int8_write.py: ``eligible`` (:53-58) and
``decode_write`` (:61-82), the fused decode-step write (V's per-token
quantize and scatter, K's scatter into the fp16 last-page residual), plus
``finalize_blocks``, the per-block K quantizer of
Int8PagedKVCache._finalize_blocks (cache/int8_paged_cache.py:670-699), so a
completed page is quantized on the GPU too.

Codes and scales are bit-exact with the reference's torch ops.  Torch
divides by a Python number differently on the two devices (GPU: times the
fp32 reciprocal formed on the host; CPU: a true division); ``exact_division``
picks the CPU form, the default is the GPU form, which is what the reference
stores when it runs on a GPU and what its int8_write.cu computes.
"""

from __future__ import annotations

from typing import Optional

import torch

from latentserve_amd import _lib

HEAD_DIM = 128
PAGE = 16


def eligible(k: torch.Tensor, v: torch.Tensor) -> bool:
    """One token per sequence, fp16, head_dim 128, channels unit-stride."""
    return (k.is_cuda and v.is_cuda and k.dtype == v.dtype == torch.float16
            and k.dim() == 4 and v.dim() == 4 and k.shape[2] == 1 and v.shape[2] == 1
            and k.shape[-1] == HEAD_DIM and v.shape[-1] == HEAD_DIM
            and k.stride(-1) == 1 and v.stride(-1) == 1)


def _contig(t: torch.Tensor, name: str) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def decode_write(k, v, slots, res_idx, flat_v, flat_v_scale, flat_v_zero, k_res, *,
                 asym: bool, eps: float, qmax: float, levels: float, offset: float,
                 exact_division: bool = False) -> None:
    """k, v [B, H, 1, D] fp16; slots, res_idx [B] int64 flat indices;
    flat_v [S, H, D] int8, flat_v_scale / flat_v_zero [S, H] fp32;
    k_res [R, H, D] fp16.  Rows outside [0, S) / [0, R) are skipped."""
    if not eligible(k, v):
        raise ValueError("decode_write: k and v must be fp16 [B, H, 1, 128] GPU tensors")
    b, h, _, d = k.shape
    for t, name in ((slots, "slots"), (res_idx, "res_idx")):
        if t.dtype != torch.int64 or t.dim() != 1 or t.shape[0] < b or t.stride(0) != 1:
            raise ValueError(f"{name} must be a unit-stride int64 [B] tensor")
    if flat_v.dtype != torch.int8 or flat_v.shape[1:] != (h, d):
        raise ValueError("flat_v must be int8 [S, H, D]")
    if flat_v_scale.dtype != torch.float32 or flat_v_scale.shape != flat_v.shape[:2]:
        raise ValueError("flat_v_scale must be fp32 [S, H]")
    if asym and (flat_v_zero is None or flat_v_zero.shape != flat_v_scale.shape
                 or flat_v_zero.dtype != torch.float32):
        raise ValueError("asymmetric quantization needs flat_v_zero fp32 [S, H]")
    if k_res.dtype != torch.float16 or k_res.shape[1:] != (h, d):
        raise ValueError("k_res must be fp16 [R, H, D]")
    for t, name in ((flat_v, "flat_v"), (flat_v_scale, "flat_v_scale"), (k_res, "k_res")):
        _contig(t, name)
    if asym:
        _contig(flat_v_zero, "flat_v_zero")
    P, S = _lib.ptr, _lib.strides
    k2, v2 = k[:, :, 0], v[:, :, 0]
    rc = _lib.lib().ls_int8_decode_write(
        P(k2), S(k2, 2), P(v2), S(v2, 2), P(slots), P(res_idx), P(flat_v), P(flat_v_scale),
        P(flat_v_zero) if asym else None, P(k_res), flat_v.shape[0], k_res.shape[0], b, h, d,
        int(bool(asym)), float(eps), float(qmax), float(levels), float(offset),
        0 if exact_division else 1, _lib.stream_of(k.device))
    _lib.check(rc, "ls_int8_decode_write")


def finalize_blocks(data: torch.Tensor, ids: torch.Tensor, k_pool: torch.Tensor,
                    k_scale: torch.Tensor, k_zero: Optional[torch.Tensor] = None, *,
                    asym: bool, eps: float, qmax: float, levels: float, offset: float,
                    exact_division: bool = False) -> None:
    """Quantize data [N, 16, H, D] fp16 into k_pool blocks ids [N] (int64):
    one step per (block, head, channel), written to k_scale [nb, H, D] (and
    the zero point to k_zero when asym).  Ids outside the pool are skipped."""
    if data.dtype != torch.float16 or data.dim() != 4 or data.shape[1] != PAGE \
            or data.shape[-1] != HEAD_DIM or data.stride(-1) != 1:
        raise ValueError("data must be fp16 [N, 16, H, 128] with unit channel stride")
    n, _, h, d = data.shape
    if ids.dtype != torch.int64 or ids.dim() != 1 or ids.shape[0] != n or ids.stride(0) != 1:
        raise ValueError("ids must be a unit-stride int64 [N] tensor")
    if k_pool.dtype != torch.int8 or k_pool.shape[1:] != (PAGE, h, d) or k_pool.stride(-1) != 1:
        raise ValueError("k_pool must be int8 [nb, 16, H, D]")
    nb = k_pool.shape[0]
    if k_scale.dtype != torch.float32 or k_scale.shape != (nb, h, d) or k_scale.stride(-1) != 1:
        raise ValueError("k_scale must be fp32 [nb, H, D]")
    if asym and (k_zero is None or k_zero.shape != k_scale.shape
                 or k_zero.stride() != k_scale.stride() or k_zero.dtype != torch.float32):
        raise ValueError("asymmetric quantization needs k_zero shaped and strided as k_scale")
    P, S = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_int8_finalize_blocks(
        P(data), S(data, 3), P(ids), n, P(k_pool), S(k_pool, 3), P(k_scale),
        P(k_zero) if asym else None, S(k_scale, 2), nb, h, d, PAGE, int(bool(asym)), float(eps),
        float(qmax), float(levels), float(offset), 0 if exact_division else 1,
        _lib.stream_of(data.device))
    _lib.check(rc, "ls_int8_finalize_blocks")
