"""Projections of the decode step on the HIP weight-streaming GEMM.

``gate_up_silu(x, weight)`` is the MLP's gate/up projection with
silu_and_mul (kernels/fused_elementwise.py:222-233) in the GEMM's
epilogue: one launch, bit-equal to ``linear`` followed by the separate
activation kernel.

``linear(x, weight, bias)`` computes what torch.nn.functional.linear does
for fp16 operands (x [..., K], weight [N, K] as a torch Linear holds it),
with fp32 sums and one rounding to fp16 after the bias add.  The reference's
decoder layers run these projections as torch Linear modules
(model/latentserve_qwen.py, model/fused.py); at decode batch sizes each one
is a single pass over its weight matrix, which the HIP kernel streams with
K split over waves where the output width alone would not fill the chip.

Only the HIP kernel runs here: a CPU tensor, more than ``MAX_ROWS`` rows or
a shape the kernel does not take raises; nothing falls back to torch.
"""

from __future__ import annotations

from typing import Optional

import torch

from latentserve_amd import _lib

# Rows (tokens) one launch takes.
MAX_ROWS = 64


_WORKSPACE: dict = {}
# Buffers replaced by larger ones stay allocated: a captured graph keeps the
# address it was recorded with.
_RETIRED: list = []


def workspace_bytes(m: int, n: int, k: int) -> int:
    """Bytes of fp32 partial sums an [m, n, k] product needs (0: none)."""
    return int(_lib.lib().ls_decode_gemm_workspace_bytes(m, n, k))


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """One partial-sum buffer a device, grown to the largest product seen.

    Launches that share it are ordered on the current stream.  A buffer that
    is outgrown is kept, never freed, so graphs captured with it stay valid.
    """
    key = torch.device(device).index
    buf = _WORKSPACE.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _RETIRED.append(buf)
        # zero-filled: the arrival counters start at zero (and calls leave
        # them so)
        buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACE[key] = buf
    return buf


def supports(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether ``linear`` takes these operands without a copy."""
    rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
    return (x.is_cuda and weight.is_cuda and x.dtype == weight.dtype == torch.float16
            and rows <= MAX_ROWS and x.shape[-1] % 32 == 0 and weight.dim() == 2
            and weight.stride(-1) == 1 and weight.stride(0) % 8 == 0
            and weight.data_ptr() % 16 == 0)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x . weight^T (+ bias) for x [..., K] fp16 with at most 64 rows."""
    for name, t in (("x", x), ("weight", weight)):
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a GPU (the HIP kernels have no CPU path)")
        if t.dtype != torch.float16:
            raise ValueError(f"{name} must be float16, got {t.dtype}")
    if weight.dim() != 2 or weight.shape[1] != x.shape[-1]:
        raise ValueError(f"weight must be [N, {x.shape[-1]}], got {tuple(weight.shape)}")
    n, k = weight.shape
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) % 8) or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if m > MAX_ROWS:
        raise ValueError(f"at most {MAX_ROWS} rows a call, got {m}")
    if bias is not None and (bias.shape != (n,) or bias.dtype != torch.float16
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be contiguous fp16 [{n}]")
    y = torch.empty((m, n), dtype=x.dtype, device=x.device) if out is None else out.view(m, n)
    if m == 0 or n == 0:
        return y.view(*x.shape[:-1], n)
    need = workspace_bytes(m, n, k)
    ws = _workspace(x.device, need) if need else None
    rc = _lib.lib().ls_decode_gemm(
        x2.data_ptr(), x2.stride(0) if m > 1 else k, weight.data_ptr(), weight.stride(0),
        None if bias is None else bias.data_ptr(), y.data_ptr(),
        y.stride(0) if m > 1 else n, m, n, k, None if ws is None else ws.data_ptr(), need,
        torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(rc, "ls_decode_gemm")
    return y.view(*x.shape[:-1], n)


def gate_up_silu(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(x . Wg^T) * (x . Wu^T) for weight = [Wg; Wu] [2I, K]: [..., I].

    One launch where the product needs no split of K over workgroups;
    otherwise the GEMM and then the activation kernel (still HIP, same
    rounding)."""
    from latentserve_amd.kernels import fused_elementwise as fe
    for name, t in (("x", x), ("weight", weight)):
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a GPU (the HIP kernels have no CPU path)")
        if t.dtype != torch.float16:
            raise ValueError(f"{name} must be float16, got {t.dtype}")
    if weight.dim() != 2 or weight.shape[1] != x.shape[-1] or weight.shape[0] % 2:
        raise ValueError(f"weight must be [2I, {x.shape[-1]}], got {tuple(weight.shape)}")
    n2, k = weight.shape
    inter = n2 // 2
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) % 8) or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if m > MAX_ROWS:
        raise ValueError(f"at most {MAX_ROWS} rows a call, got {m}")
    if m and inter and workspace_bytes(m, n2, k):
        return fe.silu_and_mul(linear(x, weight, bias), out=out)
    if bias is not None and (bias.shape != (n2,) or bias.dtype != torch.float16
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be contiguous fp16 [{n2}]")
    y = torch.empty((m, inter), dtype=x.dtype, device=x.device) if out is None \
        else out.view(m, inter)
    if m == 0 or inter == 0:
        return y.view(*x.shape[:-1], inter)
    rc = _lib.lib().ls_decode_gate_up_silu(
        x2.data_ptr(), x2.stride(0) if m > 1 else k, weight.data_ptr(), weight.stride(0),
        None if bias is None else bias.data_ptr(), y.data_ptr(),
        y.stride(0) if m > 1 else inter, m, inter, k,
        torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(rc, "ls_decode_gate_up_silu")
    return y.view(*x.shape[:-1], inter)
