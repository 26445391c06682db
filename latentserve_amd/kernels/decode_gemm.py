"""Projections of the decode step on the HIP weight-streaming GEMM.

``gate_up_silu(x, weight)`` is the MLP's gate/up projection with
silu_and_mul (kernels/fused_elementwise.py:222-233) in the GEMM's
epilogue: one launch, bit-equal to ``linear`` followed by the separate
activation kernel.  ``qkv_rope_write(x, w_qkv, bias, ...)`` is the attention
layer's fused q/k/v projection finished in its epilogue exactly as
``fused_elementwise.rope_write_decode`` finishes it (RoPE, the query fold,
the K/V store and page bounds): one launch, bit-equal to the two.

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


KINDS = {"plain": 0, "gate_up": 1, "qkv": 2}


class PackedWeight:
    """A projection weight [N, K] packed for its launch kind (ls_pack_gemm_weight):
    every weight load then reads 1 KiB contiguous.  ``kind``: "plain" for
    linear, "gate_up" for gate_up_silu, "qkv" for qkv_rope_write (with the
    head width)."""

    def __init__(self, weight: torch.Tensor, kind: str = "plain", head_dim: int = 128):
        if not weight.is_cuda or weight.dtype != torch.float16 or weight.dim() != 2:
            raise ValueError("weight must be a 2-D fp16 GPU tensor")
        if weight.stride(-1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
            weight = weight.contiguous()
        n, k = weight.shape
        nbytes = int(_lib.lib().ls_gemm_packed_bytes(n, k, KINDS[kind], head_dim))
        if nbytes == 0:
            raise ValueError(f"cannot pack a [{n}, {k}] weight (K must be a multiple of 32)")
        self.data = torch.empty(nbytes // 2, dtype=torch.float16, device=weight.device)
        rc = _lib.lib().ls_pack_gemm_weight(weight.data_ptr(), weight.stride(0), n, k,
                                            KINDS[kind], head_dim, self.data.data_ptr(),
                                            torch.cuda.current_stream(weight.device).cuda_stream)
        _lib.check(rc, "ls_pack_gemm_weight")
        self.shape = (n, k)
        self.kind = kind
        self.head_dim = head_dim
        self.device = weight.device
        self.dtype = weight.dtype


def _weight_args(weight, kind: str):
    """(pointer, row stride, packed flag, [N, K]) of a tensor or PackedWeight."""
    if isinstance(weight, PackedWeight):
        if weight.kind != kind:
            raise ValueError(f"weight packed for {weight.kind!r}, used for {kind!r}")
        return weight.data.data_ptr(), 0, 1, weight.shape
    return weight.data_ptr(), weight.stride(0), 0, tuple(weight.shape)


def _norm_args(x2: torch.Tensor, m: int, k: int, residual, norm_weight, eps, res_out):
    """ctypes arguments of the norm prologue, and the res_out it writes.

    norm_weight None: no prologue (x is the operand).  Otherwise the operand
    is rms_norm(x + residual) with norm_weight and eps, and x + residual goes
    to res_out (allocated when None; it may not overlap x or residual)."""
    if norm_weight is None:
        return (None, 0, None, 0.0, None, 0), None
    if residual is None:
        raise ValueError("the norm prologue needs the residual")
    r2 = residual.reshape(-1, k)
    for name, t in (("residual", r2), ("norm_weight", norm_weight)):
        if not t.is_cuda or t.dtype != torch.float16:
            raise ValueError(f"{name} must be fp16 on the GPU")
    if r2.shape[0] != m or norm_weight.shape != (k,) or not norm_weight.is_contiguous():
        raise ValueError(f"residual must be [{m}, {k}] and norm_weight contiguous [{k}]")
    if r2.stride(-1) != 1 or (m > 1 and r2.stride(0) % 8) or r2.data_ptr() % 16:
        r2 = r2.contiguous()
    ro = torch.empty((m, k), dtype=x2.dtype, device=x2.device) if res_out is None \
        else res_out.view(m, k)
    return (r2.data_ptr(), r2.stride(0) if m > 1 else k, norm_weight.data_ptr(), float(eps),
            ro.data_ptr(), ro.stride(0) if m > 1 else k), ro


def supports(x: torch.Tensor, weight) -> bool:
    """Whether ``linear`` takes these operands without a copy."""
    if isinstance(weight, PackedWeight):
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        return (x.is_cuda and x.dtype == torch.float16 and rows <= MAX_ROWS
                and x.shape[-1] == weight.shape[1] and x.shape[-1] % 32 == 0)
    rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
    return (x.is_cuda and weight.is_cuda and x.dtype == weight.dtype == torch.float16
            and rows <= MAX_ROWS and x.shape[-1] % 32 == 0 and weight.dim() == 2
            and weight.stride(-1) == 1 and weight.stride(0) % 8 == 0
            and weight.data_ptr() % 16 == 0)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
           norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
           res_out: Optional[torch.Tensor] = None):
    """y = x . weight^T (+ bias) for x [..., K] fp16 with at most 64 rows.

    With norm_weight (a packed weight, at most 16 rows): y = rms_norm(x +
    residual) . weight^T (+ bias) in one launch, returning (y, x +
    residual)."""
    for name, t in (("x", x), ("weight", weight)):
        if not t.device.type == "cuda":
            raise ValueError(f"{name} must be on a GPU (the HIP kernels have no CPU path)")
        if t.dtype != torch.float16:
            raise ValueError(f"{name} must be float16, got {t.dtype}")
    wptr, wstride, packed, wshape = _weight_args(weight, "plain")
    if len(wshape) != 2 or wshape[1] != x.shape[-1]:
        raise ValueError(f"weight must be [N, {x.shape[-1]}], got {tuple(wshape)}")
    n, k = wshape
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
    nargs, ro = _norm_args(x2, m, k, residual, norm_weight, eps, res_out)
    if m == 0 or n == 0:
        return y.view(*x.shape[:-1], n) if ro is None else (y.view(*x.shape[:-1], n), ro)
    need = workspace_bytes(m, n, k)
    ws = _workspace(x.device, need) if need else None
    rc = _lib.lib().ls_decode_gemm(
        x2.data_ptr(), x2.stride(0) if m > 1 else k, wptr, wstride, packed,
        None if bias is None else bias.data_ptr(), y.data_ptr(),
        y.stride(0) if m > 1 else n, m, n, k, None if ws is None else ws.data_ptr(), need,
        *nargs, torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(rc, "ls_decode_gemm")
    y = y.view(*x.shape[:-1], n)
    return y if ro is None else (y, ro)


def gate_up_silu(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
                 norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                 res_out: Optional[torch.Tensor] = None):
    """silu(x . Wg^T) * (x . Wu^T) for weight = [Wg; Wu] [2I, K]: [..., I].

    With norm_weight, x is first replaced by rms_norm(x + residual) in the
    same launch, and (y, x + residual) is returned (as linear).

    One launch where the product needs no split of K over workgroups;
    otherwise the GEMM and then the activation kernel (still HIP, same
    rounding)."""
    from latentserve_amd.kernels import fused_elementwise as fe
    for name, t in (("x", x), ("weight", weight)):
        if not t.device.type == "cuda":
            raise ValueError(f"{name} must be on a GPU (the HIP kernels have no CPU path)")
        if t.dtype != torch.float16:
            raise ValueError(f"{name} must be float16, got {t.dtype}")
    wptr, wstride, packed, wshape = _weight_args(weight, "gate_up")
    if len(wshape) != 2 or wshape[1] != x.shape[-1] or wshape[0] % 2:
        raise ValueError(f"weight must be [2I, {x.shape[-1]}], got {tuple(wshape)}")
    n2, k = wshape
    inter = n2 // 2
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) % 8) or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if m > MAX_ROWS:
        raise ValueError(f"at most {MAX_ROWS} rows a call, got {m}")
    if m and inter and workspace_bytes(m, n2, k):
        if packed or norm_weight is not None:
            raise ValueError("this K splits over workgroups: pass the row-major weight")
        return fe.silu_and_mul(linear(x, weight, bias), out=out)
    if bias is not None and (bias.shape != (n2,) or bias.dtype != torch.float16
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be contiguous fp16 [{n2}]")
    y = torch.empty((m, inter), dtype=x.dtype, device=x.device) if out is None \
        else out.view(m, inter)
    nargs, ro = _norm_args(x2, m, k, residual, norm_weight, eps, res_out)
    if m == 0 or inter == 0:
        y = y.view(*x.shape[:-1], inter)
        return y if ro is None else (y, ro)
    rc = _lib.lib().ls_decode_gate_up_silu(
        x2.data_ptr(), x2.stride(0) if m > 1 else k, wptr, wstride, packed,
        None if bias is None else bias.data_ptr(), y.data_ptr(),
        y.stride(0) if m > 1 else inter, m, inter, k, *nargs,
        torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(rc, "ls_decode_gate_up_silu")
    y = y.view(*x.shape[:-1], inter)
    return y if ro is None else (y, ro)


def qkv_rope_write(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                   positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                   slots: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, hq: int,
                   hk: int, q_out: Optional[torch.Tensor] = None,
                   kmin: Optional[torch.Tensor] = None,
                   kmax: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
                   norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                   res_out: Optional[torch.Tensor] = None):
    """rope_write_decode(linear(x, weight, bias), ...) in one launch.

    With norm_weight, x is first replaced by rms_norm(x + residual) in the
    same launch, and (q, x + residual) is returned.

    x [B, K] (or [B, 1, K]) fp16; weight [(hq + 2 hk) * D, K]; the rest as
    fused_elementwise.rope_write_decode.  Returns q folded to [B, hk, hq //
    hk, D] (q_out when given).  Where the GEMM would split K over
    workgroups, the two launches run instead (same results)."""
    from latentserve_amd.kernels import fused_elementwise as fe
    for name, t in (("x", x), ("weight", weight)):
        if not t.device.type == "cuda":
            raise ValueError(f"{name} must be on a GPU (the HIP kernels have no CPU path)")
        if t.dtype != torch.float16:
            raise ValueError(f"{name} must be float16, got {t.dtype}")
    wptr, wstride, packed, (n, k) = _weight_args(weight, "qkv")
    b = x.shape[0]
    x2 = x.reshape(b, k)
    if x2.stride(-1) != 1 or (b > 1 and x2.stride(0) % 8) or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    d = cos.shape[-1]
    two = (n != (hq + 2 * hk) * d or d % 16 or b > MAX_ROWS or not supports(x2, weight)
           or (b and workspace_bytes(b, n, k)))
    if two:
        if packed or norm_weight is not None:
            raise ValueError("this shape takes two launches: pass the row-major weight")
        return fe.rope_write_decode(linear(x2, weight, bias), positions, cos, sin, slots, k_pool,
                                    v_pool, hq, hk, q_out=q_out, kmin=kmin, kmax=kmax)
    if packed and weight.head_dim != d:
        raise ValueError(f"weight packed for head_dim {weight.head_dim}, tables are {d} wide")
    if bias is not None and (bias.shape != (n,) or bias.dtype != torch.float16
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be contiguous fp16 [{n}]")
    args = fe.rope_write_args(positions, cos, sin, slots, k_pool, v_pool, hq, hk, b, d, q_out,
                              kmin, kmax)
    nargs, ro = _norm_args(x2, b, k, residual, norm_weight, eps, res_out)
    rc = _lib.lib().ls_decode_qkv_rope_write(
        x2.data_ptr(), x2.stride(0) if b > 1 else k, wptr, wstride, packed,
        None if bias is None else bias.data_ptr(), k, *args["pre"], b, hq, hk, d, *nargs,
        torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(rc, "ls_decode_qkv_rope_write")
    return args["q_out"] if ro is None else (args["q_out"], ro)
