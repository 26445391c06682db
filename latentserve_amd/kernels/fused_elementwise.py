"""Fused elementwise ops of the decode step on the HIP kernels.

Mirrors the reference's kernels/fused_elementwise.py: the same functions
(``rms_norm`` :194-205, ``fused_add_rms_norm`` :207-220, ``silu_and_mul``
:222-233, ``rope_qk`` :235-252) and their Hugging Face references
(``rms_norm_ref`` :75-80, ``fused_add_rms_norm_ref`` :83-85,
``silu_and_mul_ref`` :88-90, ``rope_qk_ref`` :98-110), which stay plain torch
as the reference has them.  The dispatching functions run only the HIP
kernels: a CPU tensor or a missing library raises, nothing falls back to the
references.

``embed_rms_norm`` is the token embedding lookup and the first layer's
input norm in one launch; ``argmax_rows`` is torch.argmax over the last
dimension (the greedy next token).

``rope_write_decode`` has no single counterpart: it is the decode layer's
rope_qk (model/attention/gqa.py:251-253), its paged store of the new K/V rows
(cache/paged_cache.py write, with the page K bounds of :457-460) and the fold
of q to [B, H_kv, n_rep, D] (gqa.py:290-341) in one launch.

Each kernel rounds to fp16 where Hugging Face's fp16 computation does: the
residual sum is one fp16 add, the normalised value is cast to fp16 before
the weight multiply, RoPE rounds both products and their sum.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
import torch.nn.functional as F

from latentserve_amd import _lib

# ----------------------------------------------------------------------
# References: the Hugging Face computation (torch, any device)
# ----------------------------------------------------------------------


def rms_norm_ref(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    dtype = x.dtype
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return weight * h.to(dtype)


def fused_add_rms_norm_ref(x, residual, weight, eps):
    s = residual + x
    return rms_norm_ref(s, weight, eps), s


def silu_and_mul_ref(gate_up: torch.Tensor) -> torch.Tensor:
    gate, up = gate_up.chunk(2, dim=-1)
    return F.silu(gate) * up


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def rope_qk_ref(q, k, cos, sin, hq: int, hk: int, d: int):
    """q [B, S, HQ*D], k [B, S, HK*D], cos/sin [B or 1, 1, S, D]."""
    b, s = q.shape[0], q.shape[1]
    c = cos.reshape(cos.shape[0], s, 1, d)
    sn = sin.reshape(sin.shape[0], s, 1, d)
    q4 = q.reshape(b, s, hq, d)
    k4 = k.reshape(b, s, hk, d)
    qo = (q4 * c) + (_rotate_half(q4) * sn)
    ko = (k4 * c) + (_rotate_half(k4) * sn)
    return qo.reshape(b, s, hq * d), ko.reshape(b, s, hk * d)


# ----------------------------------------------------------------------
# HIP dispatch
# ----------------------------------------------------------------------


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _fp16_gpu(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU (the HIP kernels have no CPU path)")
    if t.dtype != torch.float16:
        raise ValueError(f"{name} must be float16, got {t.dtype}")
    if t.dim() >= 1 and t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit stride in its last dimension")


def _rows(t: torch.Tensor) -> torch.Tensor:
    """[..., n] -> a [rows, n] view (a copy only when the leading dims do not
    merge)."""
    r = t.reshape(-1, t.shape[-1])
    return r if r.stride(-1) == 1 else r.contiguous()


def _row_stride(t: torch.Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else t.shape[-1]


def _norm(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
          out: Optional[torch.Tensor] = None, res_out: Optional[torch.Tensor] = None):
    _fp16_gpu("x", x)
    _fp16_gpu("weight", weight)
    if weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(f"weight must be [{x.shape[-1]}], got {tuple(weight.shape)}")
    x2 = _rows(x)
    y = torch.empty_like(x2) if out is None else out.view(x2.shape)
    r2 = ro = None
    if residual is not None:
        _fp16_gpu("residual", residual)
        if residual.shape != x.shape:
            raise ValueError("residual must have x's shape")
        r2 = _rows(residual)
        ro = torch.empty_like(x2) if res_out is None else res_out.view(x2.shape)
    rc = _lib.lib().ls_rms_norm(
        x2.data_ptr(), _row_stride(x2), None if r2 is None else r2.data_ptr(),
        0 if r2 is None else _row_stride(r2), weight.data_ptr(), y.data_ptr(), _row_stride(y),
        None if ro is None else ro.data_ptr(), 0 if ro is None else _row_stride(ro),
        x2.shape[0], x2.shape[1], float(eps), _stream(x))
    _lib.check(rc, "ls_rms_norm")
    if residual is None:
        return y.view(x.shape)
    return y.view(x.shape), ro.view(x.shape)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Qwen2 RMSNorm of the last axis in one launch."""
    return _norm(x, None, weight, eps, out)


def fused_add_rms_norm(x, residual, weight, eps, out: Optional[torch.Tensor] = None,
                       res_out: Optional[torch.Tensor] = None):
    """(norm(residual + x), residual + x) in one kernel."""
    return _norm(x, residual, weight, eps, out, res_out)


def silu_and_mul(gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    _fp16_gpu("gate_up", gate_up)
    if gate_up.shape[-1] % 2:
        raise ValueError("gate_up's last dimension must be even")
    gu = _rows(gate_up)
    inter = gu.shape[-1] // 2
    o = torch.empty((gu.shape[0], inter), dtype=gu.dtype, device=gu.device) if out is None \
        else out.view(gu.shape[0], inter)
    rc = _lib.lib().ls_silu_and_mul(gu.data_ptr(), _row_stride(gu), o.data_ptr(), _row_stride(o),
                                    gu.shape[0], inter, _stream(gu))
    _lib.check(rc, "ls_silu_and_mul")
    return o.reshape(*gate_up.shape[:-1], inter)


def rope_qk(q, k, cos, sin, hq: int, hk: int, d: int):
    """RoPE on q and k in one launch, on the [B, S, H*D] layout the fused
    projection produces — before the transpose to [B, H, S, D]."""
    for name, t in (("q", q), ("k", k), ("cos", cos), ("sin", sin)):
        _fp16_gpu(name, t)
    b, s = q.shape[0], q.shape[1]
    q2 = _rows(q.reshape(b * s, hq * d))
    k2 = _rows(k.reshape(b * s, hk * d))
    c2 = _rows(cos.expand(b, 1, s, d).reshape(b * s, d))
    s2 = _rows(sin.expand(b, 1, s, d).reshape(b * s, d))
    qo = torch.empty((b * s, hq * d), dtype=q.dtype, device=q.device)
    ko = torch.empty((b * s, hk * d), dtype=k.dtype, device=k.device)
    rows = b * s
    rc = _lib.lib().ls_rope_qk(
        q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0), c2.data_ptr(),
        c2.stride(0) if rows > 1 else 0, s2.data_ptr(), s2.stride(0) if rows > 1 else 0,
        qo.data_ptr(), qo.stride(0), ko.data_ptr(), ko.stride(0), rows, hq, hk, d, _stream(q))
    _lib.check(rc, "ls_rope_qk")
    return qo.reshape(b, s, hq * d), ko.reshape(b, s, hk * d)


def _i64p(vals):
    return (ctypes.c_int64 * len(vals))(*vals)


def rope_write_decode(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                      sin: torch.Tensor, slots: torch.Tensor, k_pool: torch.Tensor,
                      v_pool: torch.Tensor, hq: int, hk: int,
                      q_out: Optional[torch.Tensor] = None,
                      kmin: Optional[torch.Tensor] = None,
                      kmax: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The decode token's attention inputs from the fused projection output.

    qkv [B, (hq + 2 hk) * D] (or [B, 1, ...]) fp16; positions / slots [B]
    (or [B, 1]) int64; cos / sin [max_pos, D] fp16 tables; k_pool / v_pool
    [nb, page, hk, D].  Returns q rotated and folded to [B, hk, hq // hk, D]
    (into q_out when given); the rotated key and the value are stored at the
    slots, and the page K bounds kmin / kmax [nb, hk, D] updated when given.
    Positions past the table are clamped to its last row (the caller builds
    the tables to the cache's capacity).
    """
    _fp16_gpu("qkv", qkv)
    b = qkv.shape[0]
    d = cos.shape[-1]
    q2 = _rows(qkv.reshape(b, -1))
    if q2.shape[1] != (hq + 2 * hk) * d:
        raise ValueError(f"qkv rows must hold {(hq + 2 * hk) * d} values, got {q2.shape[1]}")
    args = rope_write_args(positions, cos, sin, slots, k_pool, v_pool, hq, hk, b, d, q_out, kmin,
                           kmax)
    rc = _lib.lib().ls_rope_write_decode(q2.data_ptr(), _row_stride(q2), *args["pre"], b, hq, hk,
                                         d, _stream(qkv))
    _lib.check(rc, "ls_rope_write_decode")
    return args["q_out"]


def rope_write_args(positions, cos, sin, slots, k_pool, v_pool, hq: int, hk: int, b: int, d: int,
                    q_out=None, kmin=None, kmax=None) -> dict:
    """Checked C arguments shared by the decode-token writers: "pre" holds
    positions .. bounds strides in ABI order, "q_out" the output."""
    for name, t in (("cos", cos), ("sin", sin), ("k_pool", k_pool), ("v_pool", v_pool)):
        _fp16_gpu(name, t)
    pos = positions.reshape(b)
    sl = slots.reshape(b)
    for name, t in (("positions", pos), ("slots", sl)):
        if t.dtype != torch.int64 or not t.is_cuda:
            raise ValueError(f"{name} must be int64 on the GPU")
    if not pos.is_contiguous() or not sl.is_contiguous():
        raise ValueError("positions and slots must be contiguous")
    if cos.dim() != 2 or cos.shape != sin.shape or cos.stride() != sin.stride():
        raise ValueError("cos / sin must be matching [max_pos, D] tables")
    if k_pool.dim() != 4 or k_pool.shape != v_pool.shape or k_pool.stride() != v_pool.stride() \
            or k_pool.shape[2] != hk or k_pool.shape[3] != d:
        raise ValueError(f"k_pool / v_pool must be matching [nb, page, {hk}, {d}] pools")
    n_rep = hq // hk
    if q_out is None:
        q_out = torch.empty((b, hk, n_rep, d), dtype=torch.float16, device=k_pool.device)
    elif q_out.shape != (b, hk, n_rep, d) or q_out.stride(-1) != 1 or q_out.dtype != torch.float16:
        raise ValueError(f"q_out must be fp16 [{b}, {hk}, {n_rep}, {d}] with unit last stride")
    bounds = None
    if kmin is not None:
        if kmax is None or kmin.shape != (k_pool.shape[0], hk, d) or kmax.shape != kmin.shape \
                or kmin.stride() != kmax.stride() or kmin.stride(-1) != 1 \
                or kmin.dtype != torch.float16 or kmax.dtype != torch.float16:
            raise ValueError("kmin / kmax must be matching fp16 [nb, hk, D] with unit last stride")
        bounds = _i64p(kmin.stride()[:2])
    pre = (pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0],
           sl.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), _i64p(k_pool.stride()[:3]),
           k_pool.shape[0], k_pool.shape[1], q_out.data_ptr(), _i64p(q_out.stride()[:3]),
           None if kmin is None else kmin.data_ptr(), None if kmax is None else kmax.data_ptr(),
           bounds)
    return {"pre": pre, "q_out": q_out}


def embed_rms_norm(table: torch.Tensor, ids: torch.Tensor, weight: torch.Tensor, eps: float,
                   out: Optional[torch.Tensor] = None,
                   rows_out: Optional[torch.Tensor] = None):
    """(rms_norm(table[ids]), table[ids]) in one launch: ids [B] or [B, 1]
    int64 (clamped into the table), table [vocab, n] fp16.  The second
    tensor is the residual the first layer carries."""
    _fp16_gpu("table", table)
    _fp16_gpu("weight", weight)
    if table.dim() != 2 or weight.shape != (table.shape[1],):
        raise ValueError("table must be [vocab, n] and weight [n]")
    if not ids.is_cuda:
        raise ValueError("ids must be on the GPU")
    ids1 = ids.reshape(-1)
    if ids1.dtype != torch.int64 or not ids1.is_contiguous():
        ids1 = ids1.to(torch.int64).contiguous()     # a small copy (any integer ids)
    b, n = ids1.shape[0], table.shape[1]
    y = torch.empty((b, n), dtype=table.dtype, device=table.device) if out is None else out
    r = torch.empty((b, n), dtype=table.dtype, device=table.device) if rows_out is None \
        else rows_out
    for name, t in (("out", y), ("rows_out", r)):
        if t.shape != (b, n) or t.stride(-1) != 1 or t.dtype != table.dtype:
            raise ValueError(f"{name} must be fp16 [{b}, {n}] with unit last stride")
    rc = _lib.lib().ls_embed_rms_norm(
        table.data_ptr(), table.stride(0), table.shape[0], ids1.data_ptr(), weight.data_ptr(),
        y.data_ptr(), _row_stride(y), r.data_ptr(), _row_stride(r), b, n, float(eps),
        _stream(table))
    _lib.check(rc, "ls_embed_rms_norm")
    return y, r


def argmax_rows(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """torch.argmax(x, dim=-1, keepdim=True) for fp16 x [..., n]: int64."""
    _fp16_gpu("x", x)
    x2 = _rows(x)
    rows = x2.shape[0]
    o = torch.empty((rows,), dtype=torch.int64, device=x.device) if out is None \
        else out.view(rows)
    if o.dtype != torch.int64 or not o.is_contiguous():
        raise ValueError("out must be contiguous int64")
    need = int(_lib.lib().ls_argmax_workspace_bytes(rows, x2.shape[1]))
    ws = _workspace(x.device, need) if need else None
    rc = _lib.lib().ls_argmax_rows(x2.data_ptr(), _row_stride(x2), o.data_ptr(), rows,
                                   x2.shape[1], None if ws is None else ws.data_ptr(), need,
                                   _stream(x))
    _lib.check(rc, "ls_argmax_rows")
    return o.view(*x.shape[:-1], 1)


_WORKSPACE: dict = {}
_RETIRED: list = []


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The argmax workspace of a device: zero-filled (its counters start at
    zero and every call leaves them so), grown to the largest call seen;
    outgrown buffers are kept, so graphs captured with them stay valid."""
    key = torch.device(device).index
    buf = _WORKSPACE.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _RETIRED.append(buf)
        buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _WORKSPACE[key] = buf
    return buf
