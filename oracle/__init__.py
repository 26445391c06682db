"""CPU oracle for the paged decode-attention path — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package, and only as the checker. The product package
``latentserve_amd`` never imports it.

The arithmetic lives in ``ls_oracle.c`` (plain fp32 C, one function per
reference algorithm, each citing the reference file:line it restates); this
module is a numpy/ctypes front end with the reference's argument names.
Arrays are numpy: fp16 as ``np.float16``, codes ``np.int8``, scales
``np.float32``, tables and lengths ``np.int32``. Strides are taken from the
arrays, so views work.

How each function is pinned (tests/test_oracle.py):

* ``paged_decode`` — fp64 brute-force softmax attention over the gathered
  live tokens (the closed form), split-count invariance, empty splits, ragged
  final pages, no cross-sequence leak; INT8 dequant axes and zero points
  against dense attention over independently dequantised tensors; the
  residual last page against a hand-assembled cache.
* ``quantize_k`` / ``quantize_v`` — bit-exact against numpy float32 IEEE
  arithmetic and against torch CPU's ops in the reference's order, plus the
  error bound |x - q*s| <= s/2 and the all-zero block.
* ``page_scores`` — brute-force Quest bound from per-page min/max computed by
  numpy over the gathered K; forced pages are the sets {0, P-recent..P-1}.
* ``page_scores_mass`` — an fp64 numpy brute force from the same bounds
  (per-head softmax over the pages of bound * scale + log(count), summed),
  a closed form (one live page below the forced ones gets all the mass of
  every head: score n_rep), and the sum over the unforced live pages of
  the unforced mass bounded by n_rep.
* ``sparse_decode`` — brute-force attention over exactly the listed pages,
  and full-budget equality with ``paged_decode``.
* ``combine`` — the all-empty split case and equality with one-split decode.
* ``gather`` / ``bounds_update`` — numpy fancy indexing / running min-max.
* ``rms_norm`` / ``silu_and_mul`` / ``rope`` — Hugging Face's own Qwen2
  modules (transformers' ``Qwen2RMSNorm``, ``apply_rotary_pos_emb``, the
  ``silu`` activation) on torch CPU in fp16, plus closed forms (a constant
  row normalises to the weight; cos 1 / sin 0 is the identity; a quarter
  turn is rotate_half).
* ``rope_write_decode`` — ``rope`` per head, the fold q -> [B, H_kv, n_rep,
  D] by index, the slot rule block * page + offset, and ``bounds_update``.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblsoracle.so")
_lib = None

_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_VP = ctypes.c_void_p


class _Args(ctypes.Structure):
    _fields_ = [
        ("q", _VP), ("sq_b", _I64), ("sq_h", _I64), ("sq_r", _I64),
        ("k_pool", _VP), ("v_pool", _VP),
        ("sk_b", _I64), ("sk_p", _I64), ("sk_h", _I64),
        ("kv_kind", _I32),
        ("k_scale", _VP), ("sks_b", _I64), ("sks_h", _I64),
        ("v_scale", _VP), ("svs_b", _I64), ("svs_p", _I64), ("svs_h", _I64),
        ("k_zero", _VP), ("v_zero", _VP),
        ("k_res", _VP), ("sr_r", _I64), ("sr_p", _I64), ("sr_h", _I64),
        ("res_rows", _VP),
        ("block_tables", _VP), ("sbt_b", _I64),
        ("seq_lens", _VP),
        ("B", _I32), ("H", _I32), ("NR", _I32), ("D", _I32), ("PAGE", _I32),
        ("scale", _F32),
    ]


def build(force: bool = False) -> str:
    """Compile ls_oracle.c with the Makefile beside it."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "liblsoracle.so"], cwd=_HERE, check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.ls_ref_num_threads.restype = ctypes.c_int
        _lib.ls_ref_sparse_count.restype = ctypes.c_int
        _lib.ls_ref_h2f.restype = ctypes.c_float
    return _lib


def set_num_threads(n: int) -> None:
    lib().ls_ref_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().ls_ref_num_threads())


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_VP)


def _st(a):
    """Element strides of a numpy array."""
    return tuple(s // a.itemsize for s in a.strides)


def _args(q, k_pool, v_pool, block_tables, seq_lens, k_scale, v_scale, k_zero, v_zero,
          softmax_scale, k_residual, res_rows):
    b, h, nr, d = q.shape
    if q.dtype != np.float16:
        raise TypeError("q must be float16")
    if k_pool.dtype == np.float16:
        kind = 0
    elif k_pool.dtype == np.int8:
        kind = 1
    else:
        raise TypeError("k_pool must be float16 or int8")
    if v_pool.dtype != k_pool.dtype or _st(v_pool) != _st(k_pool):
        raise ValueError("K and V pools must share dtype and strides")
    if block_tables.dtype != np.int32 or seq_lens.dtype != np.int32:
        raise TypeError("block tables and lengths must be int32")
    for t in (k_scale, v_scale, k_zero, v_zero):
        if t is not None and t.dtype != np.float32:
            raise TypeError("scales and zero points must be float32")
    if (k_residual is None) != (res_rows is None):
        raise ValueError("k_residual and res_rows go together")
    a = _Args()
    a.q = _ptr(q)
    a.sq_b, a.sq_h, a.sq_r = _st(q)[:3]
    a.k_pool, a.v_pool = _ptr(k_pool), _ptr(v_pool)
    a.sk_b, a.sk_p, a.sk_h = _st(k_pool)[:3]
    a.kv_kind = kind
    a.k_scale = _ptr(k_scale)
    if k_scale is not None:
        a.sks_b, a.sks_h = _st(k_scale)[:2]
        if k_zero is not None and _st(k_zero) != _st(k_scale):
            raise ValueError("k_zero must share k_scale's strides")
    a.v_scale = _ptr(v_scale)
    if v_scale is not None:
        a.svs_b, a.svs_p, a.svs_h = _st(v_scale)
        if v_zero is not None and _st(v_zero) != _st(v_scale):
            raise ValueError("v_zero must share v_scale's strides")
    a.k_zero, a.v_zero = _ptr(k_zero), _ptr(v_zero)
    a.k_res = _ptr(k_residual)
    if k_residual is not None:
        if k_residual.dtype != np.float16 or res_rows.dtype != np.int32:
            raise TypeError("k_residual must be float16 and res_rows int32")
        a.sr_r, a.sr_p, a.sr_h = _st(k_residual)[:3]
    a.res_rows = _ptr(res_rows)
    a.block_tables = _ptr(block_tables)
    a.sbt_b = _st(block_tables)[0]
    a.seq_lens = _ptr(seq_lens)
    a.B, a.H, a.NR, a.D, a.PAGE = b, h, nr, d, k_pool.shape[1]
    a.scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    for t in (q, k_pool, block_tables, k_residual):
        if t is not None and _st(t)[-1] != 1:
            raise ValueError("last dimension must be unit-stride")
    return a


def paged_decode(q, k_pool, v_pool, block_tables, seq_lens, k_scale=None, v_scale=None,
                 k_zero=None, v_zero=None, num_splits: int = 1, softmax_scale=None,
                 k_residual=None, res_rows=None) -> np.ndarray:
    """``paged_decode_reference`` (kernels/gqa/paged_decode.py:152-269) on the CPU.

    Returns fp32 [B, H_kv, N_REP, D] — the value before the reference's final
    ``.to(q.dtype)``; ``.astype(np.float16)`` gives the reference's output.
    """
    a = _args(q, k_pool, v_pool, block_tables, seq_lens, k_scale, v_scale, k_zero, v_zero,
              softmax_scale, k_residual, res_rows)
    out = np.zeros(q.shape, dtype=np.float32)
    s = _st(out)
    lib().ls_ref_paged_decode(ctypes.byref(a), _I32(max(1, int(num_splits or 1))),
                              out.ctypes.data_as(_VP), _I64(s[0]), _I64(s[1]), _I64(s[2]))
    return out


def sparse_count(num_pages: int, num_sel: int, ratio, recent: int = 2) -> int:
    """The sparse kernel's per-sequence count (paged_sparse_fp16.cu:242-247)."""
    return int(lib().ls_ref_sparse_count(_I32(num_pages), _I32(num_sel),
                                         _F32(0.0 if ratio is None else ratio), _I32(recent)))


def sparse_decode(q, k_pool, v_pool, block_tables, seq_lens, sel, num_splits: int = 1,
                  softmax_scale=None, ratio=None, recent: int = 2) -> np.ndarray:
    """``sparse_decode`` (kernels/cuda/paged_sparse.py:185-219) on the CPU: fp32 out."""
    if sel.dtype != np.int32:
        raise TypeError("sel must be int32")
    a = _args(q, k_pool, v_pool, block_tables, seq_lens, None, None, None, None,
              softmax_scale, None, None)
    out = np.zeros(q.shape, dtype=np.float32)
    s, ss = _st(out), _st(sel)
    lib().ls_ref_sparse_decode(ctypes.byref(a), _ptr(sel), _I64(ss[0]), _I64(ss[1]),
                               _I32(sel.shape[-1]), _F32(0.0 if ratio is None else ratio),
                               _I32(recent), _I32(max(1, int(num_splits or 1))),
                               out.ctypes.data_as(_VP), _I64(s[0]), _I64(s[1]), _I64(s[2]))
    return out


def combine(partial_acc, partial_m, partial_l) -> np.ndarray:
    """``combine_splits`` (kernels/gqa/paged_decode.py:689-706): fp32 [B, H, N_REP, D]."""
    acc = np.ascontiguousarray(partial_acc, dtype=np.float32)
    m = np.ascontiguousarray(partial_m, dtype=np.float32)
    l = np.ascontiguousarray(partial_l, dtype=np.float32)
    b, h, s, nr, d = acc.shape
    out = np.zeros((b, h, nr, d), dtype=np.float32)
    lib().ls_ref_combine(_I32(b), _I32(h), _I32(s), _I32(nr), _I32(d), _ptr(acc), _ptr(m),
                         _ptr(l), _ptr(out))
    return out


def quantize_k(data, asym: bool = False, eps: float = 1e-8, bits: int = 8, recip: bool = False):
    """``_finalize_blocks`` (cache/int8_paged_cache.py:670-699).  recip: divide
    by qmax / levels as torch does on a GPU (times the fp32 reciprocal).

    data fp16 [N, PAGE, H, D] -> (codes int8 [N, PAGE, H, D], step fp32 [N, H, D],
    zero fp32 [N, H, D] or None).
    """
    data = np.ascontiguousarray(data, dtype=np.float16)
    n, page, h, d = data.shape
    codes = np.empty(data.shape, dtype=np.int8)
    step = np.empty((n, h, d), dtype=np.float32)
    zero = np.empty((n, h, d), dtype=np.float32) if asym else None
    lib().ls_ref_quantize_k(_ptr(data), _I32(n), _I32(page), _I32(h), _I32(d), _I32(int(asym)),
                            _F32(eps), _F32(2 ** (bits - 1) - 1), _F32(2 ** bits - 1),
                            _F32(2 ** (bits - 1)), _I32(int(recip)), _ptr(codes), _ptr(step),
                            _ptr(zero))
    return codes, step, zero


def quantize_v(v, asym: bool = False, eps: float = 1e-8, bits: int = 8, recip: bool = False):
    """V's per-token quantizer (cache/int8_paged_cache.py:741-758); recip as
    for quantize_k.

    v fp16 [..., H, D] -> (codes int8 same shape, step fp32 [..., H], zero or None).
    """
    v = np.ascontiguousarray(v, dtype=np.float16)
    lead = v.shape[:-2]
    h, d = v.shape[-2:]
    t = int(np.prod(lead)) if lead else 1
    codes = np.empty(v.shape, dtype=np.int8)
    step = np.empty(lead + (h,), dtype=np.float32)
    zero = np.empty(lead + (h,), dtype=np.float32) if asym else None
    lib().ls_ref_quantize_v(_ptr(v), _I32(t), _I32(h), _I32(d), _I32(int(asym)), _F32(eps),
                            _F32(2 ** (bits - 1) - 1), _F32(2 ** bits - 1),
                            _F32(2 ** (bits - 1)), _I32(int(recip)), _ptr(codes), _ptr(step),
                            _ptr(zero))
    return codes, step, zero


def page_scores(q, kmin, kmax, block_tables, seq_lens, recent: int = 2, page: int = 16):
    """``page_scores`` (kernels/cuda/paged_sparse.py:104-123 -> page_index) on the CPU.

    Returns fp32 [B, H, max_pages].
    """
    b, h, nr, d = q.shape
    maxp = block_tables.shape[1]
    out = np.empty((b, h, maxp), dtype=np.float32)
    sq, sb = _st(q), _st(kmin)
    if _st(kmax) != sb:
        raise ValueError("kmin and kmax must share strides")
    lib().ls_ref_page_scores(_ptr(q), _I64(sq[0]), _I64(sq[1]), _I64(sq[2]), _ptr(kmin),
                             _ptr(kmax), _I64(sb[0]), _I64(sb[1]), _ptr(block_tables),
                             _I64(_st(block_tables)[0]), _ptr(seq_lens), _I32(b), _I32(h),
                             _I32(nr), _I32(d), _I32(page), _I32(maxp), _I32(recent), _ptr(out))
    return out


def page_scores_mass(q, kmin, kmax, block_tables, seq_lens, recent: int = 2,
                     softmax_scale=None, page: int = 16):
    """``page_scores_mass`` (kernels/cuda/paged_sparse.py:126-161) on the CPU:
    fp32 [B, H, max_pages] summed-mass scores."""
    b, h, nr, d = q.shape
    maxp = block_tables.shape[1]
    out = np.empty((b, h, maxp), dtype=np.float32)
    sq, sb = _st(q), _st(kmin)
    if _st(kmax) != sb:
        raise ValueError("kmin and kmax must share strides")
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale
    lib().ls_ref_page_scores_mass(
        _ptr(q), _I64(sq[0]), _I64(sq[1]), _I64(sq[2]), _ptr(kmin), _ptr(kmax), _I64(sb[0]),
        _I64(sb[1]), _ptr(block_tables), _I64(_st(block_tables)[0]), _ptr(seq_lens), _I32(b),
        _I32(h), _I32(nr), _I32(d), _I32(page), _I32(maxp), _I32(recent), _F32(scale),
        _ptr(out))
    return out


def budget(ratio: float, max_pages: int, recent: int = 2) -> int:
    """``budget`` (kernels/cuda/paged_sparse.py:74-78)."""
    if ratio >= 1.0:
        return max_pages
    return min(max_pages, max(recent + 1, math.ceil(ratio * max_pages)))


def select(scores: np.ndarray, k: int) -> np.ndarray:
    """Top-k page indices per (b, h), highest score first (``select``,
    kernels/cuda/paged_sparse.py:164-168). Equal scores keep the lower page
    index first; the reference's ``torch.topk`` leaves tie order unspecified,
    so tests compare selected *sets* away from ties."""
    order = np.argsort(-scores, axis=-1, kind="stable")
    return np.ascontiguousarray(order[..., :k]).astype(np.int32)


def bounds_update(k_new, slots, kmin, kmax, page: int = 16) -> None:
    """Running page bounds on write (paged_sparse_fp16.cu:54-72), in place."""
    k_new = np.ascontiguousarray(k_new, dtype=np.float16)
    b, h, d = k_new.shape[0], k_new.shape[1], k_new.shape[-1]
    slots = np.ascontiguousarray(slots, dtype=np.int64)
    assert kmin.flags.c_contiguous and kmax.flags.c_contiguous
    lib().ls_ref_bounds_update(_ptr(k_new), _ptr(slots), _I32(b), _I32(h), _I32(d), _I32(page),
                               _ptr(kmin), _ptr(kmax))


def gather(pool, block_tables, seq_lens, lmax: int):
    """The gather read (cache/paged_cache.py:486-506): [B, H, lmax, D]; positions
    past a sequence's length hold flat slot 0, as the reference's padded slot
    table reads (:305-323)."""
    pool = np.ascontiguousarray(pool)
    nb, page, h, d = pool.shape
    b = block_tables.shape[0]
    out = np.zeros((b, h, lmax, d), dtype=pool.dtype)
    lib().ls_ref_gather(_ptr(pool), _I32(pool.itemsize), _ptr(block_tables),
                        _I64(_st(block_tables)[0]), _ptr(seq_lens), _I32(b), _I32(h), _I32(d),
                        _I32(page), _I32(lmax), _ptr(out))
    return out


# ---- fused elementwise ops of the decode step (numpy, fp16 step by step) --


def _f16(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16)


def rms_norm(x, w, eps: float, residual=None):
    """(y, s): s = x, or fp16(residual + x); y = w * fp16(s * rsqrt(mean(s^2)
    + eps)) with the variance in float64 (kernels/fused_elementwise.py:75-85,
    Hugging Face's Qwen2RMSNorm: fp32 variance, the normalised value cast to
    fp16 before the fp16 weight multiply)."""
    x = np.asarray(x, np.float16)
    s = x if residual is None else _f16(np.asarray(residual, np.float32) + x.astype(np.float32))
    h = s.astype(np.float64)
    inv = 1.0 / np.sqrt((h * h).mean(-1, keepdims=True) + eps)
    hn = _f16(s.astype(np.float32) * inv.astype(np.float32))
    y = _f16(np.asarray(w, np.float16).astype(np.float32) * hn.astype(np.float32))
    return y, s


def silu_and_mul(gate_up):
    """fp16(fp16(silu(g)) * u) over the halves of the last axis
    (kernels/fused_elementwise.py:88-90: F.silu(gate) * up in fp16)."""
    gu = np.asarray(gate_up, np.float16)
    n = gu.shape[-1] // 2
    g = gu[..., :n].astype(np.float32)
    with np.errstate(over="ignore"):
        sg = _f16(g / (np.float32(1) + np.exp(-g)))
    return _f16(sg.astype(np.float32) * gu[..., n:].astype(np.float32))


def rope(x, cos, sin):
    """fp16(fp16(x * cos) + fp16(rotate_half(x) * sin)) on the last axis
    (kernels/fused_elementwise.py:93-110, Hugging Face's
    apply_rotary_pos_emb in fp16); cos / sin broadcast against x."""
    x = np.asarray(x, np.float16)
    d = x.shape[-1]
    rot = np.concatenate([-x[..., d // 2:], x[..., :d // 2]], axis=-1)
    a = _f16(x.astype(np.float32) * np.asarray(cos, np.float16).astype(np.float32))
    b = _f16(rot.astype(np.float32) * np.asarray(sin, np.float16).astype(np.float32))
    return _f16(a.astype(np.float32) + b.astype(np.float32))


def rope_write_decode(qkv, positions, cos, sin, slots, k_pool, v_pool, hq: int, hk: int,
                      kmin=None, kmax=None, page: int = 16):
    """One decode token per sequence: q_out [B, hk, hq // hk, d] returned;
    the rotated key and the value stored into k_pool / v_pool [nb, page, hk,
    d] at flat slots[b] (negative or past the pool: not stored), the page K
    bounds updated when given.  Positions are clamped into the table."""
    qkv = np.asarray(qkv, np.float16)
    b, d = qkv.shape[0], cos.shape[-1]
    pos = np.clip(np.asarray(positions, np.int64), 0, cos.shape[0] - 1)
    c, s = cos[pos][:, None, :], sin[pos][:, None, :]
    q = rope(qkv[:, :hq * d].reshape(b, hq, d), c, s)
    k = rope(qkv[:, hq * d:(hq + hk) * d].reshape(b, hk, d), c, s)
    v = qkv[:, (hq + hk) * d:(hq + 2 * hk) * d].reshape(b, hk, d)
    nb = k_pool.shape[0]
    stored = []
    for i in range(b):
        slot = int(slots[i])
        if slot < 0 or slot // page >= nb:
            continue
        k_pool[slot // page, slot % page] = k[i]
        v_pool[slot // page, slot % page] = v[i]
        stored.append(i)
    if kmin is not None and stored:            # the bounds of the rows stored
        bounds_update(k[stored], np.asarray(slots, np.int64)[stored], kmin, kmax, page)
    return q.reshape(b, hk, hq // hk, d)
