"""Seeded synthetic inputs and closed-form checkers shared by the tests.

Block tables are always scattered (a seeded permutation of the pool), as the
reference's tests insist (tests/test_phase11_kernel.py:41-56): contiguous ids
would let a broken block-table lookup pass.
"""

from __future__ import annotations

import math

import numpy as np


def paged_case(lengths, h_kv=2, n_rep=6, d=128, page=16, seed=0, extra_blocks=5, width=None):
    """fp16 q [B,H,NR,D], pools [nb,PAGE,H,D], int32 tables [B,maxP], int32 lens [B]."""
    rng = np.random.default_rng(seed)
    b = len(lengths)
    max_pages = max(1, max((l + page - 1) // page for l in lengths))
    width = width or max_pages
    nb = b * width + extra_blocks
    k_pool = rng.standard_normal((nb, page, h_kv, d), dtype=np.float32).astype(np.float16)
    v_pool = rng.standard_normal((nb, page, h_kv, d), dtype=np.float32).astype(np.float16)
    tables = rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32)
    q = rng.standard_normal((b, h_kv, n_rep, d), dtype=np.float32).astype(np.float16)
    lens = np.asarray(lengths, dtype=np.int32)
    return q, k_pool, v_pool, tables, lens


def gather_tokens(pool, tables, b, length, page=16):
    """[H, L, D] of the live tokens of sequence b, in logical order."""
    idx = np.arange(length)
    blk = tables[b, idx // page]
    return np.transpose(pool[blk, idx % page], (1, 0, 2))


def dense_attention(q, k_pool, v_pool, tables, lens, page=16, scale=None, keep_pages=None,
                    k_res=None, res_rows=None):
    """fp64 brute force: gather every live token, one softmax per query row.

    keep_pages[b][h]: optional iterable of logical pages to attend (others masked).
    k_res/res_rows: the last page's K comes from k_res[res_rows[b]] (INT8 residual).
    """
    b, h_kv, n_rep, d = q.shape
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros(q.shape, dtype=np.float64)
    for i in range(b):
        length = int(lens[i])
        if length == 0:
            continue
        k = gather_tokens(k_pool, tables, i, length, page).astype(np.float64)
        v = gather_tokens(v_pool, tables, i, length, page).astype(np.float64)
        if k_res is not None:
            last = (length - 1) // page
            n_last = length - last * page
            k[:, last * page:] = np.transpose(
                k_res[int(res_rows[i]), :n_last], (1, 0, 2)).astype(np.float64)
        for hh in range(h_kv):
            logits = (q[i, hh].astype(np.float64) @ k[hh].T) * scale
            if keep_pages is not None:
                keep = np.zeros(length, dtype=bool)
                for p in keep_pages[i][hh]:
                    keep[p * page: min(length, (p + 1) * page)] = True
                if not keep.any():
                    continue
                logits = np.where(keep[None, :], logits, -np.inf)
            logits -= logits.max(axis=-1, keepdims=True)
            w = np.exp(logits)
            w /= w.sum(axis=-1, keepdims=True)
            out[i, hh] = w @ v[hh]
    return out


def int8_case(lengths, asym=False, res=True, h_kv=2, n_rep=6, d=128, page=16, seed=0):
    """Random int8 codes with positive fp32 scales (the reference's own INT8
    test recipe, tests/test_cuda_decode.py:174-198); residual rows reversed so
    an identity mapping would not hide a by-batch-index read."""
    rng = np.random.default_rng(seed)
    b = len(lengths)
    pages = max(1, max((l + page - 1) // page for l in lengths))
    nb = b * pages + 3
    k = rng.integers(-127, 128, (nb, page, h_kv, d), dtype=np.int8)
    v = rng.integers(-127, 128, (nb, page, h_kv, d), dtype=np.int8)
    ks = (rng.random((nb, h_kv, d), dtype=np.float32) * 0.02 + 1e-3).astype(np.float32)
    vs = (rng.random((nb, page, h_kv), dtype=np.float32) * 0.02 + 1e-3).astype(np.float32)
    extra = dict(k_scale=ks, v_scale=vs)
    if asym:
        extra.update(k_zero=(rng.standard_normal((nb, h_kv, d), dtype=np.float32) * 0.1),
                     v_zero=(rng.standard_normal((nb, page, h_kv), dtype=np.float32) * 0.1))
    if res:
        extra.update(
            k_residual=rng.standard_normal((b + 2, page, h_kv, d), dtype=np.float32).astype(np.float16),
            res_rows=(np.arange(b, dtype=np.int32)[::-1] + 1).astype(np.int32))
    tables = rng.permutation(nb)[: b * pages].reshape(b, pages).astype(np.int32)
    q = rng.standard_normal((b, h_kv, n_rep, d), dtype=np.float32).astype(np.float16)
    return (q, k, v, tables, np.asarray(lengths, dtype=np.int32)), extra


def dequant_pools(k, v, k_scale, v_scale, k_zero=None, v_zero=None):
    """fp64 dequantised pools, K scale per (block, head, channel), V per (block, token, head)."""
    kd = k.astype(np.float64) * k_scale[:, None, :, :]
    vd = v.astype(np.float64) * v_scale[:, :, :, None]
    if k_zero is not None:
        kd = kd + k_zero[:, None, :, :]
    if v_zero is not None:
        vd = vd + v_zero[:, :, :, None]
    return kd, vd


def assert_close(got, want, atol, rtol, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    if bad.any():
        i = np.unravel_index(np.argmax(err - atol - rtol * np.abs(want)), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside atol={atol} "
                             f"rtol={rtol}; worst at {i}: got {got[i]} want {want[i]}; "
                             f"max abs err {err.max():.3g}")
