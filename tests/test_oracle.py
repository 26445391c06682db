"""Pins the CPU oracle (oracle/) before anything is compared against it.

Every check here is independent of the oracle's own formula: fp64
brute-force attention over gathered tokens (the closed form), invariants the
mathematics fixes (split-count invariance, empty splits, no leaks, full
budget = dense), numpy/torch IEEE arithmetic for the quantizer, and
brute-force min/max for the selector. The cases are the reference's own CPU
tests (tests/test_phase11_kernel.py:87-195, tests/test_phase14_int8_graph.py:
139-183, tests/test_phase7_int8_cache.py:89-118, 420-442), restated.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from tests.cases import (assert_close, dense_attention, dequant_pools, gather_tokens,
                         int8_case, paged_case)

# fp32 arithmetic on fp16 inputs against fp64: the reference's CPU tolerance.
RTOL, ATOL = 1e-4, 1e-5


def small(lengths, **kw):
    kw.setdefault("d", 32)
    kw.setdefault("n_rep", 3)
    return paged_case(lengths, **kw)


def test_matches_dense_attention():
    q, k, v, t, l = small([40, 17])
    assert_close(oracle.paged_decode(q, k, v, t, l), dense_attention(q, k, v, t, l), ATOL, RTOL)


def test_matches_dense_attention_at_production_geometry():
    q, k, v, t, l = paged_case([300, 1, 77])
    assert_close(oracle.paged_decode(q, k, v, t, l, num_splits=3),
                 dense_attention(q, k, v, t, l), ATOL, RTOL)


@pytest.mark.parametrize("num_splits", [1, 2, 3, 4, 8])
def test_split_k_is_exact(num_splits):
    q, k, v, t, l = small([63, 40])
    assert_close(oracle.paged_decode(q, k, v, t, l, num_splits=num_splits),
                 dense_attention(q, k, v, t, l), ATOL, RTOL)


def test_more_splits_than_pages_is_harmless():
    q, k, v, t, l = small([10, 5])
    got = oracle.paged_decode(q, k, v, t, l, num_splits=8)
    assert np.isfinite(got).all()
    assert_close(got, dense_attention(q, k, v, t, l), ATOL, RTOL)


@pytest.mark.parametrize("length", [1, 15, 16, 17, 31, 32, 33])
def test_ragged_final_page(length):
    q, k, v, t, l = small([length])
    assert_close(oracle.paged_decode(q, k, v, t, l, num_splits=2),
                 dense_attention(q, k, v, t, l), ATOL, RTOL)


def test_empty_sequence_gives_zeros():
    q, k, v, t, l = small([0, 20])
    got = oracle.paged_decode(q, k, v, t, l, num_splits=3)
    assert (got[0] == 0).all()
    assert_close(got, dense_attention(q, k, v, t, l), ATOL, RTOL)


def test_sequences_do_not_leak_into_each_other():
    q, k, v, t, l = small([64, 3])
    got = oracle.paged_decode(q, k, v, t, l)
    solo = oracle.paged_decode(q[1:2], k, v, t[1:2], l[1:2])
    np.testing.assert_array_equal(got[1:2], solo)


def test_a_wrong_block_table_is_detected():
    """Sanity of the checker itself: reading pages in identity order must fail."""
    q, k, v, t, l = small([64, 40])
    ident = np.arange(t.size, dtype=np.int32).reshape(t.shape)
    with pytest.raises(AssertionError):
        assert_close(oracle.paged_decode(q, k, v, ident, l), dense_attention(q, k, v, t, l),
                     ATOL, RTOL)


def test_int8_uses_the_right_scale_axes():
    (q, k, v, t, l), ex = int8_case([40], res=False, d=32, n_rep=4)
    kd, vd = dequant_pools(k, v, ex["k_scale"], ex["v_scale"])
    want = dense_attention(q, kd, vd, t, l)
    got = oracle.paged_decode(q, k, v, t, l, num_splits=2, **ex)
    assert_close(got, want, ATOL, RTOL)
    # Swapping the axes (the easiest mistake) produces different numbers.
    wrong_v = v.astype(np.float64) * ex["v_scale"].mean(axis=1)[:, None, :, None]
    with pytest.raises(AssertionError):
        assert_close(got, dense_attention(q, kd, wrong_v, t, l), ATOL, RTOL)


def test_int8_zero_points_on_the_right_axes():
    (q, k, v, t, l), ex = int8_case([30, 55], asym=True, res=False, d=32, n_rep=3, seed=4)
    kd, vd = dequant_pools(k, v, ex["k_scale"], ex["v_scale"], ex["k_zero"], ex["v_zero"])
    assert_close(oracle.paged_decode(q, k, v, t, l, num_splits=2, **ex),
                 dense_attention(q, kd, vd, t, l), ATOL, RTOL)


@pytest.mark.parametrize("lengths", [[40, 21], [16, 32, 1, 33]])
def test_int8_last_page_comes_from_the_residual(lengths):
    (q, k, v, t, l), ex = int8_case(lengths, res=True, d=16, n_rep=4, seed=2)
    kd, vd = dequant_pools(k, v, ex["k_scale"], ex["v_scale"])
    want = dense_attention(q, kd, vd, t, l, k_res=ex["k_residual"], res_rows=ex["res_rows"])
    assert_close(oracle.paged_decode(q, k, v, t, l, num_splits=2, **ex), want, ATOL, RTOL)


def test_combine_handles_an_all_empty_split():
    acc = np.zeros((1, 1, 3, 4, 8), np.float32)
    m = np.full((1, 1, 3, 4), -np.inf, np.float32)
    l = np.zeros((1, 1, 3, 4), np.float32)
    m[:, :, 0] = 0.0
    l[:, :, 0] = 1.0
    acc[:, :, 0] = 1.0
    out = oracle.combine(acc, m, l)
    assert np.isfinite(out).all()
    np.testing.assert_array_equal(out, np.ones((1, 1, 4, 8), np.float32))


def test_combine_of_all_empty_is_zero():
    out = oracle.combine(np.zeros((1, 1, 2, 3, 4), np.float32),
                         np.full((1, 1, 2, 3), -np.inf, np.float32), np.zeros((1, 1, 2, 3), np.float32))
    np.testing.assert_array_equal(out, 0)


# ------------------------------------------------------------- quantizer --


def _np_quant_sym(f32, axis, qmax=127.0, eps=1e-8):
    step = np.maximum(np.abs(f32).max(axis=axis, keepdims=True), np.float32(eps)) / np.float32(qmax)
    q = np.clip(np.rint(f32 / step), -qmax, qmax).astype(np.int8)
    return q, np.squeeze(step, axis=axis).astype(np.float32)


def _np_quant_asym(f32, axis, levels=255.0, offset=128.0, eps=1e-8):
    lo = f32.min(axis=axis, keepdims=True)
    hi = f32.max(axis=axis, keepdims=True)
    step = np.maximum((hi - lo) / np.float32(levels), np.float32(eps)).astype(np.float32)
    u = np.clip(np.rint((f32 - lo) / step), 0, levels)
    q = (u - np.float32(offset)).astype(np.int8)
    zero = (lo + np.float32(offset) * step).astype(np.float32)
    return q, np.squeeze(step, axis=axis), np.squeeze(zero, axis=axis)


def _fp16(shape, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * scale).astype(np.float16)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_k_quantizer_is_ieee_exact(seed):
    data = _fp16((37, 16, 2, 128), seed, scale=[1.0, 3.0, 0.01][seed])
    codes, step, zero = oracle.quantize_k(data)
    assert zero is None
    q, s = _np_quant_sym(data.astype(np.float32), axis=1)
    np.testing.assert_array_equal(step, s)
    np.testing.assert_array_equal(codes, q)


def test_k_quantizer_asymmetric_is_ieee_exact():
    data = _fp16((9, 16, 2, 64), 5) + np.float16(0.7)
    codes, step, zero = oracle.quantize_k(data, asym=True)
    q, s, z = _np_quant_asym(data.astype(np.float32), axis=1)
    np.testing.assert_array_equal(step, s)
    np.testing.assert_array_equal(zero, z)
    np.testing.assert_array_equal(codes, q)


def test_v_quantizer_is_ieee_exact():
    v = _fp16((16, 7, 2, 128), 6, scale=2.0)
    codes, step, _ = oracle.quantize_v(v)
    q, s = _np_quant_sym(v.astype(np.float32), axis=-1)
    np.testing.assert_array_equal(step, s)
    np.testing.assert_array_equal(codes, q)
    codes_a, step_a, zero_a = oracle.quantize_v(v, asym=True)
    qa, sa, za = _np_quant_asym(v.astype(np.float32), axis=-1)
    np.testing.assert_array_equal(codes_a, qa)
    np.testing.assert_array_equal(step_a, sa)
    np.testing.assert_array_equal(zero_a, za)


def test_quantizer_matches_torch_cpu_ops_in_the_reference_order():
    """The reference fits scales with torch CPU ops: f.abs().amax().clamp_min(eps) / 127,
    clamp(round(f / step)).to(int8) (cache/int8_paged_cache.py:694-697, 753-756)."""
    torch = pytest.importorskip("torch")
    data = _fp16((11, 16, 2, 128), 7, scale=1.7)
    f = torch.from_numpy(data).to(torch.float32)
    step = f.abs().amax(dim=1).clamp_min(1e-8) / 127
    q = torch.clamp(torch.round(f / step.unsqueeze(1)), -127, 127).to(torch.int8)
    codes, s, _ = oracle.quantize_k(data)
    np.testing.assert_array_equal(s, step.numpy())
    np.testing.assert_array_equal(codes, q.numpy())
    vf = f[:, 0]                                                    # [11, 2, 128] tokens
    vstep = vf.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / 127
    vq = torch.clamp(torch.round(vf / vstep), -127, 127).to(torch.int8)
    vc, vs, _ = oracle.quantize_v(data[:, 0])
    np.testing.assert_array_equal(vs, vstep.squeeze(-1).numpy())
    np.testing.assert_array_equal(vc, vq.numpy())


def test_division_is_true_division_not_a_reciprocal_product():
    """x / 127 differs from x * fl(1/127) for some fp32 x; the CPU reference
    divides. Find such an x and check the oracle follows the division."""
    xs = np.float32(np.linspace(0.5, 8.0, 200001))
    div = xs / np.float32(127)
    mul = xs * (np.float32(1) / np.float32(127))
    i = int(np.nonzero(div != mul)[0][0])
    x = xs[i]
    data = np.zeros((1, 16, 1, 1), np.float16)
    # an fp16 value whose fp32 widening has the differing property
    cand = xs[np.nonzero(div != mul)[0]].astype(np.float16).astype(np.float32)
    ok = cand[(cand / np.float32(127)) != cand * (np.float32(1) / np.float32(127))]
    assert ok.size, x
    data[0, 0, 0, 0] = np.float16(ok[0])
    _, step, _ = oracle.quantize_k(data)
    assert step[0, 0, 0] == ok[0] / np.float32(127)
    assert step[0, 0, 0] != ok[0] * (np.float32(1) / np.float32(127))


def _np_quant_sym_recip(f32, axis, qmax=127.0, eps=1e-8):
    inv = np.float32(1) / np.float32(qmax)
    step = np.maximum(np.abs(f32).max(axis=axis, keepdims=True), np.float32(eps)) * inv
    q = np.clip(np.rint(f32 / step), -qmax, qmax).astype(np.int8)
    return q, np.squeeze(step, axis=axis).astype(np.float32)


def _np_quant_asym_recip(f32, axis, levels=255.0, offset=128.0, eps=1e-8):
    inv = np.float32(1) / np.float32(levels)
    lo = f32.min(axis=axis, keepdims=True)
    hi = f32.max(axis=axis, keepdims=True)
    step = np.maximum((hi - lo) * inv, np.float32(eps)).astype(np.float32)
    u = np.clip(np.rint((f32 - lo) / step), 0, levels)
    q = (u - np.float32(offset)).astype(np.int8)
    zero = (lo + np.float32(offset) * step).astype(np.float32)
    return q, np.squeeze(step, axis=axis), np.squeeze(zero, axis=axis)


def test_reciprocal_mode_is_torch_on_a_gpu():
    """recip=1: `t / python_number` as torch computes it on a GPU, times the
    fp32 reciprocal formed on the host (kernels/cuda/int8_write.cu:20-24 and
    int8_write.py:77-80 state it); tensor / tensor stays a true division."""
    data = _fp16((23, 16, 2, 128), 11, scale=1.3)
    f = data.astype(np.float32)
    codes, step, _ = oracle.quantize_k(data, recip=True)
    q, s = _np_quant_sym_recip(f, axis=1)
    np.testing.assert_array_equal(step, s)
    np.testing.assert_array_equal(codes, q)
    codes, step, zero = oracle.quantize_k(data, asym=True, recip=True)
    q, s, z = _np_quant_asym_recip(f, axis=1)
    np.testing.assert_array_equal(step, s)
    np.testing.assert_array_equal(zero, z)
    np.testing.assert_array_equal(codes, q)
    v = data[:, 0]
    vc, vs, _ = oracle.quantize_v(v, recip=True)
    q, s = _np_quant_sym_recip(v.astype(np.float32), axis=-1)
    np.testing.assert_array_equal(vs, s)
    np.testing.assert_array_equal(vc, q)
    vc, vs, vz = oracle.quantize_v(v, asym=True, recip=True)
    q, s, z = _np_quant_asym_recip(v.astype(np.float32), axis=-1)
    np.testing.assert_array_equal(vc, q)
    np.testing.assert_array_equal(vs, s)
    np.testing.assert_array_equal(vz, z)


def test_the_two_division_forms_differ_in_a_few_percent_of_scales():
    """The reference measured 4.7% of /127 scales off by one bit between the
    forms (kernels/cuda/int8_write.cu:20-24); the modes must really differ."""
    data = _fp16((400, 16, 2, 128), 12)
    _, s_div, _ = oracle.quantize_k(data)
    _, s_mul, _ = oracle.quantize_k(data, recip=True)
    frac = float((s_div != s_mul).mean())
    assert 0.005 < frac < 0.2, frac
    ulp = np.abs(s_div.view(np.int32).astype(np.int64) - s_mul.view(np.int32).astype(np.int64))
    assert ulp.max() == 1


def test_quantization_error_is_within_half_a_step():
    data = _fp16((20, 16, 2, 128), 8, scale=2.5)
    codes, step, _ = oracle.quantize_k(data)
    err = np.abs(codes.astype(np.float32) * step[:, None] - data.astype(np.float32))
    assert (err <= 0.51 * step[:, None]).all()      # the reference's own bound (tests/test_phase7_int8_cache.py:118)
    # the channel's absmax maps to +-127 exactly
    assert (np.abs(codes).max(axis=1) == 127).all()


def test_all_zero_block_quantizes_to_zero_with_the_eps_floor():
    codes, step, _ = oracle.quantize_k(np.zeros((2, 16, 2, 8), np.float16))
    assert (codes == 0).all()
    assert (step == np.float32(1e-8) / np.float32(127)).all()
    vc, vs, _ = oracle.quantize_v(np.zeros((3, 2, 8), np.float16))
    assert (vc == 0).all() and np.isfinite(vs).all()


# -------------------------------------------------------------- selector --


def _bounds_from_pool(k_pool):
    """Per-block per-channel min/max over all PAGE rows (rebuild_bounds,
    kernels/cuda/paged_sparse.py:81-85)."""
    return k_pool.min(axis=1), k_pool.max(axis=1)


def test_page_scores_are_the_brute_force_quest_bound():
    q, k, v, t, l = paged_case([700, 333], seed=1)
    kmin, kmax = _bounds_from_pool(k)
    got = oracle.page_scores(q, kmin, kmax, t, l, recent=2)
    qf = q.astype(np.float64)
    for b, L in enumerate(l):
        np_ = -(-int(L) // 16)
        K = gather_tokens(k, t, b, np_ * 16).astype(np.float64)        # [H, T, D]
        pages_min = K.reshape(2, np_, 16, -1).min(axis=2)               # [H, P, D]
        pages_max = K.reshape(2, np_, 16, -1).max(axis=2)
        bound = np.maximum(qf[b][:, :, None, :] * pages_min[:, None],
                           qf[b][:, :, None, :] * pages_max[:, None]).sum(-1).max(axis=1)
        mid = slice(1, np_ - 2)
        assert_close(got[b, :, mid], bound[:, mid], 1e-3, 1e-4)
        assert (got[b, :, 0] == np.inf).all()
        assert (got[b, :, np_ - 2:np_] == np.inf).all()
        assert (got[b, :, np_:] == -np.inf).all()


def _mass_brute_force(q, kmin, kmax, t, l, recent, scale):
    """fp64: per query head, softmax over the live pages of bound * scale +
    log(tokens in the page); summed over the heads; forced / past-end
    overrides (kernels/cuda/paged_sparse.py:126-161)."""
    b_, h_, nr, d = q.shape
    maxp = t.shape[1]
    out = np.zeros((b_, h_, maxp))
    for b in range(b_):
        L = int(l[b])
        np_ = -(-L // 16)
        cnt = np.clip(L - np.arange(np_) * 16, 0, 16).astype(np.float64)
        lo = kmin[t[b, :np_]].astype(np.float64)                     # [P, H, D]
        hi = kmax[t[b, :np_]].astype(np.float64)
        for h in range(h_):
            qf = q[b, h].astype(np.float64)                          # [NR, D]
            bound = np.maximum(qf[:, None, :] * lo[None, :, h], qf[:, None, :] * hi[None, :, h]).sum(-1)
            logit = bound * scale + np.log(cnt)[None]
            w = np.exp(logit - logit.max(axis=1, keepdims=True))
            out[b, h, :np_] = (w / w.sum(axis=1, keepdims=True)).sum(0)
            out[b, h, np_:] = -np.inf
            out[b, h, 0] = np.inf
            if recent:
                out[b, h, max(0, np_ - recent):np_] = np.inf
    return out


@pytest.mark.parametrize("recent", [2, 0])
def test_page_scores_mass_is_the_brute_force_softmax_sum(recent):
    q, k, v, t, l = paged_case([700, 333, 16, 1], seed=4, extra_blocks=3)
    kmin, kmax = _bounds_from_pool(k)
    scale = 1.0 / math.sqrt(128)
    got = oracle.page_scores_mass(q, kmin, kmax, t, l, recent=recent)
    want = _mass_brute_force(q, kmin, kmax, t, l, recent, scale)
    fin = np.isfinite(want)
    assert np.array_equal(got[~fin], want[~fin])
    assert_close(got[fin], want[fin], 1e-7, 1e-5, "mass scores")
    # the unforced mass of a row never exceeds the n_rep heads' total
    assert (np.where(fin, got, 0).sum(-1) <= 6 + 1e-5).all()


def test_page_scores_mass_one_dominant_page_takes_every_head():
    """Every query row positive, every page's K bounds -1 except page 5's
    +10: page 5 takes (to fp32) all of each head's softmax, score = n_rep."""
    q = np.ones((1, 2, 6, 128), np.float16)
    nb = 12
    kmin = np.full((nb, 2, 128), -1, np.float16)
    kmax = kmin.copy()
    t = np.arange(10, dtype=np.int32)[None]
    kmin[5] = kmax[5] = 10
    l = np.array([160], np.int32)
    got = oracle.page_scores_mass(q, kmin, kmax, t, l, recent=2)
    assert np.allclose(got[0, :, 5], 6.0, rtol=0, atol=1e-6)
    others = [p for p in range(1, 8) if p != 5]
    assert (got[0][:, others] < 1e-30).all()


def test_bounds_update_tracks_running_min_max():
    rng = np.random.default_rng(1)
    nb, h, d = 8, 2, 16
    kmin = np.full((nb, h, d), 99.0, np.float16)
    kmax = np.full((nb, h, d), -99.0, np.float16)
    blocks, written = [5, 2], {}
    for pos in range(27):
        slot = blocks[pos // 16] * 16 + pos % 16
        k_new = rng.standard_normal((1, h, d), dtype=np.float32).astype(np.float16)
        oracle.bounds_update(k_new, np.array([slot]), kmin, kmax)
        written.setdefault(blocks[pos // 16], []).append(k_new[0])
    for blk, rows in written.items():
        st = np.stack(rows)
        np.testing.assert_array_equal(kmin[blk], st.min(0))
        np.testing.assert_array_equal(kmax[blk], st.max(0))


def test_budget_rules():
    assert oracle.budget(0.5, 2048) == 1024
    assert oracle.budget(0.001, 100) == 3
    assert oracle.budget(1.0, 77) == 77
    # the in-kernel count: fp32 multiply then ceilf
    assert oracle.sparse_count(2048, 1024, 0.5) == 1024
    assert oracle.sparse_count(10, 1024, 0.5) == 5
    assert oracle.sparse_count(2, 1024, 0.25) == 2          # capped at the pages it has
    assert oracle.sparse_count(100, 7, 0.5) == 7            # capped at the list length
    assert oracle.sparse_count(100, 50, 0.0) == 50          # ratio <= 0: whole list
    for pages in range(1, 300):
        want = min(pages, max(3, int(math.ceil(np.float32(0.3) * np.float32(pages)))))
        assert oracle.sparse_count(pages, 4096, 0.3) == want


@pytest.mark.parametrize("num_splits", [1, 3])
def test_sparse_attends_exactly_the_given_pages(num_splits):
    q, k, v, t, l = paged_case([700, 150], seed=2)
    picks = [[0, 3, 7, 12, 20, 43], [0, 2, 5, 9, 30, 40]]          # seq 1 has 10 pages
    sel = np.array([[p, p[::-1]] for p in picks], dtype=np.int32)
    got = oracle.sparse_decode(q, k, v, t, l, sel, num_splits=num_splits)
    keep = [[[p for p in picks[b] if p < -(-int(l[b]) // 16)]] * 2 for b in range(2)]
    assert_close(got, dense_attention(q, k, v, t, l, keep_pages=keep), ATOL, RTOL)


def test_sparse_full_budget_is_dense():
    q, k, v, t, l = paged_case([1024, 300], seed=3)
    kmin, kmax = _bounds_from_pool(k)
    sc = oracle.page_scores(q, kmin, kmax, t, l)
    sel = oracle.select(sc, oracle.budget(1.0, t.shape[1]))
    got = oracle.sparse_decode(q, k, v, t, l, sel, num_splits=4, ratio=1.0)
    assert_close(got, oracle.paged_decode(q, k, v, t, l), 1e-6, 1e-5)


def test_sparse_budget_keeps_sink_and_recent_pages():
    q, k, v, t, l = paged_case([2048], seed=4)
    kmin, kmax = _bounds_from_pool(k)
    sel = oracle.select(oracle.page_scores(q, kmin, kmax, t, l), oracle.budget(0.25, t.shape[1]))
    for h in range(2):
        s = set(sel[0, h].tolist())
        assert {0, 126, 127} <= s
    keep = [[sorted(set(sel[0, h].tolist())) for h in range(2)]]
    assert_close(oracle.sparse_decode(q, k, v, t, l, sel, ratio=0.25),
                 dense_attention(q, k, v, t, l, keep_pages=keep), ATOL, RTOL)


# ---------------------------------------------------------------- gather --


def test_gather_follows_the_slot_rule():
    q, k, v, t, l = paged_case([40, 17, 0])
    g = oracle.gather(k, t, l, 48)
    for b in range(3):
        L = int(l[b])
        for p in range(L):
            slot = int(t[b, p // 16]) * 16 + p % 16
            np.testing.assert_array_equal(g[b, :, p], k.reshape(-1, 2, 128)[slot])
        # past the length: flat slot 0 (the reference pads its slot table with 0)
        np.testing.assert_array_equal(g[b, :, L:], np.broadcast_to(
            k.reshape(-1, 2, 128)[0][:, None], (2, 48 - L, 128)))
