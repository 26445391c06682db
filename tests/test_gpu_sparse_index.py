"""HIP page selection (indexer, top-k, bounds) against the CPU oracle, on an
MI355X.

Selection is integer work on given scores: ``select`` is compared
entry-for-entry with the oracle's stable descending sort (ties -> lower page,
the rule both sides document; the reference's torch.topk leaves tie order
open).  Scores are fp32 sums of exact fp16 products whose summation order
differs from the oracle's, so they are compared at rtol 1e-5, and the
selection the GPU makes from its own scores is compared as a *set* with the
oracle's, allowing swaps only across a score gap below 1e-4 relative (the
reference's own indexer test tolerance, tests/test_phase14_sparse_kernels.py:
92-107).  Bounds are fp16 min/max: bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.cases import assert_close, paged_case

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

ATOL, RTOL = 2e-3, 1e-2


def dev(*arrays):
    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def ps():
    from latentserve_amd.kernels.hip import paged_sparse
    return paged_sparse


def bounds_of(k_pool):
    return k_pool.min(axis=1), k_pool.max(axis=1)


def index_case(lengths, width=None, n_rep=6, seed=0, h_kv=2):
    q, k, v, t, l = paged_case(lengths, h_kv=h_kv, n_rep=n_rep, seed=seed, width=width)
    kmin, kmax = bounds_of(k)
    return q, k, v, t, l, np.ascontiguousarray(kmin), np.ascontiguousarray(kmax)


def sets_agree(got, want, scores, k_rows, tol=1e-4):
    """got/want: selected page lists per (b, h); disagreements only where the
    oracle's scores of the swapped pages sit within tol of the threshold."""
    b, h = scores.shape[:2]
    for i in range(b):
        for j in range(h):
            g, w = set(got[i][j]), set(want[i][j])
            if g == w:
                continue
            thr = min(scores[i, j, p] for p in w) if w else 0.0
            for p in g ^ w:
                s = scores[i, j, p]
                assert np.isfinite(s) and abs(s - thr) <= tol * max(1.0, abs(thr)), \
                    (i, j, p, s, thr)


# ------------------------------------------------------------- scores ----
@pytest.mark.parametrize("n_rep", [1, 6, 16])
def test_page_scores_match_the_oracle(n_rep):
    q, k, v, t, l, kmin, kmax = index_case([2048 + 5, 700, 33, 1, 0], width=200, n_rep=n_rep)
    want = oracle.page_scores(q, kmin, kmax, t, l, recent=2)
    Q, KN, KX, T, L = dev(q, kmin, kmax, t, l)
    got = ps().page_scores(Q, KN, KX, T, L, recent=2).cpu().numpy()
    assert got.shape == want.shape
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    assert np.allclose(got[fin], want[fin], rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("recent", [0, 1, 2, 5])
def test_forced_pages_follow_recent(recent):
    q, k, v, t, l, kmin, kmax = index_case([40 * 16 + 3, 16 * 7], width=48)
    Q, KN, KX, T, L = dev(q, kmin, kmax, t, l)
    got = ps().page_scores(Q, KN, KX, T, L, recent=recent).cpu().numpy()
    for b, n in enumerate([41, 7]):
        forced = {0} | set(range(max(0, n - recent), n))
        assert set(np.flatnonzero(np.isposinf(got[b, 0]))) == forced
        assert set(np.flatnonzero(np.isneginf(got[b, 0]))) == set(range(n, 48))


def test_block_ids_outside_the_pool_score_minus_inf():
    q, k, v, t, l, kmin, kmax = index_case([64 * 16], width=64)
    t = t.copy()
    t[0, 10] = 10 ** 6
    t[0, 11] = -3
    Q, KN, KX, T, L = dev(q, kmin, kmax, t, l)
    got = ps().page_scores(Q, KN, KX, T, L).cpu().numpy()
    assert np.isneginf(got[0, :, 10]).all() and np.isneginf(got[0, :, 11]).all()
    assert np.isfinite(got[0, :, 12]).all()


# ------------------------------------------------------------- select ----
def random_scores(b, h, p, seed, ties=False):
    rng = np.random.default_rng(seed)
    s = rng.standard_normal((b, h, p)).astype(np.float32)
    if ties:
        s = np.round(s * 2) / 2          # a handful of distinct values, many ties
    s[:, :, 0] = np.inf
    s[:, :, -3:] = -np.inf
    return s


@pytest.mark.parametrize("p,k", [(1, 1), (37, 5), (200, 200), (2048, 1024), (8192, 4000)])
@pytest.mark.parametrize("ties", [False, True])
def test_select_sorted_equals_the_oracle(p, k, ties):
    s = random_scores(3, 2, p, seed=p + k, ties=ties)
    got = ps().select(dev(s)[0], k, sorted=True).cpu().numpy()
    assert np.array_equal(got, oracle.select(s, k))


@pytest.mark.parametrize("p,k", [(37, 5), (2048, 1024), (1000, 999)])
def test_select_unsorted_is_the_top_k_in_page_order(p, k):
    s = random_scores(2, 2, p, seed=k, ties=True)
    got = ps().select(dev(s)[0], k).cpu().numpy()
    want = np.sort(oracle.select(s, k), axis=-1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("ratio", [0.25, 0.5, 0.9])
def test_select_ratio_puts_each_sequences_budget_first(ratio):
    p = 512
    lens = np.array([p * 16, 300 * 16 + 1, 17, 0, 3 * 16], dtype=np.int32)
    s = random_scores(len(lens), 2, p, seed=3, ties=True)
    k = ps().budget(ratio, p)
    got = ps().select(dev(s)[0], k, seq_lens=dev(lens)[0], ratio=ratio).cpu().numpy()
    full = oracle.select(s, k)
    for b, length in enumerate(lens):
        pages = min(p, (int(length) + 15) // 16)
        n = oracle.sparse_count(pages, k, ratio, 2)
        for h in range(2):
            assert np.array_equal(got[b, h, :n], np.sort(full[b, h, :n])), (b, h)
            assert np.array_equal(got[b, h, n:], np.sort(full[b, h, n:k])), (b, h)


def test_select_zero_k_and_errors():
    s = dev(random_scores(1, 1, 10, 0))[0]
    assert ps().select(s, 0).shape == (1, 1, 0)
    with pytest.raises(ValueError):
        ps().select(s, 11)


# ------------------------------------------------------- fused index -----
@pytest.mark.parametrize("width", [200, 33, 2048])
def test_fused_index_select_equals_scores_then_select(width):
    lens = [width * 16, width * 8 + 3, 100, 1]
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, seed=width)
    Q, KN, KX, T, L = dev(q, kmin, kmax, t, l)
    kk = ps().budget(0.5, width)
    for _ in range(3):      # the arrival counters must come back to zero every call
        fused = ps().index_select(Q, KN, KX, T, L, kk, 0.5).cpu().numpy()
        scores = ps().page_scores(Q, KN, KX, T, L)
        split = ps().select(scores, kk, seq_lens=L, ratio=0.5).cpu().numpy()
        assert np.array_equal(fused, split)


def test_gpu_selection_agrees_with_the_oracle_selection():
    width = 512
    lens = [width * 16, 5000, 777]
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, seed=9)
    Q, KN, KX, T, L = dev(q, kmin, kmax, t, l)
    kk = ps().budget(0.5, width)
    got = ps().index_select(Q, KN, KX, T, L, kk, 0.5).cpu().numpy()
    scores = oracle.page_scores(q, kmin, kmax, t, l)
    full = oracle.select(scores, kk)
    g, w = [], []
    for b, length in enumerate(lens):
        n = oracle.sparse_count((length + 15) // 16, kk, 0.5, 2)
        g.append([got[b, h, :n] for h in range(2)])
        w.append([full[b, h, :n] for h in range(2)])
    sets_agree(g, w, scores, None)


# ------------------------------------------------------- mass scoring ----
@pytest.mark.parametrize("n_rep,recent", [(6, 2), (1, 0), (16, 3)])
def test_page_scores_mass_match_the_oracle(n_rep, recent):
    width = 300
    lens = [width * 16, 2500, 700, 40, 1, 0]
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, n_rep=n_rep, seed=n_rep)
    Q, T, L, KN, KX = dev(q, t, l, kmin, kmax)
    got = ps().page_scores_mass(Q, KN, KX, T, L, recent=recent).cpu().numpy()
    want = oracle.page_scores_mass(q, kmin, kmax, t, l, recent=recent)
    fin = np.isfinite(want)
    assert np.array_equal(got[~fin], want[~fin])
    assert_close(got[fin], want[fin], 1e-7, 1e-4, f"mass n_rep={n_rep}")


@pytest.mark.parametrize("fused", [True, False])
def test_sparse_attention_mass_scoring(fused):
    """scoring="mass" (kernels/cuda/paged_sparse.py:236-237): the pages the
    GPU keeps agree with the oracle's top-k of the oracle's mass scores, and
    the output is the oracle's attention over the GPU's pages."""
    width = 256
    lens = [width * 16, 2500, 700, 40]
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, seed=11)
    Q, K, V, T, L, KN, KX = dev(q, k, v, t, l, kmin, kmax)
    out = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=0.25, scoring="mass",
                                fused=fused).float().cpu().numpy()
    kk = ps().budget(0.25, width)
    mass = ps().page_scores_mass(Q, KN, KX, T, L)
    sel = ps().select(mass, kk, seq_lens=L, ratio=0.25).cpu().numpy()
    want_scores = oracle.page_scores_mass(q, kmin, kmax, t, l)
    for i, length in enumerate(lens):
        n = oracle.sparse_count(-(-length // 16), kk, 0.25)
        want_rows = oracle.select(want_scores[i:i + 1], n)[0]
        sets_agree([[sel[i, j, :n].tolist() for j in range(2)]],
                   [[want_rows[j].tolist() for j in range(2)]], want_scores[i:i + 1], None,
                   tol=1e-4)
    want = oracle.sparse_decode(q, k, v, t, l, sel, ratio=0.25, recent=2)
    assert_close(out, want, ATOL, RTOL, f"mass fused={fused}")


# --------------------------------------------------- sparse attention ----
@pytest.mark.parametrize("ratio", [0.25, 0.5, 1.0])
def test_sparse_attention_end_to_end(ratio):
    width = 256
    lens = [width * 16, 2500, 700, 40]
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, seed=int(ratio * 8))
    Q, K, V, T, L, KN, KX = dev(q, k, v, t, l, kmin, kmax)
    out = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio).float().cpu().numpy()
    kk = ps().budget(ratio, width)
    sel = ps().index_select(Q, KN, KX, T, L, kk, ratio).cpu().numpy()
    want = oracle.sparse_decode(q, k, v, t, l, sel, ratio=ratio, recent=2)
    assert_close(out, want, ATOL, RTOL, f"ratio={ratio}")
    if ratio >= 1.0:
        assert_close(out, oracle.paged_decode(q, k, v, t, l), ATOL, RTOL, "full = dense")


@pytest.mark.parametrize("width,lens,ratio,splits", [
    (256, [256 * 16, 2500, 700, 40], 0.5, 1),          # one split: the whole list a group
    (256, [256 * 16, 3333, 17], 0.3, 7),
    (3000, [3000 * 16, 10000, 1], 0.5, None),          # rows past 2048 pages: 32 keys a thread
    (2200, [2200 * 16], 1.0, 1),                       # k 2200 > 1024 a split: splits raised to 3
])
def test_selecting_decode_attends_the_selected_pages(width, lens, ratio, splits):
    """The decode that selects its own lists from the scores attends what
    index_select's lists give the oracle, and agrees with the three-launch
    path."""
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, seed=width + len(lens))
    Q, K, V, T, L, KN, KX = dev(q, k, v, t, l, kmin, kmax)
    out = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio, num_splits=splits)
    three = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio, num_splits=splits,
                                  fused=False)
    torch.cuda.synchronize()
    kk = ps().budget(ratio, width)
    sel = ps().index_select(Q, KN, KX, T, L, kk, ratio).cpu().numpy()
    want = oracle.sparse_decode(q, k, v, t, l, sel, ratio=ratio, recent=2)
    assert_close(out.float().cpu().numpy(), want, ATOL, RTOL, f"w={width} r={ratio} s={splits}")
    assert (out.float() - three.float()).abs().max().item() < 1e-3


def test_sparse_attention_graph_replays():
    width = 128
    q, k, v, t, l, kmin, kmax = index_case([width * 16, 900], width=width, seed=4)
    Q, K, V, T, L, KN, KX = dev(q, k, v, t, l, kmin, kmax)
    eager = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=0.5).clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=0.5)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        ps().page_scores(Q, KN, KX, T, L)      # eager work between replays
        torch.cuda.synchronize()


# ------------------------------------------------------------- bounds ----
def test_rebuild_bounds_is_exact():
    _, k, _, _, _ = paged_case([300], seed=2)
    K = dev(k)[0]
    kmin = torch.empty(k.shape[0], k.shape[2], k.shape[3], dtype=torch.float16, device="cuda")
    kmax = torch.empty_like(kmin)
    ps().rebuild_bounds(K, kmin, kmax)
    lo, hi = bounds_of(k)
    assert np.array_equal(kmin.cpu().numpy().view(np.uint16), lo.view(np.uint16))
    assert np.array_equal(kmax.cpu().numpy().view(np.uint16), hi.view(np.uint16))


def test_update_bounds_is_bit_exact_over_a_decode_stream():
    rng = np.random.default_rng(5)
    nb, h, d, b = 12, 2, 128, 3
    kmin = rng.standard_normal((nb, h, d)).astype(np.float16)
    kmax = kmin.copy()
    KN, KX = dev(kmin, kmax)
    starts = np.array([0, 4 * 16 + 9, 9 * 16], dtype=np.int64)   # a mid-page start too
    for step in range(20):
        k_new = rng.standard_normal((b, h, d)).astype(np.float16)
        slots = starts + step
        oracle.bounds_update(k_new, slots, kmin, kmax)
        kn, sl = dev(k_new, slots)
        ps().update_bounds(kn, sl, KN, KX)
    torch.cuda.synchronize()
    assert np.array_equal(KN.cpu().numpy().view(np.uint16), kmin.view(np.uint16))
    assert np.array_equal(KX.cpu().numpy().view(np.uint16), kmax.view(np.uint16))


def test_update_bounds_skips_slots_outside_the_pool():
    kmin = torch.zeros(2, 1, 128, dtype=torch.float16, device="cuda")
    kmax = torch.zeros_like(kmin)
    k_new = torch.ones(2, 1, 128, dtype=torch.float16, device="cuda")
    slots = torch.tensor([2 * 16, -1], dtype=torch.int64, device="cuda")
    ps().update_bounds(k_new, slots, kmin, kmax)
    torch.cuda.synchronize()
    assert kmin.abs().sum().item() == 0 and kmax.abs().sum().item() == 0


# ------------------------------------------- the decode's own selection ----
def _crafted_scores(kind, b, h, p, lens, seed):
    """Score rows that drive the selecting decode's threshold search through
    each of its outcomes: a threshold bin taken whole, ranked directly, ties
    taken in page order, another round over a crowded bin."""
    rng = np.random.default_rng(seed)
    s = rng.standard_normal((b, h, p)).astype(np.float32)
    if kind == "ties":
        s = np.round(s * 2) / 2                         # few values, many ties
    elif kind == "equal":
        s[:] = 1.5                                      # one finite value
    elif kind == "outlier":
        s[:, :, p // 2] = 1e30                          # stretches the range: a crowded bin
        s[:, :, p // 3] = -1e30
    elif kind == "forced":
        s[:, :, : p // 2] = np.inf                      # more +inf pages than the budget
    elif kind == "ulps":
        # adjacent floats: keys one apart, bins of width one
        s = (np.float32(1.0) + rng.integers(0, 40, (b, h, p)).astype(np.float32) *
             np.finfo(np.float32).eps).astype(np.float32)
    elif kind == "zeros":
        s = np.where(rng.random((b, h, p)) < 0.5, np.float32(0.0), np.float32(-0.0))
        s[:, :, ::7] = -1.0
    elif kind == "dead":
        s[:, :, 3::4] = -np.inf                         # dead pages inside the length
    s[:, :, 0] = np.inf
    for i, n in enumerate(lens):
        np_ = -(-n // 16)
        s[i, :, np_:] = -np.inf                         # past the end
        s[i, :, max(0, np_ - 2):np_] = np.inf           # recent pages
    return np.ascontiguousarray(s.astype(np.float32))


@pytest.mark.parametrize("kind", ["normal", "ties", "equal", "outlier", "forced", "ulps",
                                  "zeros", "dead"])
@pytest.mark.parametrize("width,ratio,splits", [(2048, 0.5, 32), (300, 0.3, 4), (3000, 0.5, 8)])
def test_selecting_decode_selects_what_select_does(kind, width, ratio, splits):
    """The decode that selects from given scores attends exactly the lists
    select() gives the list decode: bit-equal outputs (same lists, same split
    partition), for score rows that exercise every outcome of its search."""
    import ctypes
    from latentserve_amd import _lib
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh
    lens = [width * 16, width * 16 // 3 + 5, 40, 0]
    q, k, v, t, l = paged_case(lens, h_kv=2, n_rep=6, seed=width, width=width)
    Q, K, V, T, L = dev(q, k, v, t, l)
    s = _crafted_scores(kind, len(lens), 2, width, lens, seed=width + len(kind))
    S_ = dev(s)[0]
    kk = ps().budget(ratio, width)
    sel = ps().select(S_, kk, seq_lens=L, ratio=ratio)
    want = ps().sparse_decode(Q, K, V, T, L, sel, num_splits=splits, ratio=ratio).clone()
    b, h, n_rep, d = Q.shape
    buf, work, cnt = pdh._buffers("sparse", b, h, splits, n_rep, Q.device)
    P, St = _lib.ptr, _lib.strides
    rc = _lib.lib().ls_sparse_attention_fp16(
        P(Q), St(Q, 3), P(K), P(V), St(K, 3), K.shape[0], P(T), T.stride(0), T.shape[1], P(L),
        P(S_), St(S_, 2), width, kk, float(ratio), 2, P(buf), St(buf, 3), P(work), P(cnt),
        b, h, n_rep, d, 16, splits, 0, float(1.0 / np.sqrt(d)), _lib.stream_of(Q.device))
    _lib.check(rc, "ls_sparse_attention_fp16")
    torch.cuda.synchronize()
    got = buf[:, :, :n_rep]
    # (the waves claim pages dynamically: the same lists, merged in another
    # order; the lists themselves are checked exactly through select())
    err = (got.float() - want.float()).abs().max().item()
    assert err < 1e-3, (kind, err)


@pytest.mark.parametrize("kind", ["normal", "ties", "equal", "outlier", "forced", "ulps",
                                  "zeros", "dead"])
@pytest.mark.parametrize("p,k", [(2048, 1024), (300, 91), (3000, 1500), (5, 2), (600, 600)])
def test_one_threshold_select_equals_the_oracle(kind, p, k):
    """select() without a ratio takes one threshold (the search the selecting
    decode runs): the top k in page order, ties to the lower page, exactly the
    oracle's set."""
    lens = [p * 16, p * 16 // 3 + 5, 40, 0]
    s = _crafted_scores(kind, len(lens), 2, p, lens, seed=p + k + len(kind))
    got = ps().select(dev(s)[0], k).cpu().numpy()
    want = np.sort(oracle.select(s, k), axis=-1)
    assert np.array_equal(got, want), kind


@pytest.mark.parametrize("h_kv,n_rep,width,lens,splits", [
    (1, 1, 17, [17 * 16, 5, 0], 3),                     # one head a group, empty sequence
    (2, 4, 300, [300 * 16, 2000, 1, 16], None),
    (3, 8, 300, [4000, 300 * 16], 5),                   # odd heads: one head a group
    (2, 6, 2048, [2048 * 16, 700], 32),                 # the bench's row length
    (2, 6, 64, [64 * 16, 100], 64),                     # more splits than a row has list entries
])
def test_one_launch_bounds_path_matches_three_launches_and_the_oracle(h_kv, n_rep, width, lens,
                                                                      splits):
    """Bounds scoring in one launch (workgroups score, exchange, select and
    attend) against index + select + list decode and against the oracle over
    index_select's lists, across head counts, query rows, row lengths, split
    counts and ragged lengths; twice, so the score buffer's reset is
    exercised."""
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, n_rep=n_rep, h_kv=h_kv,
                                           seed=width + n_rep)
    Q, K, V, T, L, KN, KX = dev(q, k, v, t, l, kmin, kmax)
    ratio = 0.5
    kk = ps().budget(ratio, width)
    sel = ps().index_select(Q, KN, KX, T, L, kk, ratio).cpu().numpy()
    want = oracle.sparse_decode(q, k, v, t, l, sel, ratio=ratio, recent=2)
    for rep in range(2):
        one = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio, num_splits=splits)
        three = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio, num_splits=splits,
                                      fused=False)
        torch.cuda.synchronize()
        assert_close(one.float().cpu().numpy(), want, ATOL, RTOL, f"one launch, rep {rep}")
        assert (one.float() - three.float()).abs().max().item() < 1e-3, rep


@pytest.mark.parametrize("order,width,splits", [("rising", 2048, 32), ("falling", 2048, 32),
                                                 ("chunks", 2048, 16), ("rising", 300, 5),
                                                 ("chunks", 1024, 16)])
def test_one_launch_path_with_skewed_shares(order, width, splits):
    """Page scores laid out so that the workgroups' shares of a row hold very
    different numbers of selected pages (rising / falling with the page, or
    alternating chunks of high and low pages): the one-launch path's
    partition moves a share's surplus to the groups short of pages, and the
    pages each group requested before the selection (its share's best) are
    often not its items or not selected at all.  Every selected page must
    still be attended exactly once: the output equals the three-launch path
    and the oracle over the same lists."""
    lens = [width * 16, width * 16 - 37]
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, seed=width + 3)
    q = np.abs(q)                            # scores monotone in the bounds below
    pages = np.arange(width)
    c = {"rising": pages / width, "falling": 1.0 - pages / width,
         "chunks": ((pages // 96) % 2) + pages / (4.0 * width)}[order]
    for b in range(len(lens)):
        kmin[t[b]] = kmax[t[b]] = c.astype(np.float16)[:, None, None]
    Q, K, V, T, L, KN, KX = dev(q, k, v, t, l, kmin, kmax)
    ratio = 0.5
    kk = ps().budget(ratio, width)
    sel = ps().index_select(Q, KN, KX, T, L, kk, ratio).cpu().numpy()
    want = oracle.sparse_decode(q, k, v, t, l, sel, ratio=ratio, recent=2)
    for rep in range(2):
        one = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio, num_splits=splits)
        three = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio, num_splits=splits,
                                      fused=False)
        torch.cuda.synchronize()
        assert_close(one.float().cpu().numpy(), want, ATOL, RTOL, f"{order}, rep {rep}")
        assert (one.float() - three.float()).abs().max().item() < 1e-3, (order, rep)


@pytest.mark.parametrize("width,lens,splits", [(2048, [2048 * 16, 5000], 32), (300, [4800, 7], 5)])
def test_one_launch_path_with_the_fallback_forced(width, lens, splits):
    """With the wait bound at 0 every workgroup of the one-launch path scores
    whatever it finds missing itself (the fallback that keeps a launch from
    depending on its workgroups being resident together): the same output,
    and the score buffer's count words left all ones for the next call."""
    from latentserve_amd import _lib
    q, k, v, t, l, kmin, kmax = index_case(lens, width=width, seed=width + 1)
    Q, K, V, T, L, KN, KX = dev(q, k, v, t, l, kmin, kmax)
    ratio = 0.5
    base = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio, num_splits=splits).clone()
    try:
        _lib.lib().ls_set_coop_wait_ticks(0)
        for _ in range(2):
            forced = ps().sparse_attention(Q, K, V, T, L, KN, KX, ratio=ratio, num_splits=splits)
            torch.cuda.synchronize()
            assert (forced.float() - base.float()).abs().max().item() < 1e-3
    finally:
        _lib.lib().ls_set_coop_wait_ticks(5000)
    kk = ps().budget(ratio, width)
    sel = ps().index_select(Q, KN, KX, T, L, kk, ratio).cpu().numpy()
    want = oracle.sparse_decode(q, k, v, t, l, sel, ratio=ratio, recent=2)
    assert_close(forced.float().cpu().numpy(), want, ATOL, RTOL, "fallback forced")
    from latentserve_amd.kernels.gqa import _SCRATCH
    for key, buf in _SCRATCH.items():
        if key[0] == "sparse_coop_scores" and buf.shape[2] == (width + 4) // 4 * 4:
            # the word after every row (the count after each head group's
            # first row; untouched after the others)
            assert bool((buf[:, :, width] == -1).all()), "count words not left all ones"
