"""HIP decode kernels against the CPU oracle, on an MI355X.

The bar: fp16 outputs within max-abs 2e-3 and
rel 1e-2 of an fp32 evaluation of the reference formula (oracle/, itself
pinned by tests/test_oracle.py). Cases follow the reference's GPU tests
(tests/test_cuda_decode.py:82-122, 201-254; tests/test_phase14_sparse_kernels.py:
110-163) at the production geometry (H_kv 2, n_rep 6, D 128, page 16).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.cases import assert_close, dense_attention, dequant_pools, int8_case, paged_case

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

ATOL, RTOL = 2e-3, 1e-2


def dev(*arrays):
    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def hip_mod():
    from latentserve_amd.kernels.hip import paged_decode_hip
    return paged_decode_hip


def run_fp16(case, num_splits=None, max_len=None):
    q, k, v, t, l = case
    Q, K, V, T, L = dev(q, k, v, t, l)
    out = hip_mod().paged_decode_hip(Q, K, V, T, L, max_len or int(l.max()), num_splits=num_splits)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_library_is_the_hip_build():
    from latentserve_amd import _lib
    assert _lib.lib().ls_abi_version() == _lib.ABI_VERSION == 19


@pytest.mark.parametrize("splits", [None, 1, 3, 16, 17, 32, 33, 64])
def test_ragged_lengths_match_the_oracle(splits):
    # (16 / 17 and 32 / 33 splits: the edges of the split merge's rounds of
    # 16 and 32 records; 64: two rounds of 32)
    case = paged_case([1024, 300, 61, 17, 1], seed=0)
    want = oracle.paged_decode(*case, num_splits=1)
    assert_close(run_fp16(case, splits), want, ATOL, RTOL, f"splits={splits}")


@pytest.mark.parametrize("batch", [63, 64, 65, 150])
@pytest.mark.parametrize("splits", [None, 3])
def test_large_ragged_batches_match_the_oracle(batch, splits):
    """Split workgroups are dealt to sequences in proportion to their pages,
    one sequence a lane up to 64 sequences and runs of sequences a lane past
    that; empty sequences and a few long ones test both deals."""
    rng = np.random.default_rng(batch)
    lens = rng.integers(0, 120, batch)
    lens[::7] = 0
    lens[3] = 900
    case = paged_case([int(x) for x in lens], seed=batch)
    want = oracle.paged_decode(*case, num_splits=1)
    assert_close(run_fp16(case, splits), want, ATOL, RTOL, f"B={batch} splits={splits}")


@pytest.mark.parametrize("max_len", [None, 4096])
def test_counters_are_zero_after_every_call(max_len):
    """The arrival counts are reset by the group that closes each (sequence,
    head), so back-to-back calls with different split counts (and graph
    replays) start from zero."""
    case = paged_case([4096, 4096, 3000, 17], seed=5)
    want = oracle.paged_decode(*case, num_splits=1)
    for splits in (8, 8, 3, 16):
        assert_close(run_fp16(case, splits, max_len), want, ATOL, RTOL, f"splits={splits}")
        _, _, cnt = hip_mod()._buffers("hip", 4, 2, splits, 6, torch.device("cuda"))
        assert int(cnt.abs().sum()) == 0, cnt.cpu().numpy()


def test_config1_b1_2048_pool256():
    """B1 x 2048, pool of 256 blocks, permuted table."""
    rng = np.random.default_rng(1)
    k = rng.standard_normal((256, 16, 2, 128), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((256, 16, 2, 128), dtype=np.float32).astype(np.float16)
    t = rng.permutation(256)[:128].reshape(1, 128).astype(np.int32)
    q = rng.standard_normal((1, 2, 6, 128), dtype=np.float32).astype(np.float16)
    l = np.array([2048], np.int32)
    want = dense_attention(q, k, v, t, l)
    for splits in (None, 1, 8, 128):
        assert_close(run_fp16((q, k, v, t, l), splits), want, ATOL, RTOL, f"splits={splits}")


@pytest.mark.parametrize("length", [1, 15, 16, 17, 31, 32, 33, 4095, 4096, 4097])
def test_ragged_final_page(length):
    case = paged_case([length], seed=length)
    assert_close(run_fp16(case, 3), dense_attention(*case), ATOL, RTOL, f"len={length}")


def test_empty_and_tiny_sequences():
    case = paged_case([0, 1, 2, 0, 40], seed=5)
    got = run_fp16(case, 4)
    assert (got[0] == 0).all() and (got[3] == 0).all()
    assert_close(got, dense_attention(*case), ATOL, RTOL)


@pytest.mark.parametrize("splits", [5, 33])
@pytest.mark.parametrize("n_rep", [1, 4, 6, 8, 16])
def test_other_group_sizes(n_rep, splits):
    # (33 splits: the split merge's rounds of 32 records and a second round,
    # with the query rows of one to sixteen half-waves)
    case = paged_case([500, 77], n_rep=n_rep, seed=n_rep)
    assert_close(run_fp16(case, splits), dense_attention(*case), ATOL, RTOL,
                 f"n_rep={n_rep} splits={splits}")


def test_four_kv_heads_and_strided_q():
    q, k, v, t, l = paged_case([300, 129], h_kv=4, seed=7)
    Q, K, V, T, L = dev(q, k, v, t, l)
    big = torch.zeros(2, 4, 8, 128, dtype=torch.float16, device="cuda")
    big[:, :, :6] = Q
    out = hip_mod().paged_decode_hip(big[:, :, :6], K, V, T, L, 300, num_splits=2)
    assert_close(out.float().cpu().numpy(), dense_attention(q, k, v, t, l), ATOL, RTOL)


def test_more_splits_than_pages():
    case = paged_case([40, 5, 17], seed=9)
    assert_close(run_fp16(case, 64), dense_attention(*case), ATOL, RTOL)


def test_out_of_range_block_ids_are_not_read():
    """A corrupt table entry must not be dereferenced: the page is skipped."""
    q, k, v, t, l = paged_case([64], seed=3)
    bad = t.copy()
    bad[0, 1] = 10_000_000
    got = run_fp16((q, k, v, bad, l), 2)
    keep = [[[0, 2, 3]] * 2]
    assert_close(got, dense_attention(q, k, v, t, l, keep_pages=keep), ATOL, RTOL)


def test_dispatch_through_the_normal_entry_point():
    from latentserve_amd.kernels.gqa import paged_decode as pd
    q, k, v, t, l = paged_case([700, 33], seed=11)
    Q, K, V, T, L = dev(q, k, v, t, l)
    pd.set_decode_backend("hip")
    got = pd.paged_decode_attention(Q, K, V, T, L, max_seq_len=700)
    torch.cuda.synchronize()
    assert_close(got.float().cpu().numpy(), oracle.paged_decode(q, k, v, t, l), ATOL, RTOL)
    with pytest.raises(ValueError):
        pd.set_decode_backend("cuda")


def test_ineligible_inputs_raise_instead_of_falling_back():
    from latentserve_amd.kernels.gqa import paged_decode as pd
    q, k, v, t, l = paged_case([64], d=64, seed=1)
    Q, K, V, T, L = dev(q, k, v, t, l)
    with pytest.raises(ValueError, match="128"):
        pd.paged_decode_attention(Q, K, V, T, L, max_seq_len=64)
    with pytest.raises(ValueError):
        pd.paged_decode_attention(*[torch.from_numpy(x) for x in (q, k, v, t, l)])


def test_survives_graph_capture_and_replays():
    """Graph replays read the current inputs; the arrival counters reset
    themselves, so every replay (with eager work between) is correct."""
    q, k, v, t, l = paged_case([500, 200], seed=12)
    Q, K, V, T, L = dev(q, k, v, t, l)
    f = hip_mod().paged_decode_hip
    f(Q, K, V, T, L, 500, num_splits=8)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f(Q, K, V, T, L, 500, num_splits=8)
    rng = np.random.default_rng(0)
    for rep in range(4):
        qn = rng.standard_normal(q.shape, dtype=np.float32).astype(np.float16)
        Q.copy_(torch.from_numpy(qn).cuda())
        eager = f(Q, K, V, T, L, 500, num_splits=3).clone()
        g.replay()
        torch.cuda.synchronize()
        want = oracle.paged_decode(qn, k, v, t, l)
        assert_close(out.float().cpu().numpy(), want, ATOL, RTOL, f"replay {rep}")
        assert_close(eager.float().cpu().numpy(), want, ATOL, RTOL, f"eager {rep}")


def test_combine_splits_matches_the_oracle():
    from latentserve_amd.kernels.gqa import paged_decode as pd
    rng = np.random.default_rng(4)
    acc = rng.standard_normal((2, 2, 5, 16, 128), dtype=np.float32)
    m = rng.standard_normal((2, 2, 5, 16), dtype=np.float32)
    l = rng.random((2, 2, 5, 16), dtype=np.float32) + 0.5
    m[0, 0, 2] = -np.inf
    l[0, 0, 2] = 0
    m[1, 1, :] = -np.inf
    l[1, 1, :] = 0
    A, M, Lt = dev(acc, m, l)
    for dt in (torch.float32, torch.float16):
        got = pd.combine_splits(A, M, Lt, dt)
        torch.cuda.synchronize()
        assert_close(got.float().cpu().numpy(), oracle.combine(acc, m, l), 1e-3, 1e-3, str(dt))


# ---------------------------------------------------------------- INT8 ----


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("res", [False, True])
@pytest.mark.parametrize("splits", [None, 3, 64])
def test_int8_matches_the_oracle(asym, res, splits):
    (q, k, v, t, l), ex = int8_case([1024, 300, 61, 17, 1], asym=asym, res=res)
    want = oracle.paged_decode(q, k, v, t, l, num_splits=1, **ex)
    Q, K, V, T, L = dev(q, k, v, t, l)
    dex = {key: dev(val)[0] for key, val in ex.items()}
    got = hip_mod().paged_decode_hip(Q, K, V, T, L, 1024, num_splits=splits, **dex)
    torch.cuda.synchronize()
    assert_close(got.float().cpu().numpy(), want, ATOL, RTOL, f"asym={asym} res={res}")


@pytest.mark.parametrize("h_kv", [1, 3, 4])
@pytest.mark.parametrize("asym", [False, True])
def test_int8_head_counts(h_kv, asym):
    """An even head count takes two heads a workgroup (each head's last page
    from the residual by a wave of its own half), an odd count one, for
    symmetric and asymmetric pools: every head's output against the
    oracle."""
    (q, k, v, t, l), ex = int8_case([700, 33, 16, 290], asym=asym, res=True, h_kv=h_kv,
                                    seed=11 + h_kv)
    want = oracle.paged_decode(q, k, v, t, l, num_splits=1, **ex)
    Q, K, V, T, L = dev(q, k, v, t, l)
    dex = {key: dev(val)[0] for key, val in ex.items()}
    for splits in (None, 5):
        got = hip_mod().paged_decode_hip(Q, K, V, T, L, 700, num_splits=splits, **dex)
        torch.cuda.synchronize()
        assert_close(got.float().cpu().numpy(), want, ATOL, RTOL, f"h_kv={h_kv} splits={splits}")


def test_int8_equals_fp16_attention_over_the_dequantised_cache():
    (q, k, v, t, l), ex = int8_case([777, 64], res=True, seed=3)
    kd, vd = dequant_pools(k, v, ex["k_scale"], ex["v_scale"])
    want = dense_attention(q, kd, vd, t, l, k_res=ex["k_residual"], res_rows=ex["res_rows"])
    Q, K, V, T, L = dev(q, k, v, t, l)
    dex = {key: dev(val)[0] for key, val in ex.items()}
    got = hip_mod().paged_decode_hip(Q, K, V, T, L, 777, **dex)
    torch.cuda.synchronize()
    assert_close(got.float().cpu().numpy(), want, ATOL, RTOL)


def test_int8_eligibility_needs_a_complete_set_of_arguments():
    pdh = hip_mod()
    (q, k, v, t, l), ex = int8_case([200, 40], asym=True, res=True)
    Q, K = dev(q, k)
    dex = {key: dev(val)[0] for key, val in ex.items()}
    assert pdh.eligible(Q, K, **dex)
    assert not pdh.eligible(Q, K, **{kk: vv for kk, vv in dex.items() if kk != "v_scale"})
    assert not pdh.eligible(Q, K, **{kk: vv for kk, vv in dex.items() if kk != "v_zero"})
    assert not pdh.eligible(Q, K, **{kk: vv for kk, vv in dex.items() if kk != "res_rows"})


def test_int8_survives_graph_capture():
    (q, k, v, t, l), ex = int8_case([500, 200], res=True, seed=6)
    Q, K, V, T, L = dev(q, k, v, t, l)
    dex = {key: dev(val)[0] for key, val in ex.items()}
    f = hip_mod().paged_decode_hip
    f(Q, K, V, T, L, 500, **dex)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f(Q, K, V, T, L, 500, **dex)
    rng = np.random.default_rng(1)
    for rep in range(3):
        qn = rng.standard_normal(q.shape, dtype=np.float32).astype(np.float16)
        Q.copy_(torch.from_numpy(qn).cuda())
        g.replay()
        torch.cuda.synchronize()
        want = oracle.paged_decode(qn, k, v, t, l, **ex)
        assert_close(out.float().cpu().numpy(), want, ATOL, RTOL, f"replay {rep}")


# -------------------------------------------------------------- sparse ----


@pytest.mark.parametrize("num_splits", [None, 1, 3])
def test_sparse_kernel_attends_exactly_the_given_pages(num_splits):
    from latentserve_amd.kernels.hip import paged_sparse as ps
    q, k, v, t, l = paged_case([700, 150], seed=2)
    picks = [[0, 3, 7, 12, 20, 43], [0, 2, 5, 9, 30, 40]]          # seq 1 has 10 pages
    sel = np.array([[p, p[::-1]] for p in picks], dtype=np.int32)
    Q, K, V, T, L, SEL = dev(q, k, v, t, l, sel)
    got = ps.sparse_decode(Q, K, V, T, L, SEL, num_splits=num_splits)
    torch.cuda.synchronize()
    keep = [[[p for p in picks[b] if p < -(-int(l[b]) // 16)]] * 2 for b in range(2)]
    assert_close(got.float().cpu().numpy(), dense_attention(q, k, v, t, l, keep_pages=keep),
                 ATOL, RTOL)
    assert_close(got.float().cpu().numpy(), oracle.sparse_decode(q, k, v, t, l, sel), ATOL, RTOL)


def test_sparse_in_kernel_budget_follows_each_length():
    from latentserve_amd.kernels.hip import paged_sparse as ps
    q, k, v, t, l = paged_case([2048, 900, 33], seed=8)
    rng = np.random.default_rng(3)
    sel = np.stack([np.stack([rng.permutation(t.shape[1]) for _ in range(2)]) for _ in range(3)])
    sel = sel[..., :64].astype(np.int32)
    Q, K, V, T, L, SEL = dev(q, k, v, t, l, sel)
    got = ps.sparse_decode(Q, K, V, T, L, SEL, num_splits=4, ratio=0.25, recent=2)
    torch.cuda.synchronize()
    want = oracle.sparse_decode(q, k, v, t, l, sel, num_splits=1, ratio=0.25, recent=2)
    assert_close(got.float().cpu().numpy(), want, ATOL, RTOL)


def test_sparse_full_selection_is_dense():
    """The whole list (ratio None) in any order, and the in-kernel budget at
    ratio 1.0 over a list whose first entries are the sequence's pages, both
    reproduce dense attention."""
    from latentserve_amd.kernels.hip import paged_sparse as ps
    q, k, v, t, l = paged_case([1024, 300], seed=3)
    rev = np.ascontiguousarray(np.tile(np.arange(t.shape[1], dtype=np.int32)[::-1], (2, 2, 1)))
    asc = np.ascontiguousarray(np.tile(np.arange(t.shape[1], dtype=np.int32), (2, 2, 1)))
    Q, K, V, T, L, REV, ASC = dev(q, k, v, t, l, rev, asc)
    dense = hip_mod().paged_decode_hip(Q, K, V, T, L, 1024).float().cpu().numpy()
    got = ps.sparse_decode(Q, K, V, T, L, REV).float().cpu().numpy()
    assert_close(got, dense, ATOL, RTOL, "whole list")
    got = ps.sparse_decode(Q, K, V, T, L, ASC, ratio=1.0).float().cpu().numpy()
    assert_close(got, dense, ATOL, RTOL, "ratio 1.0")
    # A budgeted call over an unsorted list attends exactly the first n entries.
    got = ps.sparse_decode(Q, K, V, T, L, REV, ratio=1.0).float().cpu().numpy()
    assert_close(got, oracle.sparse_decode(q, k, v, t, l, rev, ratio=1.0), ATOL, RTOL, "budget")


@pytest.mark.parametrize("max_len", [1, 700, 3000, 1 << 20])
def test_any_max_seq_len_gives_the_same_result(max_len):
    """max_seq_len only sets the partition of pages over splits: too small a
    bound is re-derived on the device per sequence, too large wastes splits;
    the output never changes."""
    case = paged_case([2900, 700, 33, 1], seed=21)
    want = dense_attention(*case)
    for splits in (1, 5, 16):
        assert_close(run_fp16(case, splits, max_len=max_len), want, ATOL, RTOL,
                     f"max_len={max_len} splits={splits}")


def test_kernel_resources_report_no_spills():
    """Every decode and page-subset kernel as the runtime loaded it
    (kernel_resources, the reference's kernels/cuda/paged_decode_cuda.py:
    163-186 and paged_sparse.py:254-265): no private (spill) memory, and the
    decode walks fit one workgroup of 8 waves (paired heads) a CU."""
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh
    from latentserve_amd.kernels.hip import paged_sparse as ps
    seen = {}
    for variant, asym, res in (("fp16", False, False), ("int8", False, False),
                               ("int8", False, True), ("int8", True, False), ("int8", True, True)):
        for heads in (2, 3):
            r = pdh.kernel_resources(variant=variant, asym=asym, has_res=res, kv_heads=heads,
                                     min_blocks=12)
            seen[(variant, asym, res, heads)] = r
            assert r["local_bytes"] == 0, (variant, asym, res, heads, r)
            assert r["groups_per_cu"] >= 1 and r["threads"] == (512 if heads == 2 else 256), r
            assert r["regs"] <= 256 and r["shared_bytes"] <= 160 * 1024, r
    for name, r in ps.kernel_resources().items():
        assert r["local_bytes"] == 0, (name, r)
        assert r["groups_per_cu"] >= 1, (name, r)
    print(seen)


def test_paged_decode_cuda_name_ignores_min_blocks():
    """The reference's launcher name and signature (min_blocks accepted):
    the same kernel as paged_decode_hip, against the oracle (the waves
    claim pages dynamically, so two calls may differ in the last bit)."""
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh
    case = paged_case([700, 33, 2048], seed=9)
    want = oracle.paged_decode(*case)
    Q, K, V, T, L = dev(*case)
    for mb in (None, 1, 12):
        got = pdh.paged_decode_cuda(Q, K, V, T, L, 2048, num_splits=4, min_blocks=mb)
        assert_close(got.float().cpu().numpy(), want, ATOL, RTOL, f"min_blocks={mb}")

