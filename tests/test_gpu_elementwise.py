"""HIP fused elementwise kernels against the oracle, on an MI355X.

Cases follow the reference's GPU tests (tests/test_phase14_elementwise.py:
161-205): widths 1536 / 128 / 100, the residual sum exact, SiLU at the
Qwen2.5-1.5B intermediate width, RoPE on a strided slice of the fused
projection.  RoPE and the decode-token kernel are held to bit equality with
the oracle (which is bit-equal to Hugging Face's apply_rotary_pos_emb); the
norms to the reference's 4e-3 and to two fp16 steps (the variance is summed
in another order); SiLU to two steps (the exponential's last bit, carried
through the multiply).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.test_elementwise_oracle import ulps

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def fe():
    from latentserve_amd.kernels import fused_elementwise
    return fused_elementwise


def g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("n", [1536, 128, 100, 8960, 12288])
@pytest.mark.parametrize("rows", [1, 7, 16])
def test_rms_norm(n, rows):
    rng = np.random.default_rng(n + rows)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float16)
    w = rng.standard_normal(n).astype(np.float16)
    got = fe().rms_norm(g(x), g(w), 1e-6)
    torch.cuda.synchronize()
    want, _ = oracle.rms_norm(x, w, 1e-6)
    got = got.cpu().numpy()
    np.testing.assert_allclose(got.astype(np.float32), want.astype(np.float32), rtol=4e-3,
                               atol=4e-3)
    assert ulps(got, want).max() <= 2


@pytest.mark.parametrize("n", [1536, 100])
def test_fused_add_rms_norm(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((5, n)).astype(np.float16)
    r = rng.standard_normal((5, n)).astype(np.float16)
    w = rng.standard_normal(n).astype(np.float16)
    y, s = fe().fused_add_rms_norm(g(x), g(r), g(w), 1e-6)
    torch.cuda.synchronize()
    y_ref, s_ref = oracle.rms_norm(x, w, 1e-6, residual=r)
    assert (s.cpu().numpy() == s_ref).all()                 # one exact fp16 add
    assert ulps(y.cpu().numpy(), y_ref).max() <= 2


def test_norm_on_strided_rows_and_into_given_buffers():
    rng = np.random.default_rng(9)
    big = g(rng.standard_normal((4, 3000)).astype(np.float16))
    x = big[:, 8:8 + 1536]                                  # row stride 3000
    r = g(rng.standard_normal((4, 1536)).astype(np.float16))
    w = g(rng.standard_normal(1536).astype(np.float16))
    out, res_out = torch.empty_like(r), torch.empty_like(r)
    y, s = fe().fused_add_rms_norm(x, r, w, 1e-6, out=out, res_out=res_out)
    torch.cuda.synchronize()
    assert y.data_ptr() == out.data_ptr() and s.data_ptr() == res_out.data_ptr()
    y_ref, s_ref = oracle.rms_norm(x.cpu().numpy(), w.cpu().numpy(), 1e-6,
                                   residual=r.cpu().numpy())
    assert (s.cpu().numpy() == s_ref).all() and ulps(y.cpu().numpy(), y_ref).max() <= 2


@pytest.mark.parametrize("inter", [8960, 100])
def test_silu_and_mul(inter):
    rng = np.random.default_rng(inter)
    gu = (rng.standard_normal((3, 2 * inter)) * 4).astype(np.float16)
    got = fe().silu_and_mul(g(gu))
    torch.cuda.synchronize()
    # silu(g) may land one fp16 step apart (the exponential's last bit), which
    # the multiply by u carries to two steps of the product
    d = ulps(got.cpu().numpy(), oracle.silu_and_mul(gu))
    assert d.max() <= 2 and (d == 0).mean() > 0.99


def test_rope_qk_on_a_strided_slice_is_bit_exact():
    """q and k arrive as slices of the fused q/k/v output, their rows strided
    by the whole projection width."""
    rng = np.random.default_rng(3)
    b, s, hq, hk, d = 2, 3, 12, 2, 128
    qkv = g((rng.standard_normal((b, s, (hq + 2 * hk) * d)) * 2).astype(np.float16))
    q, k, _ = qkv.split([hq * d, hk * d, hk * d], dim=-1)
    ang = rng.uniform(0, 6, (b, 1, s, d // 2))
    cos = np.cos(np.concatenate([ang, ang], -1)).astype(np.float16)
    sin = np.sin(np.concatenate([ang, ang], -1)).astype(np.float16)
    qo, ko = fe().rope_qk(q, k, g(cos), g(sin), hq, hk, d)
    torch.cuda.synchronize()
    c, sn = cos.reshape(b, s, 1, d), sin.reshape(b, s, 1, d)
    want_q = oracle.rope(q.cpu().numpy().reshape(b, s, hq, d), c, sn).reshape(b, s, hq * d)
    want_k = oracle.rope(k.cpu().numpy().reshape(b, s, hk, d), c, sn).reshape(b, s, hk * d)
    assert (qo.cpu().numpy() == want_q).all() and (ko.cpu().numpy() == want_k).all()


def test_rope_qk_broadcast_table():
    rng = np.random.default_rng(4)
    b, s, hq, hk, d = 4, 1, 6, 2, 64
    q = (rng.standard_normal((b, s, hq * d))).astype(np.float16)
    k = (rng.standard_normal((b, s, hk * d))).astype(np.float16)
    ang = rng.uniform(0, 6, (1, 1, s, d // 2))
    cos = np.cos(np.concatenate([ang, ang], -1)).astype(np.float16)
    sin = np.sin(np.concatenate([ang, ang], -1)).astype(np.float16)
    qo, ko = fe().rope_qk(g(q), g(k), g(cos), g(sin), hq, hk, d)
    torch.cuda.synchronize()
    want = oracle.rope(q.reshape(b, s, hq, d), cos.reshape(1, s, 1, d), sin.reshape(1, s, 1, d))
    assert (qo.cpu().numpy() == want.reshape(b, s, hq * d)).all()


@pytest.mark.parametrize("bounds", [False, True])
def test_rope_write_decode_matches_the_oracle(bounds):
    rng = np.random.default_rng(5)
    b, hq, hk, d, nb, page = 5, 12, 2, 128, 9, 16
    qkv = rng.standard_normal((b, (hq + 2 * hk) * d)).astype(np.float16)
    ang = rng.uniform(0, 6, (64, d // 2))
    cos = np.cos(np.concatenate([ang, ang], -1)).astype(np.float16)
    sin = np.sin(np.concatenate([ang, ang], -1)).astype(np.float16)
    pos = np.array([0, 17, 63, 200, 5], np.int64)          # 200: past the table
    slots = np.array([3 * page, 8 * page + 15, -1, 1 * page + 4, nb * page + 2], np.int64)
    kp = rng.standard_normal((nb, page, hk, d)).astype(np.float16)
    vp = rng.standard_normal((nb, page, hk, d)).astype(np.float16)
    kmin = rng.standard_normal((nb, hk, d)).astype(np.float16)
    kmax = (kmin + np.float16(0.5)).astype(np.float16)
    K, V, KMIN, KMAX = g(kp), g(vp), g(kmin), g(kmax)
    q = fe().rope_write_decode(g(qkv), g(pos), g(cos), g(sin), g(slots), K, V, hq, hk,
                               kmin=KMIN if bounds else None, kmax=KMAX if bounds else None)
    torch.cuda.synchronize()
    want_q = oracle.rope_write_decode(qkv, pos, cos, sin, slots, kp, vp, hq, hk,
                                      kmin if bounds else None, kmax if bounds else None, page)
    assert (q.cpu().numpy() == want_q).all()
    assert (K.cpu().numpy() == kp).all() and (V.cpu().numpy() == vp).all()
    if bounds:
        assert (KMIN.cpu().numpy() == kmin).all() and (KMAX.cpu().numpy() == kmax).all()


def test_rope_write_decode_into_a_strided_q_buffer():
    rng = np.random.default_rng(6)
    b, hq, hk, d, nb, page = 3, 6, 2, 128, 4, 16
    qkv = rng.standard_normal((b, 1, (hq + 2 * hk) * d)).astype(np.float16)
    tab = np.ones((8, d), np.float16)
    zero = np.zeros((8, d), np.float16)
    buf = torch.zeros((b, hk, 16, d), dtype=torch.float16, device="cuda")
    q_out = buf[:, :, :hq // hk]
    K = torch.zeros((nb, page, hk, d), dtype=torch.float16, device="cuda")
    V = torch.zeros_like(K)
    q = fe().rope_write_decode(g(qkv), g(np.array([[1], [2], [3]], np.int64)), g(tab), g(zero),
                               g(np.array([[0], [17], [33]], np.int64)), K, V, hq, hk,
                               q_out=q_out)
    torch.cuda.synchronize()
    assert q.data_ptr() == buf.data_ptr()
    want = qkv[:, 0, :hq * d].reshape(b, hk, hq // hk, d)   # cos 1, sin 0: no turn
    assert (buf[:, :, :hq // hk].cpu().numpy() == want).all()
    assert (buf[:, :, hq // hk:].cpu().numpy() == 0).all()   # padding rows untouched


def test_cpu_tensors_raise():
    x = torch.zeros(2, 8, dtype=torch.float16)
    with pytest.raises(ValueError):
        fe().rms_norm(x, torch.ones(8, dtype=torch.float16), 1e-6)
    with pytest.raises(ValueError):
        fe().silu_and_mul(x)


@pytest.mark.parametrize("n", [1536, 100])
def test_embed_rms_norm_is_the_lookup_then_the_norm(n):
    rng = np.random.default_rng(n)
    table = g((rng.standard_normal((50, n)) * 2).astype(np.float16))
    w = g(rng.standard_normal(n).astype(np.float16))
    ids = torch.tensor([3, 0, 49, 3, 17], dtype=torch.int64, device="cuda")
    y, rows = fe().embed_rms_norm(table, ids, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(rows, table[ids])
    assert torch.equal(y, fe().rms_norm(table[ids], w, 1e-6))


def test_embed_rms_norm_clamps_ids_into_the_table():
    table = g(np.arange(4 * 8, dtype=np.float16).reshape(4, 8))
    w = g(np.ones(8, np.float16))
    ids = torch.tensor([-5, 9], dtype=torch.int64, device="cuda")
    _, rows = fe().embed_rms_norm(table, ids, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(rows[0], table[0]) and torch.equal(rows[1], table[3])


@pytest.mark.parametrize("rows,n", [(16, 151936), (3, 1000), (5, 37), (1, 8)])
def test_argmax_rows_is_torch_argmax(rows, n):
    gen = torch.Generator(device="cuda").manual_seed(rows * n)
    x = torch.randn(rows, n, device="cuda", generator=gen).half()
    got = fe().argmax_rows(x)
    torch.cuda.synchronize()
    assert torch.equal(got, x.argmax(dim=-1, keepdim=True))


def test_argmax_rows_ties_nan_inf_and_strided_rows():
    n = 4096
    x = torch.zeros(6, n, dtype=torch.float16, device="cuda")
    x[0] = 1.0                                      # all equal: the first index
    x[1, 100] = 7.0; x[1, 3000] = 7.0               # a tie: the first of the two
    x[2] = float("-inf")                            # all -inf: index 0
    x[3, 2500] = float("nan"); x[3, 10] = float("inf")   # NaN above +inf
    x[4, 200] = float("nan"); x[4, 100] = float("nan")   # the first NaN
    x[5, n - 1] = 1.0                               # the last element
    got = fe().argmax_rows(x)
    torch.cuda.synchronize()
    assert got.view(-1).tolist() == [0, 100, 0, 2500, 100, n - 1]
    assert torch.equal(got, x.argmax(dim=-1, keepdim=True))
    big = torch.randn(4, n + 64, device="cuda").half()
    view = big[:, 16:16 + n]                        # rows strided by n + 64
    assert torch.equal(fe().argmax_rows(view), view.argmax(dim=-1, keepdim=True))


def test_argmax_rows_split_rows_repeat_and_replay_in_a_graph():
    """Rows long enough to be split over workgroups: the last to arrive picks
    the best part; repeated calls and graph replays (counters left at zero)
    agree with torch."""
    gen = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(16, 151936, device="cuda", generator=gen).half()
    want = x.argmax(dim=-1, keepdim=True)
    for _ in range(3):
        assert torch.equal(fe().argmax_rows(x), want)
    out = torch.empty(16, 1, dtype=torch.int64, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fe().argmax_rows(x, out=out)
    for i in range(3):
        x[i, 1000 * i + 7] = 100.0                     # move the maximum between replays
        want = x.argmax(dim=-1, keepdim=True)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
