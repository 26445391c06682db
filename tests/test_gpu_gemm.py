"""HIP decode GEMM against an fp32 evaluation of the same product, on an MI355X.

Shapes are the Qwen2.5-1.5B decode projections (qkv 2048 x 1536 with bias,
o 1536 x 1536, gate_up 17920 x 1536, down 1536 x 8960, lm_head 151936 x
1536) at 1, 7, 16 and 64 rows, plus ragged widths that end inside a 16-row
tile and rows that end inside a 16-row column block.  The kernel sums in
fp32 and rounds once: each output is held to one fp16 step of the
correctly rounded fp32 result, plus the fp32 summation-order slack.
"""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def dg():
    from latentserve_amd.kernels import decode_gemm
    return decode_gemm


def check(y, x, w, b=None):
    want = x.float() @ w.float().t()
    if b is not None:
        want = want + b.float()
    err = (y.float() - want).abs()
    # one fp16 rounding (half a step, 2^-11 relative) plus fp32 order slack
    tol = want.abs() * 2.0**-10 + 1e-3
    assert (err <= tol).all(), (err.max().item(), (err / tol).max().item())


@pytest.mark.parametrize("m", [1, 7, 16, 64])
@pytest.mark.parametrize("n,k,bias", [(2048, 1536, True), (1536, 1536, False),
                                      (17920, 1536, False), (1536, 8960, False)])
def test_qwen_projections(m, n, k, bias):
    gen = torch.Generator(device="cuda").manual_seed(m * 7 + n + k)
    x = torch.randn(m, k, device="cuda", generator=gen).half()
    w = (torch.randn(n, k, device="cuda", generator=gen) * k**-0.5).half()
    b = torch.randn(n, device="cuda", generator=gen).half() if bias else None
    y = dg().linear(x, w, b)
    torch.cuda.synchronize()
    check(y, x, w, b)


@pytest.mark.parametrize("m", [1, 16])
def test_lm_head(m):
    gen = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(m, 1536, device="cuda", generator=gen).half()
    w = (torch.randn(151936, 1536, device="cuda", generator=gen) * 0.03).half()
    y = dg().linear(x, w)
    torch.cuda.synchronize()
    check(y, x, w)
    assert torch.equal(y.float().argmax(-1), (x.float() @ w.float().t()).half().float().argmax(-1))


@pytest.mark.parametrize("m,n,k", [(3, 100, 64), (17, 37, 96), (33, 5, 32), (50, 8200, 4096),
                                   (64, 1, 32)])
def test_ragged_shapes(m, n, k):
    gen = torch.Generator(device="cuda").manual_seed(m + n + k)
    x = torch.randn(m, k, device="cuda", generator=gen).half()
    w = (torch.randn(n, k, device="cuda", generator=gen) * k**-0.5).half()
    b = torch.randn(n, device="cuda", generator=gen).half()
    y = dg().linear(x, w, b)
    torch.cuda.synchronize()
    check(y, x, w, b)


def test_strided_input_and_given_output_and_no_overwrite():
    gen = torch.Generator(device="cuda").manual_seed(5)
    big = torch.randn(9, 2048, device="cuda", generator=gen).half()
    x = big[:, 256:256 + 1536]                     # rows strided by 2048
    w = (torch.randn(300, 1536, device="cuda", generator=gen) * 0.03).half()
    out_big = torch.full((9, 320), 7.0, device="cuda", dtype=torch.float16)
    out = out_big[:, :300]
    y = dg().linear(x, w, out=out)
    torch.cuda.synchronize()
    assert y.data_ptr() == out_big.data_ptr()
    check(out_big[:, :300], x, w)
    assert (out_big[:, 300:] == 7).all()          # columns past N untouched


def test_zero_rows_and_rejections():
    w = torch.zeros(16, 64, device="cuda", dtype=torch.float16)
    assert dg().linear(torch.zeros(0, 64, device="cuda", dtype=torch.float16), w).shape == (0, 16)
    with pytest.raises(ValueError):
        dg().linear(torch.zeros(65, 64, device="cuda", dtype=torch.float16), w)
    with pytest.raises(ValueError):
        dg().linear(torch.zeros(2, 64, dtype=torch.float16), w.cpu())
    with pytest.raises(ValueError):                 # K not a multiple of 32
        dg().linear(torch.zeros(2, 48, device="cuda", dtype=torch.float16),
                    torch.zeros(16, 48, device="cuda", dtype=torch.float16))


def fe():
    from latentserve_amd.kernels import fused_elementwise
    return fused_elementwise


@pytest.mark.parametrize("m", [1, 7, 16])
@pytest.mark.parametrize("inter,k,bias", [(8960, 1536, False), (100, 64, True), (36, 96, False),
                                          (1000, 4096, True)])
def test_gate_up_silu_is_the_gemm_then_the_activation_bit_for_bit(m, inter, k, bias):
    gen = torch.Generator(device="cuda").manual_seed(m + inter + k)
    x = torch.randn(m, k, device="cuda", generator=gen).half()
    w = (torch.randn(2 * inter, k, device="cuda", generator=gen) * k**-0.5 * 2).half()
    b = torch.randn(2 * inter, device="cuda", generator=gen).half() if bias else None
    fused = dg().gate_up_silu(x, w, b)
    two = fe().silu_and_mul(dg().linear(x, w, b))
    torch.cuda.synchronize()
    assert fused.shape == (m, inter)
    assert torch.equal(fused, two)
    # and within the activation's fp16 rounding of an fp32 evaluation
    gu = x.float() @ w.float().t() + (b.float() if bias else 0)
    want = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    assert ((fused.float() - want).abs() <= want.abs() * 2.0**-8 + 2e-3).all()


def test_gate_up_silu_too_long_k_takes_two_launches():
    # K long enough at this width that the product splits over workgroups
    gen = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(4, 8960, device="cuda", generator=gen).half()
    w = (torch.randn(2 * 200, 8960, device="cuda", generator=gen) * 0.01).half()
    assert dg().workspace_bytes(4, 400, 8960) > 0
    y = dg().gate_up_silu(x, w)
    torch.cuda.synchronize()
    assert torch.equal(y, fe().silu_and_mul(dg().linear(x, w)))


@pytest.mark.parametrize("m,n,k", [(16, 1536, 8960), (3, 37, 8960), (64, 200, 4096)])
def test_split_products_repeat_exactly(m, n, k):
    """K split over workgroups: partials summed by the last group to arrive,
    in split order, so repeated calls agree bit for bit (and the arrival
    counters were left at zero, or the second call would not sum)."""
    assert dg().workspace_bytes(m, n, k) > 0
    gen = torch.Generator(device="cuda").manual_seed(m * n)
    x = torch.randn(m, k, device="cuda", generator=gen).half()
    w = (torch.randn(n, k, device="cuda", generator=gen) * k**-0.5).half()
    b = torch.randn(n, device="cuda", generator=gen).half()
    ys = [dg().linear(x, w, b) for _ in range(4)]
    torch.cuda.synchronize()
    check(ys[0], x, w, b)
    assert all(torch.equal(ys[0], y) for y in ys[1:])


def test_split_product_in_a_graph_replays_exactly():
    gen = torch.Generator(device="cuda").manual_seed(8)
    x = torch.randn(16, 8960, device="cuda", generator=gen).half()
    w = (torch.randn(1536, 8960, device="cuda", generator=gen) * 0.01).half()
    want = dg().linear(x, w)
    out = torch.empty_like(want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dg().linear(x, w, out=out)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        dg().linear(x, w)                          # eager work between replays


@pytest.mark.parametrize("m", [1, 7, 16])
@pytest.mark.parametrize("bounds", [False, True])
def test_qkv_rope_write_is_the_gemm_then_rope_write_bit_for_bit(m, bounds):
    """The fused q/k/v projection (Qwen2.5-1.5B: 12 / 2 heads of 128, K 1536,
    bias) equals linear followed by rope_write_decode: q, the K/V pools and
    the page bounds, bit for bit; slots -1 and past the pool store nothing."""
    gen = torch.Generator(device="cuda").manual_seed(m * 3 + bounds)
    hq, hk, d, k, nb, page = 12, 2, 128, 1536, 40, 16
    n = (hq + 2 * hk) * d
    x = torch.randn(m, k, device="cuda", generator=gen).half()
    w = (torch.randn(n, k, device="cuda", generator=gen) * k**-0.5).half()
    b = torch.randn(n, device="cuda", generator=gen).half()
    ang = torch.rand(300, d // 2, device="cuda", generator=gen) * 6
    cos = torch.cat([ang, ang], -1).cos().half()
    sin = torch.cat([ang, ang], -1).sin().half()
    pos = torch.randint(0, 400, (m,), device="cuda", generator=gen)        # some past the table
    # distinct pages (a step writes each sequence into its own page)
    pages = torch.randperm(nb, device="cuda", generator=gen)[:m]
    slots = pages * page + torch.randint(0, page, (m,), device="cuda", generator=gen)
    slots[0] = -1
    if m > 2:
        slots[2] = nb * page + 3                                            # past the pool
        slots[1] = (slots[1] // page) * page                                # a page's first token
    pools = [torch.randn(nb, page, hk, d, device="cuda", generator=gen).half() for _ in range(2)]
    kmin = torch.randn(nb, hk, d, device="cuda", generator=gen).half()
    kmax = kmin + 1
    outs = []
    for fused in (True, False):
        K, V = pools[0].clone(), pools[1].clone()
        mn, mx = kmin.clone(), kmax.clone()
        kw = dict(kmin=mn, kmax=mx) if bounds else {}
        if fused:
            q = dg().qkv_rope_write(x, w, b, pos, cos, sin, slots, K, V, hq, hk, **kw)
        else:
            q = fe().rope_write_decode(dg().linear(x, w, b), pos, cos, sin, slots, K, V, hq, hk,
                                       **kw)
        outs.append((q, K, V, mn, mx))
    torch.cuda.synchronize()
    for a, c in zip(*outs):
        assert torch.equal(a, c)


@pytest.mark.parametrize("m", [1, 16, 40])
@pytest.mark.parametrize("n,k", [(2048, 1536), (1536, 8960), (300, 64), (17920, 1536)])
def test_packed_weight_gives_the_same_bits(m, n, k):
    """A packed weight (every load 1 KiB contiguous; at <= 16 rows X through
    LDS) gives the row-major path's outputs bit for bit, split K included."""
    gen = torch.Generator(device="cuda").manual_seed(m + n)
    x = torch.randn(m, k, device="cuda", generator=gen).half()
    w = (torch.randn(n, k, device="cuda", generator=gen) * k**-0.5).half()
    b = torch.randn(n, device="cuda", generator=gen).half()
    pw = dg().PackedWeight(w, "plain")
    y = dg().linear(x, pw, b)
    torch.cuda.synchronize()
    assert torch.equal(y, dg().linear(x, w, b))


@pytest.mark.parametrize("m", [1, 7, 16])
def test_packed_gate_up_and_qkv_give_the_same_bits(m):
    gen = torch.Generator(device="cuda").manual_seed(m)
    x = torch.randn(m, 1536, device="cuda", generator=gen).half()
    wg = (torch.randn(2 * 8960, 1536, device="cuda", generator=gen) * 0.03).half()
    assert torch.equal(dg().gate_up_silu(x, dg().PackedWeight(wg, "gate_up")),
                       dg().gate_up_silu(x, wg))
    hq, hk, d, nb, page = 12, 2, 128, 20, 16
    n = (hq + 2 * hk) * d
    w = (torch.randn(n, 1536, device="cuda", generator=gen) * 0.03).half()
    b = torch.randn(n, device="cuda", generator=gen).half()
    ang = torch.rand(64, d // 2, device="cuda", generator=gen) * 6
    cos, sin = torch.cat([ang, ang], -1).cos().half(), torch.cat([ang, ang], -1).sin().half()
    pos = torch.randint(0, 64, (m,), device="cuda", generator=gen)
    slots = torch.randperm(nb, device="cuda", generator=gen)[:m] * page + 3
    outs = []
    for wk in (dg().PackedWeight(w, "qkv", d), w):
        K = torch.zeros(nb, page, hk, d, device="cuda", dtype=torch.float16)
        V = torch.zeros_like(K)
        q = dg().qkv_rope_write(x, wk, b, pos, cos, sin, slots, K, V, hq, hk)
        outs.append((q, K, V))
    torch.cuda.synchronize()
    for a, c in zip(*outs):
        assert torch.equal(a, c)


def test_packed_weight_kind_is_checked():
    w = torch.zeros(64, 64, device="cuda", dtype=torch.float16)
    pw = dg().PackedWeight(w, "gate_up")
    with pytest.raises(ValueError):
        dg().linear(torch.zeros(2, 64, device="cuda", dtype=torch.float16), pw)


def _normed_operand_bound(h_ref, w):
    """Per-output bound for a product whose operand rows may differ from
    h_ref by one fp16 step per element (the prologue sums the squares in
    another order than the norm kernel, which can move the scale's last
    bit): sum_k |h_k| |w_nk| 2^-10, plus two fp16 roundings of y."""
    return (h_ref.float().abs() @ w.float().abs().t()) * 2.0**-10


@pytest.mark.parametrize("m", [1, 7, 16])
@pytest.mark.parametrize("n,k", [(1536, 1536), (300, 64), (2048, 1120), (151936, 1536)])
def test_norm_prologue_matches_the_norm_then_the_gemm(m, n, k):
    """linear(x, residual=, norm_weight=) equals fused_add_rms_norm followed by
    the GEMM: x + residual bit for bit, y within what one fp16 step of the
    normalised operand moves it (and bit-equal in most places)."""
    gen = torch.Generator(device="cuda").manual_seed(m * 5 + n + k)
    x = torch.randn(m, k, device="cuda", generator=gen).half()
    res = (torch.randn(m, k, device="cuda", generator=gen) * 4).half()
    nw = (torch.rand(k, device="cuda", generator=gen) + 0.5).half()
    w = (torch.randn(n, k, device="cuda", generator=gen) * k**-0.5).half()
    b = torch.randn(n, device="cuda", generator=gen).half()
    pw = dg().PackedWeight(w, "plain")
    if dg().workspace_bytes(m, n, k):
        pytest.skip("splits K")
    y, ro = dg().linear(x, pw, b, residual=res, norm_weight=nw, eps=1e-6)
    h_ref, r_ref = fe().fused_add_rms_norm(x, res, nw, 1e-6)
    y_ref = dg().linear(h_ref, pw, b)
    torch.cuda.synchronize()
    assert torch.equal(ro, r_ref)
    err = (y.float() - y_ref.float()).abs()
    tol = _normed_operand_bound(h_ref, w) + y_ref.float().abs() * 2.0**-10 + 1e-3
    assert (err <= tol).all(), (err / tol).max().item()
    assert (y == y_ref).float().mean().item() > 0.5
    # against fp32 end to end: a dropped weight or residual would fail here
    s = res.float() + x.float()
    want = (s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + 1e-6)) * nw.float() @ w.float().t()
    want = want + b.float()
    assert ((y.float() - want).abs() <= want.abs() * 2.0**-8 + 2e-2).all()


@pytest.mark.parametrize("m", [1, 16])
def test_norm_prologue_gate_up_and_qkv(m):
    gen = torch.Generator(device="cuda").manual_seed(100 + m)
    k = 1536
    x = torch.randn(m, k, device="cuda", generator=gen).half()
    res = (torch.randn(m, k, device="cuda", generator=gen) * 4).half()
    nw = (torch.rand(k, device="cuda", generator=gen) + 0.5).half()
    h_ref, r_ref = fe().fused_add_rms_norm(x, res, nw, 1e-6)
    wg = (torch.randn(2 * 8960, k, device="cuda", generator=gen) * 0.03).half()
    pg = dg().PackedWeight(wg, "gate_up")
    g, ro = dg().gate_up_silu(x, pg, residual=res, norm_weight=nw, eps=1e-6)
    g_ref = dg().gate_up_silu(h_ref, pg)
    torch.cuda.synchronize()
    assert torch.equal(ro, r_ref)
    assert (g == g_ref).float().mean().item() > 0.5
    # silu(a) * b moves by at most ~1.1 (|b| da + |silu(a)| db) for the bound of each
    gu = h_ref.float() @ wg.float().t()
    bnd = _normed_operand_bound(h_ref, wg)
    a, bb = gu[:, :8960], gu[:, 8960:]
    tol = 1.2 * (bb.abs() * bnd[:, :8960] + torch.nn.functional.silu(a).abs() * bnd[:, 8960:])
    tol = tol + g_ref.float().abs() * 2.0**-9 + 2e-3
    assert ((g.float() - g_ref.float()).abs() <= tol).all()

    hq, hk, d, nb, page = 12, 2, 128, 20, 16
    n = (hq + 2 * hk) * d
    w = (torch.randn(n, k, device="cuda", generator=gen) * 0.03).half()
    b = torch.randn(n, device="cuda", generator=gen).half()
    ang = torch.rand(64, d // 2, device="cuda", generator=gen) * 6
    cos, sin = torch.cat([ang, ang], -1).cos().half(), torch.cat([ang, ang], -1).sin().half()
    pos = torch.randint(0, 64, (m,), device="cuda", generator=gen)
    slots = torch.randperm(nb, device="cuda", generator=gen)[:m] * page + 3
    pq = dg().PackedWeight(w, "qkv", d)
    outs = []
    for fused in (True, False):
        K = torch.zeros(nb, page, hk, d, device="cuda", dtype=torch.float16)
        V = torch.zeros_like(K)
        if fused:
            q, ro = dg().qkv_rope_write(x, pq, b, pos, cos, sin, slots, K, V, hq, hk,
                                        residual=res, norm_weight=nw, eps=1e-6)
            assert torch.equal(ro, r_ref)
        else:
            q = dg().qkv_rope_write(h_ref, pq, b, pos, cos, sin, slots, K, V, hq, hk)
        outs.append((q, K, V))
    torch.cuda.synchronize()
    # RoPE mixes two channels with |cos|, |sin| <= 1: twice the product bound
    qkv_bnd = _normed_operand_bound(h_ref, w)
    for a_, c_ in zip(*outs):
        err = (a_.float() - c_.float()).abs()
        assert err.max().item() <= 2 * qkv_bnd.max().item() + 2.0**-8 * c_.float().abs().max()


def test_norm_prologue_rejections():
    k = 64
    x = torch.randn(4, k, device="cuda").half()
    res = torch.randn(4, k, device="cuda").half()
    nw = torch.ones(k, device="cuda", dtype=torch.float16)
    w = torch.randn(32, k, device="cuda").half()
    pw = dg().PackedWeight(w, "plain")
    with pytest.raises(ValueError):                # res_out aliasing the residual
        dg().linear(x, pw, residual=res, norm_weight=nw, res_out=res)
    with pytest.raises(ValueError):                # res_out aliasing x
        dg().linear(x, pw, residual=res, norm_weight=nw, res_out=x)
    with pytest.raises(ValueError):                # row-major weight
        dg().linear(x, w, residual=res, norm_weight=nw)
    with pytest.raises(ValueError):                # more than 16 rows
        x17 = torch.randn(17, k, device="cuda").half()
        dg().linear(x17, pw, residual=x17.clone(), norm_weight=nw)
