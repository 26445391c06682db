"""The elementwise oracle against Hugging Face's own Qwen2 modules (CPU).

The reference's kernels reproduce transformers' Qwen2 computation in fp16
(kernels/fused_elementwise.py:75-110, pinned there by
tests/test_phase14_elementwise.py:44-70 against the same modules).  Here the
numpy oracle is pinned against those modules directly, and against closed
forms that a wrong index, sign or half would break.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")
m = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")


def ulps(a, b):
    """Distance in fp16 steps (of the larger magnitude's binade)."""
    a = np.asarray(a, np.float16).astype(np.float64)
    b = np.asarray(b, np.float16).astype(np.float64)
    step = np.maximum(np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16)).astype(
        np.float64), 2.0**-24)
    return np.abs(a - b) / step


@pytest.mark.parametrize("n", [1536, 128, 100])
@pytest.mark.parametrize("unit_weight", [True, False])
def test_rms_norm_is_qwen2_rmsnorm(n, unit_weight):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((9, n)) * 3).astype(np.float16)
    w = np.ones(n, np.float16) if unit_weight else rng.standard_normal(n).astype(np.float16)
    norm = m.Qwen2RMSNorm(n, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(w))
    norm = norm.half()
    with torch.no_grad():
        want = norm(torch.from_numpy(x)).numpy()
    got, s = oracle.rms_norm(x, w, 1e-6)
    assert (s == x).all()
    # the variance is summed in another order (fp32 there, fp64 here): the
    # normalised value may land one fp16 step apart, which a weight of up to
    # 2 in magnitude carries to two steps of the product
    d = ulps(got, want)
    assert d.max() <= (1 if unit_weight else 2) and (d == 0).mean() > 0.97, (d.max(), (d == 0).mean())


def test_fused_add_rms_norm_is_the_add_then_the_norm():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 1536)).astype(np.float16)
    r = rng.standard_normal((5, 1536)).astype(np.float16)
    w = rng.standard_normal(1536).astype(np.float16)
    y, s = oracle.rms_norm(x, w, 1e-6, residual=r)
    s_t = (torch.from_numpy(r) + torch.from_numpy(x)).numpy()      # one fp16 add
    assert (s == s_t).all()
    y2, _ = oracle.rms_norm(s_t, w, 1e-6)
    assert (y == y2).all()


def test_rms_norm_of_a_constant_row_is_the_weight():
    w = np.linspace(-2, 2, 64).astype(np.float16)
    for c in (0.5, -3.0, 100.0):
        y, _ = oracle.rms_norm(np.full((1, 64), c, np.float16), w, 0.0)
        assert (y[0] == (w * np.float16(np.sign(c)))).all()


def test_silu_and_mul_is_the_mlp_activation():
    rng = np.random.default_rng(2)
    gu = (rng.standard_normal((3, 2 * 896)) * 4).astype(np.float16)
    g, u = torch.from_numpy(gu).chunk(2, dim=-1)
    want = (torch.nn.functional.silu(g) * u).numpy()
    got = oracle.silu_and_mul(gu)
    d = ulps(got, want)
    assert d.max() <= 1 and (d == 0).mean() > 0.99


def test_silu_closed_forms():
    gu = np.array([[0.0, 40.0, -40.0, 1.0, 1.0, 1.0]], np.float16)
    got = oracle.silu_and_mul(gu)
    assert got[0, 0] == 0.0 and got[0, 1] == 40.0 and got[0, 2] == 0.0


def test_rope_is_apply_rotary_pos_emb_bit_for_bit():
    rng = np.random.default_rng(3)
    b, h, s, d = 2, 5, 3, 128
    q = (rng.standard_normal((b, h, s, d)) * 2).astype(np.float16)
    k = (rng.standard_normal((b, 2, s, d)) * 2).astype(np.float16)
    ang = rng.uniform(0, 2 * np.pi, (b, s, d // 2))
    ang = np.concatenate([ang, ang], -1)
    cos, sin = np.cos(ang).astype(np.float16), np.sin(ang).astype(np.float16)
    wq, wk = m.apply_rotary_pos_emb(torch.from_numpy(q), torch.from_numpy(k),
                                    torch.from_numpy(cos), torch.from_numpy(sin))
    got_q = oracle.rope(q, cos[:, None], sin[:, None])
    got_k = oracle.rope(k, cos[:, None], sin[:, None])
    assert (got_q == wq.numpy()).all() and (got_k == wk.numpy()).all()


def test_rope_closed_forms():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 128)).astype(np.float16)
    one, zero = np.ones((1, 128), np.float16), np.zeros((1, 128), np.float16)
    assert (oracle.rope(x, one, zero) == x).all()                        # no turn
    quarter = np.concatenate([-x[:, 64:], x[:, :64]], -1)
    assert (oracle.rope(x, zero, one) == quarter).all()                  # a quarter turn


def test_rope_write_decode_folds_stores_and_bounds():
    rng = np.random.default_rng(5)
    b, hq, hk, d, nb, page = 3, 6, 2, 128, 7, 16
    qkv = rng.standard_normal((b, (hq + 2 * hk) * d)).astype(np.float16)
    ang = rng.uniform(0, 6, (40, d // 2))
    cos = np.cos(np.concatenate([ang, ang], -1)).astype(np.float16)
    sin = np.sin(np.concatenate([ang, ang], -1)).astype(np.float16)
    pos = np.array([5, 39, 70], np.int64)                   # the last one past the table
    slots = np.array([2 * page + 0, 6 * page + 9, -1], np.int64)
    kp = rng.standard_normal((nb, page, hk, d)).astype(np.float16)
    vp = rng.standard_normal((nb, page, hk, d)).astype(np.float16)
    kmin = rng.standard_normal((nb, hk, d)).astype(np.float16)
    kmax = kmin + np.float16(1)
    kp0, vp0, kmin0, kmax0 = kp.copy(), vp.copy(), kmin.copy(), kmax.copy()
    q = oracle.rope_write_decode(qkv, pos, cos, sin, slots, kp, vp, hq, hk, kmin, kmax, page)
    for i in range(b):
        p = min(pos[i], 39)
        qi = oracle.rope(qkv[i, :hq * d].reshape(hq, d), cos[p], sin[p])
        for h in range(hq):
            assert (q[i, h // (hq // hk), h % (hq // hk)] == qi[h]).all()
        ki = oracle.rope(qkv[i, hq * d:(hq + hk) * d].reshape(hk, d), cos[p], sin[p])
        vi = qkv[i, (hq + hk) * d:].reshape(hk, d)
        if slots[i] >= 0:
            blk, off = divmod(int(slots[i]), page)
            assert (kp[blk, off] == ki).all() and (vp[blk, off] == vi).all()
    touched = np.zeros((nb, page), bool)
    touched[2, 0] = touched[6, 9] = True
    assert (kp[~touched] == kp0[~touched]).all() and (vp[~touched] == vp0[~touched]).all()
    # page 2 was started by this token (bounds reset), page 6 extended
    k0 = oracle.rope(qkv[0, hq * d:(hq + hk) * d].reshape(hk, d), cos[5], sin[5])
    assert (kmin[2] == k0).all() and (kmax[2] == k0).all()
    k1 = kp[6, 9]
    assert (kmin[6] == np.minimum(kmin0[6], k1)).all() and (kmax[6] == np.maximum(kmax0[6], k1)).all()
    others = [0, 1, 3, 4, 5]
    assert (kmin[others] == kmin0[others]).all() and (kmax[others] == kmax0[others]).all()
