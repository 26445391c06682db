"""HIP INT8 write side against the CPU oracle, on an MI355X: bit-exact.

The decode-step write (V quantized per token and scattered, K copied into
the fp16 residual) and the completed-page K quantizer are compared byte for
byte with oracle.quantize_v / quantize_k, which tests/test_oracle.py pins to
numpy and torch CPU arithmetic, in both division forms (GPU torch's
reciprocal multiply, the default, and CPU torch's true division).  Shapes
follow the reference cache (cache/int8_paged_cache.py:256-323): flat V
[slots, H, D] over the pool, flat residual [rows * 16, H, D].
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

Q8 = dict(eps=1e-8, qmax=127.0, levels=255.0, offset=128.0)


def iw():
    from latentserve_amd.kernels.hip import int8_write
    return int8_write


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def fp16(shape, seed, scale=1.0, shift=0.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * scale + shift).astype(np.float16)


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("exact", [False, True])
def test_decode_write_is_bit_exact(asym, exact):
    b, h, d, nb, rows = 7, 2, 128, 40, 9
    k = fp16((b, h, 1, d), 1)
    v = fp16((b, h, 1, d), 2, scale=2.0)
    v[3] *= np.float16(0.001)          # a small-magnitude row
    v[4] = np.float16(0)               # an all-zero row: the eps floor
    rng = np.random.default_rng(3)
    slots = rng.choice(nb * 16, size=b, replace=False).astype(np.int64)
    res_idx = rng.choice(rows * 16, size=b, replace=False).astype(np.int64)
    flat_v = torch.zeros(nb * 16, h, d, dtype=torch.int8, device="cuda")
    flat_s = torch.zeros(nb * 16, h, dtype=torch.float32, device="cuda")
    flat_z = torch.zeros_like(flat_s) if asym else None
    k_res = torch.zeros(rows * 16, h, d, dtype=torch.float16, device="cuda")
    iw().decode_write(dev(k), dev(v), dev(slots), dev(res_idx), flat_v, flat_s, flat_z, k_res,
                      asym=asym, exact_division=exact, **Q8)
    torch.cuda.synchronize()
    codes, step, zero = oracle.quantize_v(v[:, :, 0], asym=asym, recip=not exact)
    fv, fs = flat_v.cpu().numpy(), flat_s.cpu().numpy()
    np.testing.assert_array_equal(fv[slots], codes)
    np.testing.assert_array_equal(fs[slots].view(np.uint32), step.view(np.uint32))
    if asym:
        np.testing.assert_array_equal(flat_z.cpu().numpy()[slots].view(np.uint32),
                                      zero.view(np.uint32))
    untouched = np.setdiff1d(np.arange(nb * 16), slots)
    assert (fv[untouched] == 0).all() and (fs[untouched] == 0).all()
    kr = k_res.cpu().numpy()
    np.testing.assert_array_equal(kr[res_idx].view(np.uint16), k[:, :, 0].view(np.uint16))
    assert (kr[np.setdiff1d(np.arange(rows * 16), res_idx)] == 0).all()


def test_decode_write_skips_rows_outside_the_buffers():
    b, h, d = 3, 2, 128
    k, v = fp16((b, h, 1, d), 4), fp16((b, h, 1, d), 5)
    slots = np.array([5, -1, 10 ** 6], dtype=np.int64)
    res_idx = np.array([-2, 3, 10 ** 6], dtype=np.int64)
    flat_v = torch.zeros(16, h, d, dtype=torch.int8, device="cuda")
    flat_s = torch.zeros(16, h, dtype=torch.float32, device="cuda")
    k_res = torch.zeros(16, h, d, dtype=torch.float16, device="cuda")
    iw().decode_write(dev(k), dev(v), dev(slots), dev(res_idx), flat_v, flat_s, None, k_res,
                      asym=False, **Q8)
    torch.cuda.synchronize()
    assert (flat_s.cpu().numpy()[np.arange(16) != 5] == 0).all() and flat_s[5, 0].item() > 0
    kr = k_res.cpu().numpy()
    assert (kr[np.arange(16) != 3] == 0).all()
    np.testing.assert_array_equal(kr[3].view(np.uint16), k[1, :, 0].view(np.uint16))


def test_decode_write_reads_strided_inputs():
    """k, v as views of a wider [B, H, n, D] buffer (the caller's last token)."""
    b, h, d = 4, 2, 128
    kw, vw = fp16((b, h, 3, d), 6), fp16((b, h, 3, d), 7)
    K, V = dev(kw)[:, :, 2:3], dev(vw)[:, :, 2:3]
    slots = np.arange(b, dtype=np.int64) * 3
    flat_v = torch.zeros(16, h, d, dtype=torch.int8, device="cuda")
    flat_s = torch.zeros(16, h, dtype=torch.float32, device="cuda")
    k_res = torch.zeros(16, h, d, dtype=torch.float16, device="cuda")
    iw().decode_write(K, V, dev(slots), dev(slots), flat_v, flat_s, None, k_res, asym=False, **Q8)
    torch.cuda.synchronize()
    codes, step, _ = oracle.quantize_v(vw[:, :, 2], recip=True)
    np.testing.assert_array_equal(flat_v.cpu().numpy()[slots], codes)
    np.testing.assert_array_equal(k_res.cpu().numpy()[slots].view(np.uint16),
                                  kw[:, :, 2].view(np.uint16))


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("exact", [False, True])
def test_finalize_blocks_is_bit_exact(asym, exact):
    n, h, d, nb = 11, 2, 128, 30
    data = fp16((n, 16, h, d), 8, scale=1.5, shift=0.3 if asym else 0.0)
    data[2] = np.float16(0)                       # all-zero block: eps floor
    data[5, :, 1] = np.float16(0.25)              # constant channels
    rng = np.random.default_rng(9)
    ids = rng.choice(nb, size=n, replace=False).astype(np.int64)
    k_pool = torch.zeros(nb, 16, h, d, dtype=torch.int8, device="cuda")
    k_scale = torch.zeros(nb, h, d, dtype=torch.float32, device="cuda")
    k_zero = torch.zeros_like(k_scale) if asym else None
    iw().finalize_blocks(dev(data), dev(ids), k_pool, k_scale, k_zero, asym=asym,
                         exact_division=exact, **Q8)
    torch.cuda.synchronize()
    codes, step, zero = oracle.quantize_k(data, asym=asym, recip=not exact)
    np.testing.assert_array_equal(k_pool.cpu().numpy()[ids], codes)
    np.testing.assert_array_equal(k_scale.cpu().numpy()[ids].view(np.uint32), step.view(np.uint32))
    if asym:
        np.testing.assert_array_equal(k_zero.cpu().numpy()[ids].view(np.uint32),
                                      zero.view(np.uint32))
    rest = np.setdiff1d(np.arange(nb), ids)
    assert (k_pool.cpu().numpy()[rest] == 0).all()


def test_finalize_from_the_residual_then_decode_matches_dequantized_attention():
    """The cache's page-completion path: a sequence's fp16 residual page is
    quantized into its block; the INT8 decode over the pool then agrees with
    fp16 attention over the dequantized pages (tolerance of the decode)."""
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh
    from tests.cases import assert_close, dense_attention

    h, d, pages = 2, 128, 6
    kf = fp16((pages, 16, h, d), 10)
    vf = fp16((pages, 16, h, d), 11)
    ids = np.arange(pages, dtype=np.int64)[::-1].copy()
    k_pool = torch.zeros(pages, 16, h, d, dtype=torch.int8, device="cuda")
    k_scale = torch.zeros(pages, h, d, dtype=torch.float32, device="cuda")
    iw().finalize_blocks(dev(kf), dev(ids), k_pool, k_scale, asym=False, **Q8)
    vcodes, vstep, _ = oracle.quantize_v(vf.reshape(-1, h, d), recip=True)
    v_pool = dev(vcodes.reshape(pages, 16, h, d))
    v_scale = dev(vstep.reshape(pages, 16, h))
    q = fp16((1, h, 6, d), 12)
    table = dev(ids.astype(np.int32)[None])
    lens = dev(np.array([pages * 16], np.int32))
    out = pdh.paged_decode_hip(dev(q), k_pool, v_pool, table, lens, pages * 16, k_scale=k_scale,
                               v_scale=v_scale).float().cpu().numpy()
    kd = k_pool.cpu().numpy().astype(np.float32) * k_scale.cpu().numpy()[:, None]
    vd = vcodes.reshape(pages, 16, h, d).astype(np.float32) * vstep.reshape(pages, 16, h)[..., None]
    want = dense_attention(q, kd, vd, ids.astype(np.int32)[None], np.array([pages * 16]))
    assert_close(out, want, 2e-3, 1e-2, "finalize -> decode")


def test_decode_write_graph_replays():
    b, h, d = 5, 2, 128
    k, v = dev(fp16((b, h, 1, d), 13)), dev(fp16((b, h, 1, d), 14))
    slots, res = dev(np.arange(b, dtype=np.int64) * 2), dev(np.arange(b, dtype=np.int64))
    flat_v = torch.zeros(32, h, d, dtype=torch.int8, device="cuda")
    flat_s = torch.zeros(32, h, dtype=torch.float32, device="cuda")
    k_res = torch.zeros(16, h, d, dtype=torch.float16, device="cuda")
    args = (k, v, slots, res, flat_v, flat_s, None, k_res)
    iw().decode_write(*args, asym=False, **Q8)
    want_v, want_s = flat_v.clone(), flat_s.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        iw().decode_write(*args, asym=False, **Q8)
    for i in range(4):
        flat_v.zero_()
        flat_s.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(flat_v, want_v) and torch.equal(flat_s, want_s), i
