"""Oracle parity at every BASELINE configuration's full size, on an MI355X.

The smaller GPU tests cover edge cases; these run the HIP path at the
shapes the benchmark reports, so precision choices whose error grows with
the context (fp16 softmax weights before the PV product, INT8 weights
p * v_scale rounded to fp16) are checked where they matter.  Inputs are
N(0,1) fp16 from a seeded numpy generator, block tables a seeded
permutation of the pool; the C oracle runs on the host's cores (OpenMP).

* C1 B1 x 2048 lives in tests/test_gpu_decode.py (test_config1_b1_2048_pool256).
* C2 fp16 B16 x 16384, default and 16 splits.
* C3 fp16 B8 x 32768, and ragged B16 with L ~ U[512, 32768] drawn with the
  benchmark's own seed (bench.py lengths_for).
* C4 INT8 B16 x 16384: N(0,1) fp16 quantised on the GPU by
  ls_int8_finalize_blocks (K) and ls_int8_decode_write (V), codes and scales
  bit-exact against the oracle's quantizers, the last page of K in the fp16
  residual, output against the oracle over the INT8 cache; and the same
  quantizers byte-equal to the reference cache's own torch ops run on the
  GPU, symmetric and asymmetric.
* C5 sparse 50 % B8 x 32768, and C5h the same at the headline B16 x 16384:
  page bounds bit-exact, page scores against the oracle, the GPU selection
  as sets against the oracle's stable top-k (swaps allowed only inside
  score near-ties), outputs of the list decode and of the selecting decode
  against the oracle's sparse_decode.

The reference's GPU tests take the same shape of check at smaller sizes
(tests/test_cuda_decode.py:82-91, tests/test_phase14_sparse_kernels.py:92-134).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from tests.cases import assert_close

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

ATOL, RTOL = 2e-3, 1e-2            # max-abs 2e-3, rel 1e-2
H_KV, N_REP, D, PAGE = 2, 6, 128, 16


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    oracle.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    yield


def normal16(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


def config_case(lengths, seed, width=None):
    """q [B,2,6,128], pools [nb,16,2,128] N(0,1) fp16, permuted int32 tables."""
    rng = np.random.default_rng(seed)
    b = len(lengths)
    width = width or max(1, max(-(-int(x) // PAGE) for x in lengths))
    nb = b * width + 4
    k = normal16(rng, (nb, PAGE, H_KV, D))
    v = normal16(rng, (nb, PAGE, H_KV, D))
    t = rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32)
    q = normal16(rng, (b, H_KV, N_REP, D))
    return q, k, v, t, np.asarray(lengths, np.int32)


def dev(*arrays):
    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()
            for a in arrays]


def hip_decode(Q, K, V, T, L, max_len, splits=None, **extra):
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh
    out = pdh.paged_decode_hip(Q, K, V, T, L, max_len, num_splits=splits, **extra)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_c2_fp16_b16x16k():
    print("c2: fp16 B16 x 16384", flush=True)
    case = config_case([16384] * 16, seed=2)
    want = oracle.paged_decode(*case)
    Q, K, V, T, L = dev(*case)
    for splits in (None, 16):
        assert_close(hip_decode(Q, K, V, T, L, 16384, splits), want, ATOL, RTOL,
                     f"c2 splits={splits}")


def test_c3_fp16_b8x32k():
    print("c3: fp16 B8 x 32768", flush=True)
    case = config_case([32768] * 8, seed=3)
    want = oracle.paged_decode(*case)
    Q, K, V, T, L = dev(*case)
    assert_close(hip_decode(Q, K, V, T, L, 32768), want, ATOL, RTOL, "c3")


def test_c3_ragged_b16_bench_lengths():
    """The benchmark's ragged draw (bench.py lengths_for: seed 1234,
    integers in [512, 32768]), table width 2048 pages."""
    lens = np.random.default_rng(1234).integers(512, 32768 + 1, size=16).astype(np.int32)
    print(f"c3r: fp16 B16 ragged {lens.tolist()}", flush=True)
    case = config_case(lens.tolist(), seed=33, width=2048)
    want = oracle.paged_decode(*case)
    Q, K, V, T, L = dev(*case)
    for splits in (None, 7):
        assert_close(hip_decode(Q, K, V, T, L, 32768, splits), want, ATOL, RTOL,
                     f"c3r splits={splits}")


def test_c4_int8_b16x16k_quantised_on_the_gpu():
    """N(0,1) fp16 K/V -> HIP quantizers -> INT8 decode with the fp16
    residual for each sequence's last page of K."""
    from latentserve_amd.kernels.hip import int8_write as iw

    print("c4: INT8 B16 x 16384", flush=True)
    q, k16, v16, t, l = config_case([16384] * 16, seed=4)
    nb = k16.shape[0]
    K16, V16 = dev(k16, v16)
    kq = torch.empty(k16.shape, dtype=torch.int8, device="cuda")
    vq = torch.empty_like(kq)
    ks = torch.empty(nb, H_KV, D, dtype=torch.float32, device="cuda")
    vs = torch.empty(nb, PAGE, H_KV, dtype=torch.float32, device="cuda")
    qargs = dict(asym=False, eps=1e-8, qmax=127.0, levels=255.0, offset=128.0)
    iw.finalize_blocks(K16, torch.arange(nb, device="cuda"), kq, ks, **qargs)
    # V one token row at a time, every slot of the pool (the decode write's
    # per-token quantizer); no residual rows written here (index -1)
    ntok = nb * PAGE
    k_rows = K16.view(ntok, H_KV, 1, D)
    v_rows = V16.view(ntok, H_KV, 1, D)
    k_res_dummy = torch.empty(1, H_KV, D, dtype=torch.float16, device="cuda")
    iw.decode_write(k_rows, v_rows, torch.arange(ntok, device="cuda"),
                    torch.full((ntok,), -1, dtype=torch.long, device="cuda"),
                    vq.view(ntok, H_KV, D), vs.view(ntok, H_KV), None, k_res_dummy, **qargs)
    torch.cuda.synchronize()

    want_kq, want_ks, _ = oracle.quantize_k(k16, recip=True)
    want_vq, want_vs, _ = oracle.quantize_v(v16, recip=True)
    got_kq, got_ks = kq.cpu().numpy(), ks.cpu().numpy()
    got_vq, got_vs = vq.cpu().numpy(), vs.cpu().numpy()
    assert np.array_equal(got_kq, want_kq), int((got_kq != want_kq).sum())
    assert np.array_equal(got_ks.view(np.uint32), want_ks.view(np.uint32))
    assert np.array_equal(got_vq, want_vq), int((got_vq != want_vq).sum())
    assert np.array_equal(got_vs.view(np.uint32), want_vs.view(np.uint32))

    last = (l.astype(np.int64) + PAGE - 1) // PAGE - 1
    res = np.ascontiguousarray(k16[t[np.arange(16), last]])          # [16, 16, 2, 128]
    rows = np.arange(16, dtype=np.int32)[::-1].copy()                 # not the identity
    res = np.ascontiguousarray(res[rows.argsort()])
    want = oracle.paged_decode(q, want_kq, want_vq, t, l, k_scale=want_ks, v_scale=want_vs,
                               k_residual=res, res_rows=rows)
    Q, T, L, R, RR = dev(q, t, l, res, rows)
    for splits in (None, 16):
        got = hip_decode(Q, kq, vq, T, L, 16384, splits, k_scale=ks, v_scale=vs,
                         k_residual=R, res_rows=RR)
        assert_close(got, want, ATOL, RTOL, f"c4 splits={splits}")


@pytest.mark.parametrize("asym", [False, True])
def test_c4_quantizers_equal_the_references_torch_ops_on_the_gpu(asym):
    """At C4's full size, the HIP quantizers against the reference cache's
    own torch op sequence run on the same GPU tensors (the computation its
    cache executes on a GPU): Int8PagedKVCache._finalize_blocks for K per
    (block, head, channel) and the decode write's V per (token, head),
    cache/int8_paged_cache.py:683-699 and :741-758.  Codes, steps and zero
    points byte-equal."""
    from latentserve_amd.kernels.hip import int8_write as iw

    print(f"c4: quantizers against torch on the GPU, asym={asym}", flush=True)
    _, k16, v16, _, _ = config_case([16384] * 16, seed=44)
    nb = k16.shape[0]
    K16, V16 = dev(k16, v16)
    eps, qmax, levels, offset = 1e-8, 127, 255, 128        # the reference's constants
    # ---- the reference's ops, on the GPU ----
    f = K16.to(torch.float32)
    if asym:
        lo, hi = f.amin(dim=1), f.amax(dim=1)
        step = ((hi - lo) / levels).clamp_min(eps)
        q_u = torch.clamp(torch.round((f - lo.unsqueeze(1)) / step.unsqueeze(1)), 0, levels)
        want_kq = (q_u - offset).to(torch.int8)
        want_kz = lo + offset * step
    else:
        step = f.abs().amax(dim=1).clamp_min(eps) / qmax
        want_kq = torch.clamp(torch.round(f / step.unsqueeze(1)), -qmax, qmax).to(torch.int8)
    want_ks = step
    del f
    vf = V16.to(torch.float32)
    if asym:
        v_lo = vf.amin(dim=-1, keepdim=True)
        v_hi = vf.amax(dim=-1, keepdim=True)
        v_step = ((v_hi - v_lo) / levels).clamp_min(eps)
        v_u = torch.clamp(torch.round((vf - v_lo) / v_step), 0, levels)
        want_vq = (v_u - offset).to(torch.int8)
        want_vz = (v_lo + offset * v_step).squeeze(-1)
        del v_u
    else:
        v_step = vf.abs().amax(dim=-1, keepdim=True).clamp_min(eps) / qmax
        want_vq = torch.clamp(torch.round(vf / v_step), -qmax, qmax).to(torch.int8)
    want_vs = v_step.squeeze(-1)
    del vf
    # ---- the HIP quantizers ----
    qargs = dict(asym=asym, eps=float(eps), qmax=float(qmax), levels=float(levels),
                 offset=float(offset))
    kq = torch.empty(k16.shape, dtype=torch.int8, device="cuda")
    ks = torch.empty(nb, H_KV, D, dtype=torch.float32, device="cuda")
    kz = torch.empty_like(ks) if asym else None
    iw.finalize_blocks(K16, torch.arange(nb, device="cuda"), kq, ks, k_zero=kz, **qargs)
    ntok = nb * PAGE
    vq = torch.empty(ntok, H_KV, D, dtype=torch.int8, device="cuda")
    vs = torch.empty(ntok, H_KV, dtype=torch.float32, device="cuda")
    vz = torch.empty_like(vs) if asym else None
    k_res_dummy = torch.empty(1, H_KV, D, dtype=torch.float16, device="cuda")
    iw.decode_write(K16.view(ntok, H_KV, 1, D), V16.view(ntok, H_KV, 1, D),
                    torch.arange(ntok, device="cuda"),
                    torch.full((ntok,), -1, dtype=torch.long, device="cuda"),
                    vq, vs, vz, k_res_dummy, **qargs)
    torch.cuda.synchronize()

    def same_bits(a, b, what):
        a, b = a.contiguous().view(-1), b.contiguous().view(-1)
        if a.dtype == torch.float32:
            a, b = a.view(torch.int32), b.view(torch.int32)
        bad = int((a != b).sum().item())
        assert bad == 0, f"{what}: {bad} of {a.numel()} differ"

    same_bits(kq, want_kq, "K codes")
    same_bits(ks, want_ks, "K steps")
    same_bits(vq.view(want_vq.shape), want_vq, "V codes")
    same_bits(vs.view(want_vs.shape), want_vs, "V steps")
    if asym:
        same_bits(kz, want_kz, "K zero points")
        same_bits(vz.view(want_vz.shape), want_vz, "V zero points")


def _sets_agree(got_sel, want_sel, scores, what):
    """Per (b, h), the selected sets may differ only by pages whose scores
    lie within a near-tie of the k-th score."""
    b, h, k = want_sel.shape
    for i in range(b):
        for j in range(h):
            g, w = set(got_sel[i, j].tolist()), set(want_sel[i, j].tolist())
            if g == w:
                continue
            row = scores[i, j]
            kth = np.sort(row)[::-1][k - 1]
            for p in g ^ w:
                gap = abs(float(row[p]) - float(kth))
                assert gap <= 1e-4 * max(1.0, abs(float(kth))), \
                    f"{what}: b={i} h={j} page {p} (score {row[p]}, k-th {kth})"


def _sparse_half_at_full_size(batch, ctx, seed, name):
    """Bounds, scores, selection and both sparse decodes at one full-size
    shape, keeping 50 % of every sequence's pages."""
    from latentserve_amd.kernels.hip import paged_sparse as ps

    print(f"{name}: sparse 50% B{batch} x {ctx}", flush=True)
    q, k, v, t, l = config_case([ctx] * batch, seed=seed)
    Q, K, V, T, L = dev(q, k, v, t, l)
    nb = k.shape[0]
    kmin = torch.empty(nb, H_KV, D, dtype=torch.float16, device="cuda")
    kmax = torch.empty_like(kmin)
    ps.rebuild_bounds(K, kmin, kmax)
    want_min, want_max = k.min(axis=1), k.max(axis=1)
    assert np.array_equal(kmin.cpu().numpy(), want_min)
    assert np.array_equal(kmax.cpu().numpy(), want_max)

    width = t.shape[1]
    kk = oracle.budget(0.5, width)
    assert kk == ctx // PAGE // 2
    want_scores = oracle.page_scores(q, want_min, want_max, t, l)
    got_scores = ps.page_scores(Q, kmin, kmax, T, L).cpu().numpy()
    fin = np.isfinite(want_scores)                 # forced pages +inf, past the end -inf
    assert np.array_equal(got_scores[~fin], want_scores[~fin])
    assert_close(got_scores[fin], want_scores[fin], 1e-3, 1e-4, f"{name} scores")

    want_sel = oracle.select(want_scores, kk)
    got_sel = ps.index_select(Q, kmin, kmax, T, L, kk, 0.5).cpu().numpy()
    _sets_agree(got_sel, want_sel, want_scores, f"{name} selection")

    want = oracle.sparse_decode(q, k, v, t, l, np.ascontiguousarray(got_sel), ratio=0.5)
    got_list = ps.sparse_decode(Q, K, V, T, L, torch.from_numpy(got_sel).cuda(), ratio=0.5)
    torch.cuda.synchronize()
    assert_close(got_list.float().cpu().numpy(), want, ATOL, RTOL, f"{name} list decode")
    # the benchmark's call: scoring, selection and attention in one launch
    got_fused = ps.sparse_attention(Q, K, V, T, L, kmin, kmax, ratio=0.5, max_seq_len=ctx)
    torch.cuda.synchronize()
    assert_close(got_fused.float().cpu().numpy(), want, ATOL, RTOL,
                 f"{name} selecting decode")
    # and the oracle's own selection gives the same output where the sets agree
    if all(set(got_sel[i, j].tolist()) == set(want_sel[i, j].tolist())
           for i in range(batch) for j in range(H_KV)):
        want2 = oracle.sparse_decode(q, k, v, t, l, want_sel, ratio=0.5)
        assert_close(got_fused.float().cpu().numpy(), want2, ATOL, RTOL,
                     f"{name} vs oracle select")


def test_c5_sparse_half_b8x32k():
    _sparse_half_at_full_size(8, 32768, seed=5, name="c5")


def test_c5h_sparse_half_b16x16k():
    """The headline shape with half of every sequence's pages kept (the
    reference reports its sparse pipeline at B16 x 16K:
    docs/phase14_sparse.md:130)."""
    _sparse_half_at_full_size(16, 16384, seed=51, name="c5h")


def _fp32_decode_reference(model, ctx_len, ids, positions):
    """fp32 forward of the decode tokens ids [B, T] at positions [T], each
    attending the fp16 context K/V already in the cache (positions <
    ctx_len, gathered through the block tables) and the fp32 K/V of the
    decode tokens up to itself -> logits [B, T, vocab] fp32."""
    import math

    cfg, cache = model.cfg, model.cache
    b, t = ids.shape
    hq, hk, hd = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    qd, kvd, rep = hq * hd, hk * hd, hq // hk
    cos, sin = model.rope.cos[positions].float(), model.rope.sin[positions].float()

    def rope(z):                                              # [B, H, T, D]
        rot = torch.cat([-z[..., hd // 2:], z[..., :hd // 2]], dim=-1)
        return z * cos + rot * sin

    def norm(z, w):
        return z * torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + cfg.rms_norm_eps) * w.float()

    tables = cache.block_tables_tensor(b).long()
    pages = -(-ctx_len // PAGE)
    causal = torch.full((t, t), float("-inf"), device="cuda").triu(1)
    x = model.embed[ids].float()
    for li, layer in enumerate(model.layers):
        kc = cache.k_pool[li][tables[:, :pages]].view(b, pages * PAGE, hk, hd)[:, :ctx_len]
        vc = cache.v_pool[li][tables[:, :pages]].view(b, pages * PAGE, hk, hd)[:, :ctx_len]
        kc, vc = kc.transpose(1, 2).float(), vc.transpose(1, 2).float()   # [B, hk, L, D]
        h = norm(x, layer.norm1)
        qkv = h @ layer.w_qkv.float().T + layer.b_qkv.float()
        q = rope(qkv[..., :qd].view(b, t, hq, hd).transpose(1, 2))          # [B, hq, T, D]
        k = rope(qkv[..., qd:qd + kvd].view(b, t, hk, hd).transpose(1, 2))  # [B, hk, T, D]
        v = qkv[..., qd + kvd:].view(b, t, hk, hd).transpose(1, 2)
        keys = torch.cat([kc, k], dim=2).unsqueeze(2)                       # [B, hk, 1, L+T, D]
        vals = torch.cat([vc, v], dim=2).unsqueeze(2)
        qg = q.view(b, hk, rep, t, hd)
        s = qg @ keys.transpose(-1, -2) / math.sqrt(hd)                    # [B, hk, rep, T, L+T]
        s[..., ctx_len:] += causal
        att = (torch.softmax(s, dim=-1) @ vals).view(b, hq, t, hd)
        x = x + att.transpose(1, 2).reshape(b, t, qd) @ layer.w_o.float().T
        h = norm(x, layer.norm2)
        g, u = (h @ layer.w_gate_up.float().T).chunk(2, dim=-1)
        x = x + (torch.nn.functional.silu(g) * u) @ layer.w_down.float().T
    return norm(x, model.norm) @ model.lm_head.float().T


def test_c5_full_step_b16x8k_graphed_matches_fp32():
    """BASELINE configuration 5's full step: Qwen2.5-1.5B geometry (28
    layers, vocab 151936, random weights), B16 at ~8K context, through the
    HIP-graph runner's 8192 bucket; three consecutive steps against an fp32
    forward of the same weights over the same cache context."""
    from latentserve_amd.runtime.hip_graph import GraphedDecoder
    from latentserve_amd.runtime.qwen_decoder import DecoderConfig, QwenDecoder

    print("full step: Qwen2.5-1.5B geometry B16 x 8K, graphed", flush=True)
    b, cap, start, steps = 16, 8192, 8000, 3
    model = QwenDecoder(DecoderConfig(), seed=11)
    cache = model.allocate_cache(b, cap)
    cache.advance(start, batch_size=b)
    g = torch.Generator(device="cuda").manual_seed(12)
    for li in range(model.cfg.num_layers):
        cache.k_pool[li].normal_(generator=g)
        cache.v_pool[li].normal_(generator=g)
    dec = GraphedDecoder(model, buckets=(cap,))
    ids = torch.randint(0, model.cfg.vocab_size, (b, steps), device="cuda", generator=g)
    got = []
    for s in range(steps):
        pos = torch.full((b, 1), start + s, dtype=torch.long, device="cuda")
        got.append(dec.step(ids[:, s:s + 1], pos, list(range(b)))[:, -1].float().clone())
    torch.cuda.synchronize()
    assert dec.stats()["graph_steps"] == steps and dec.stats()["captures"] == 1
    want = _fp32_decode_reference(model, start, ids,
                                  torch.arange(start, start + steps, device="cuda"))
    for s in range(steps):
        w, gt = want[:, s], got[s]
        scale = w.abs().max().item()
        err = (gt - w).abs().max().item()
        assert err <= 2e-2 * scale + 1e-3, (s, err, scale)
        top2 = w.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 2 * (2e-2 * scale + 1e-3)
        assert torch.equal(gt.argmax(-1)[clear], w.argmax(-1)[clear]), s
