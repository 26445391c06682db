"""The INT8 paged cache and the graphed INT8 decode step, on an MI355X.

* Cache invariant (cache/int8_paged_cache.py:283-298): after prefill
  chunks and decode steps crossing page boundaries, every page but a
  sequence's last holds K codes and steps bit-exact with the oracle's
  quantizer over that page's fp16 K, every token's V codes and step are
  the oracle's, and the residual row holds the last page's fp16 K exactly;
  the INT8 decode over the cache matches the oracle over the same codes.
* A decode stream through the HIP-graph runner over an INT8 cache equals
  the same stream run eagerly (the reference's
  tests/test_phase14_int8_graph.py:254-268 check), and both stay close to
  the fp32 forward of the same weights.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.cases import assert_close

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

H, D, BS = 2, 128, 16


def _cache(batch, cap, layers=2, asym=False):
    from latentserve_amd.runtime.int8_cache import Int8PagedKVCache
    from latentserve_amd.runtime.kv_cache import KVCacheSpec
    spec = KVCacheSpec(num_layers=layers, num_kv_heads=H, head_dim=D, max_batch_size=batch,
                       max_seq_len=cap, device="cuda")
    return Int8PagedKVCache(spec, asymmetric=asym)


def _check_sequence(c, layer, slot, k_all, v_all, asym):
    """Pool, scales and residual of one sequence against the oracle."""
    t = c.tables[slot]
    n = t.length
    last = (n - 1) // BS
    kp = c.k_pool[layer].cpu().numpy()
    vp = c.v_pool[layer].cpu().numpy()
    ks = c.k_scale_pool[layer].cpu().numpy()
    vs = c.v_scale_pool[layer].cpu().numpy()
    k = k_all[:n].reshape(-1, H, D)
    v = v_all[:n].reshape(-1, H, D)
    if last > 0:
        pages = k[:last * BS].reshape(last, BS, H, D)
        want_q, want_s, want_z = oracle.quantize_k(pages, asym=asym, recip=True)
        blk = t.blocks[:last]
        assert np.array_equal(kp[blk], want_q), (slot, layer)
        assert np.array_equal(ks[blk].view(np.uint32), want_s.view(np.uint32))
        if asym:
            kz = c.k_zero_pool[layer].cpu().numpy()
            assert np.array_equal(kz[blk].view(np.uint32), want_z.view(np.uint32))
    vq, vstep, _ = oracle.quantize_v(v, asym=asym, recip=True)
    slots = np.array(t.slots(0, n))
    assert np.array_equal(vp.reshape(-1, H, D)[slots], vq)
    assert np.array_equal(vs.reshape(-1, H)[slots].view(np.uint32), vstep.view(np.uint32))
    rows = n - last * BS
    res = c.residual(layer)[slot, :rows].cpu().numpy()
    assert np.array_equal(res, k[last * BS:n]), (slot, layer)


@pytest.mark.parametrize("asym", [False, True])
def test_int8_cache_keeps_the_residual_invariant(asym):
    torch.manual_seed(0)
    c = _cache(batch=3, cap=256, asym=asym)
    rng = np.random.default_rng(1)
    hist = {s: [] for s in range(3)}               # fp16 K/V per sequence, [n, H, D]
    hist_v = {s: [] for s in range(3)}

    def write(slots, n):
        c.advance(n, slots=slots)
        k = rng.standard_normal((len(slots), H, n, D), dtype=np.float32).astype(np.float16)
        v = rng.standard_normal((len(slots), H, n, D), dtype=np.float32).astype(np.float16)
        for layer in range(2):
            c.write(layer, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        for r, s in enumerate(slots):
            hist[s].append(np.transpose(k[r], (1, 0, 2)))
            hist_v[s].append(np.transpose(v[r], (1, 0, 2)))

    write([0], 37)            # partial last page
    write([1], 32)            # ends on a page boundary
    write([2], 5)
    write([2], 20)            # a chunk continuing a partial page
    for step in range(40):    # decode across page boundaries
        write([0, 1, 2], 1)
    torch.cuda.synchronize()
    for layer in range(2):
        for s in range(3):
            _check_sequence(c, layer, s, np.concatenate(hist[s]), np.concatenate(hist_v[s]),
                            asym)
    # the decode over the cache against the oracle over the same state
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh
    q = rng.standard_normal((3, H, 6, D), dtype=np.float32).astype(np.float16)
    tables = c.block_tables_tensor(3)
    lens = c.seq_lens_tensor(3)
    extra = dict(k_scale=c.k_scale_pool[1], v_scale=c.v_scale_pool[1],
                 k_residual=c.residual(1), res_rows=c.residual_rows_tensor(3))
    if asym:
        extra.update(k_zero=c.k_zero_pool[1], v_zero=c.v_zero_pool[1])
    got = pdh.paged_decode_hip(torch.from_numpy(q).cuda(), c.k_pool[1], c.v_pool[1], tables,
                               lens, 256, **extra).float().cpu().numpy()
    np_extra = {k: v.cpu().numpy() for k, v in extra.items()}
    want = oracle.paged_decode(q, c.k_pool[1].cpu().numpy(), c.v_pool[1].cpu().numpy(),
                               tables.cpu().numpy(), lens.cpu().numpy(), **np_extra)
    assert_close(got, want, 2e-3, 1e-2, f"int8 cache decode asym={asym}")


def _model(kv, seed=4):
    from latentserve_amd.runtime.qwen_decoder import DecoderConfig, QwenDecoder
    m = QwenDecoder(DecoderConfig(vocab_size=512, intermediate_size=384, num_layers=2),
                    seed=seed, std=0.05)
    m.allocate_cache(2, 128, kv_dtype=kv)
    return m


def test_graphed_int8_decode_matches_eager_int8_and_fp32():
    from latentserve_amd.runtime.hip_graph import GraphedDecoder
    from tests.test_gpu_runtime import reference_logits

    steps = 50                                       # crosses pages 16, 32 and 48
    ids = torch.randint(0, 512, (2, steps), generator=torch.Generator().manual_seed(7)).cuda()
    outs = {}
    for graphed in (False, True):
        m = _model("int8")
        dec = GraphedDecoder(m, buckets=(64,), enabled=graphed)
        got = []
        for t in range(steps):
            pos = torch.full((2, 1), t, dtype=torch.long, device="cuda")
            got.append(dec.step(ids[:, t:t + 1], pos, [0, 1])[:, -1].float().clone())
        outs[graphed] = torch.stack(got)
        st = dec.stats()
        assert (st["graph_steps"], st["eager_steps"]) == ((steps, 0) if graphed else (0, steps))
        assert m.cache.pooled_pages(0) == (steps - 1) // 16
    e, g = outs[False], outs[True]
    # the eager step splits by the current length, the graph by its bucket:
    # a different order of the split sums, a few fp16 steps of the logits
    assert (g - e).abs().max().item() <= 3e-3 * e.abs().max().item() + 1e-4
    # INT8 K/V against the fp32 forward of the same weights
    m = _model("int8")
    want = reference_logits(m, ids)
    err = (g[-1] - want).abs().max().item()
    assert err <= 5e-2 * want.abs().max().item() + 1e-3, err
