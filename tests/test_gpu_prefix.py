"""Prefix sharing on an MI355X: a sequence started on another sequence's
pages decodes exactly as the same sequence written from scratch, fp16 and
INT8 (the reference's tests/test_phase13_prefix.py:18-66 and :140-152
exactness, at the cache level: the same K/V bytes reach the kernel
through shared pages)."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

H, D, BS = 2, 128, 16


def _cache(kind, batch=3, cap=256):
    from latentserve_amd.runtime.kv_cache import KVCacheSpec, PagedKVCache
    spec = KVCacheSpec(num_layers=1, num_kv_heads=H, head_dim=D, max_batch_size=batch,
                       max_seq_len=cap, device="cuda")
    if kind == "int8":
        from latentserve_amd.runtime.int8_cache import Int8PagedKVCache
        return Int8PagedKVCache(spec)
    return PagedKVCache(spec)


def _kv(gen, n):
    k = torch.randn(1, H, n, D, generator=gen).half().cuda()
    v = torch.randn(1, H, n, D, generator=gen).half().cuda()
    return k, v


def _write(c, slot, k, v, chunk=None):
    """Prefill k, v [1, H, n, D] into slot in chunks, then nothing else."""
    n = k.shape[2]
    step = chunk or n
    for a in range(0, n, step):
        b = min(n, a + step)
        c.advance(b - a, slots=[slot])
        c.write(0, k[:, :, a:b], v[:, :, a:b])


def _decode(c, slot, q):
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh
    c.advance(0, slots=[slot])
    tables = c.block_tables_tensor(1)
    lens = c.seq_lens_tensor(1)
    extra = {}
    if hasattr(c, "residual"):
        extra = dict(k_scale=c.k_scale_pool[0], v_scale=c.v_scale_pool[0],
                     k_residual=c.residual(0), res_rows=c.residual_rows_tensor(1))
    out = pdh.paged_decode_hip(q, c.k_pool[0], c.v_pool[0], tables, lens, 256, **extra)
    return out.clone()


@pytest.mark.parametrize("kind", ["fp16", "int8"])
def test_a_shared_prefix_decodes_exactly_as_written_from_scratch(kind):
    from latentserve_amd.runtime.prefix_cache import PrefixCache

    gen = torch.Generator().manual_seed(3)
    prefix_k, prefix_v = _kv(gen, 70)                 # 4 full pages and 6 tokens
    tail_k, tail_v = _kv(gen, 29)                     # the second sequence's own tokens
    q = torch.randn(1, H, 6, D, generator=gen).half().cuda()

    c = _cache(kind)
    pc = PrefixCache(c.allocator, BS)
    _write(c, 0, prefix_k, prefix_v, chunk=24)        # sequence A: the prefix and more
    tokens_a = list(range(70))
    pages = c.shareable_blocks(0)
    assert pages == 4
    pc.register(tokens_a[:pages * BS], c.tables[0].blocks[:pages])
    # sequence B: the same first 64 tokens, then its own
    tokens_b = tokens_a[:64] + list(range(1000, 1029))
    hit = pc.match(tokens_b)
    assert len(hit) == 4
    c.attach_prefix(1, hit, 64)
    _write(c, 1, tail_k, tail_v, chunk=13)
    got = _decode(c, 1, q)

    # the same sequence B written whole into a fresh cache
    full_k = torch.cat([prefix_k[:, :, :64], tail_k], dim=2)
    full_v = torch.cat([prefix_v[:, :, :64], tail_v], dim=2)
    ref = _cache(kind)
    _write(ref, 0, full_k, full_v, chunk=13)
    want = _decode(ref, 0, q)
    assert torch.equal(got, want)
    # A is untouched by B's writes
    got_a = _decode(c, 0, q)
    ref_a = _cache(kind)
    _write(ref_a, 0, prefix_k, prefix_v, chunk=24)
    assert torch.equal(got_a, _decode(ref_a, 0, q))


def test_int8_shares_only_pages_whose_k_is_quantized():
    """A full last page keeps its K in the slot's residual until the next
    token opens a new page (cache/int8_paged_cache.py:385-396)."""
    gen = torch.Generator().manual_seed(5)
    c = _cache("int8")
    k, v = _kv(gen, 64)                               # exactly 4 pages
    _write(c, 0, k, v)
    assert c.shareable_blocks(0) == 3
    k1, v1 = _kv(gen, 1)
    _write(c, 0, k1, v1)                              # the 65th token: page 4 is quantized
    assert c.shareable_blocks(0) == 4
