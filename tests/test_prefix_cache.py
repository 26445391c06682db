"""Prefix sharing on the CPU: keys, matching, recording, eviction and the
allocator hooks (the reference's tests/test_phase13_prefix.py:113-250: a
match verified against the stored tokens, chained keys, free only at zero
with and without a hook, the O(1) reclaimable count equal to the scan after
a workload with sharing, finishing and eviction, every block free or held
by the cache alone once everything finished), and attach_prefix on the
fp16 cache."""

from __future__ import annotations

import random

import numpy as np
import pytest

from latentserve_amd.runtime.kv_cache import (BlockAllocator, BlockTable, KVCacheSpec,
                                              OutOfBlocks, PagedKVCache)
from latentserve_amd.runtime.prefix_cache import PrefixCache, block_keys


def test_a_match_is_verified_against_the_stored_tokens():
    alloc = BlockAllocator(num_blocks=8, block_size=4)
    pc = PrefixCache(alloc, 4)
    blocks = alloc.allocate(2)
    assert pc.register([1, 2, 3, 4, 5, 6, 7, 8], blocks) == 2
    assert pc.match([1, 2, 3, 4, 5, 6, 7, 8, 9]) == blocks
    # a stored page whose tokens differ under the same key (a collision)
    key, parent, _ = pc.entry[blocks[0]]
    pc.entry[blocks[0]] = (key, parent, (9, 9, 9, 9))
    assert pc.match([1, 2, 3, 4, 5, 6, 7, 8, 9]) == []


def test_keys_chain_so_equal_pages_after_different_prefixes_differ():
    a = block_keys([1, 2, 3, 4, 7, 7, 7, 7], 4)
    b = block_keys([9, 9, 9, 9, 7, 7, 7, 7], 4)
    assert a[1][2] == b[1][2] and a[1][0] != b[1][0]
    assert a[1][1] == a[0][0]                         # the parent is the previous page's key
    assert block_keys([1, 2, 3], 4) == []             # no full page, no key


def test_the_last_token_is_never_matched():
    alloc = BlockAllocator(num_blocks=8, block_size=16)
    pc = PrefixCache(alloc, 16)
    prompt = list(range(5, 5 + 64))                   # exactly 4 pages
    pc.register(prompt, alloc.allocate(4))
    assert len(pc.match(prompt)) == 3                 # the 4th page holds the last token
    assert len(pc.match(prompt + [1])) == 4
    assert pc.stats()["lookups"] == 2 and pc.stats()["hits"] == 2


@pytest.mark.parametrize("hooked", [False, True])
def test_free_returns_a_block_to_the_pool_only_at_zero(hooked):
    alloc = BlockAllocator(num_blocks=4, block_size=4)
    seen = []
    if hooked:
        alloc.on_ref_change = lambda b, old, new: seen.append((b, old, new))
    [b] = alloc.allocate(1)
    alloc.incref([b])
    alloc.free([b])
    assert alloc.ref_count(b) == 1 and alloc.num_free == 3
    alloc.free([b])
    assert alloc.ref_count(b) == 0 and alloc.num_free == 4
    if hooked:
        assert seen == [(b, 1, 2), (b, 2, 1), (b, 1, 0)]


def test_registering_a_page_twice_or_under_two_keys_keeps_one_entry():
    alloc = BlockAllocator(num_blocks=8, block_size=4)
    pc = PrefixCache(alloc, 4)
    blocks = alloc.allocate(2)
    toks = [1, 2, 3, 4, 5, 6, 7, 8]
    assert pc.register(toks, blocks) == 2
    assert pc.register(toks, blocks) == 0             # same pages, same keys: a touch
    assert pc.register([9, 9, 9, 9], blocks[:1]) == 0  # the page is recorded under another key
    assert [alloc.ref_count(b) for b in blocks] == [2, 2]


def _serve(num_blocks, prompts, max_running, seed=0, gen=(3, 30)):
    """A host-only serving loop: admit (matching the prefix cache), prefill,
    decode a few tokens, register, finish — the block traffic of a server."""
    rng = random.Random(seed)
    bs = 16
    alloc = BlockAllocator(num_blocks, bs)
    pc = PrefixCache(alloc, bs)
    waiting = list(prompts)
    running = []                                      # (table, tokens, tokens still to make)
    hit_tokens = 0
    while waiting or running:
        while waiting and len(running) < max_running:
            prompt = waiting[0]
            hit = pc.match(prompt)
            need = alloc.blocks_for_tokens(len(prompt) + gen[1]) - len(hit)
            if need > alloc.num_available:
                break
            waiting.pop(0)
            t = BlockTable(alloc)
            if hit:
                alloc.incref(hit)
                t.blocks = list(hit)
                t.length = len(hit) * bs
                hit_tokens += t.length
            t.append(len(prompt) - t.length)          # prefill the rest
            running.append((t, list(prompt), rng.randint(*gen)))
        for i, (t, toks, left) in enumerate(running):
            t.append(1)
            toks.append(rng.randint(0, 50))
            running[i] = (t, toks, left - 1)
        done = [r for r in running if r[2] <= 0]
        running = [r for r in running if r[2] > 0]
        for t, toks, _ in done:
            pc.register(toks[:t.length], t.blocks)    # every full page written
            t.free()
        assert pc.num_reclaimable() == pc.count_reclaimable_by_scan()
    return alloc, pc, hit_tokens


def test_a_workload_with_sharing_finishing_and_eviction_keeps_the_counts():
    rng = random.Random(4)
    system = list(range(100, 170))                    # 70 shared tokens: 4 full pages
    prompts = [system + [rng.randint(0, 50) for _ in range(rng.randint(5, 40))]
               for _ in range(6)]
    prompts += [[rng.randint(0, 50) for _ in range(60)] for _ in range(6)]
    alloc, pc, hits = _serve(num_blocks=24, prompts=prompts, max_running=2)
    assert hits > 0 and pc.evictions > 0
    assert pc.num_reclaimable() == pc.count_reclaimable_by_scan()
    cached = set(pc.entry)
    assert all(alloc.ref_count(b) == 1 for b in cached)
    assert alloc.num_free + len(cached) == alloc.num_blocks
    assert pc.num_reclaimable() == len(cached)


def test_allocation_reclaims_cache_only_pages_and_admission_counts_them():
    alloc = BlockAllocator(num_blocks=4, block_size=4)
    pc = PrefixCache(alloc, 4)
    t = BlockTable(alloc)
    t.append(16)                                      # all 4 blocks
    pc.register(list(range(16)), t.blocks)
    t.free()                                          # held by the cache alone now
    assert alloc.num_free == 0 and alloc.num_available == 4
    got = alloc.allocate(3)                           # evicts the 3 least recently used
    assert len(got) == 3 and pc.evictions == 3 and len(pc.entry) == 1
    with pytest.raises(OutOfBlocks):
        alloc.allocate(2)                             # one left, and the cache's last page


def _cache(batch=3, cap=128):
    spec = KVCacheSpec(num_layers=1, num_kv_heads=2, head_dim=128, max_batch_size=batch,
                       max_seq_len=cap, device="cpu")
    return PagedKVCache(spec)


def test_attach_prefix_starts_a_slot_on_shared_pages():
    c = _cache()
    c.advance(40, slots=[0])
    shared = c.tables[0].blocks[:c.shareable_blocks(0)]
    assert c.shareable_blocks(0) == 2
    c.attach_prefix(1, shared, 32)
    assert [c.allocator.ref_count(b) for b in shared] == [2, 2]
    c.advance(5, slots=[1])
    t1 = c.tables[1]
    assert t1.blocks[:2] == shared and t1.length == 37 and len(t1.blocks) == 3
    row = c.block_tables_tensor(1)[0, :3].numpy()
    assert np.array_equal(row, np.array(t1.blocks, dtype=np.int32))
    c.free_sequence(0)
    assert [c.allocator.ref_count(b) for b in shared] == [1, 1]
    with pytest.raises(ValueError):
        c.attach_prefix(1, shared, 32)                # not empty
    with pytest.raises(ValueError):
        c.attach_prefix(2, shared, 30)                # not whole pages
    assert c.can_admit(16)
