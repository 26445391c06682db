"""Cache bookkeeping on the CPU: allocator, block tables, advance / write.

Follows the reference's own cache tests (tests/test_phase3_paged_cache.py:
LIFO reuse, the slot rule, out-of-blocks as a typed error; capacity-width
persistent tables, tests/test_phase13_graph.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from latentserve_amd.runtime.kv_cache import (BlockAllocator, BlockTable, KVCacheSpec,
                                              OutOfBlocks, PagedKVCache)


def test_allocator_hands_out_ascending_then_reuses_lifo():
    a = BlockAllocator(num_blocks=8, block_size=16)
    assert a.allocate(3) == [0, 1, 2]
    a.free([1])
    a.free([0])
    assert a.allocate(2) == [0, 1]          # most recently freed first
    assert a.num_used == 3 and a.peak_used == 3


def test_allocator_out_of_blocks_is_typed_and_refcounts_hold():
    a = BlockAllocator(num_blocks=2, block_size=16)
    blocks = a.allocate(2)
    with pytest.raises(OutOfBlocks):
        a.allocate(1)
    a.incref([blocks[0]])
    a.free(blocks)
    assert a.num_free == 1                  # block 0 still referenced once
    with pytest.raises(ValueError):
        a.free([blocks[1]])


def test_block_table_slot_rule():
    a = BlockAllocator(num_blocks=10, block_size=16)
    a.allocate(3)                           # make the table's blocks non-trivial
    t = BlockTable(a)
    t.append(40)
    assert t.blocks == [3, 4, 5]
    assert t.slot(0) == 48 and t.slot(17) == 4 * 16 + 1 and t.slot(39) == 5 * 16 + 7
    with pytest.raises(IndexError):
        t.slot(40)
    v = t.version
    t.append(8)                             # still inside block 5: no new block
    assert t.version == v and len(t.blocks) == 3
    t.append(1)
    assert t.version == v + 1 and len(t.blocks) == 4


def test_allocator_stats_and_reset_follow_the_reference():
    """stats() under the reference's keys, reset() clearing the peak and the
    call counts as well (cache/block_allocator.py:147-161)."""
    a = BlockAllocator(num_blocks=8, block_size=16)
    a.allocate(5)
    a.free([4, 3])
    a.allocate(1)
    st = a.stats()
    assert st == {"num_blocks": 8, "block_size": 16, "blocks_used": 4, "blocks_free": 4,
                  "block_utilization": 0.5, "peak_blocks_used": 5, "alloc_calls": 2,
                  "free_calls": 1}
    a.reset()
    assert a.stats()["peak_blocks_used"] == 0 and a.alloc_calls == 0 and a.free_calls == 0
    assert a.allocate(2) == [0, 1]


def test_block_table_capacity_wasted_slots_and_reserve():
    """capacity / wasted_slots / reserve as the reference's BlockTable
    (cache/block_allocator.py:190-212): reserve allocates pages for tokens
    to come without counting them."""
    a = BlockAllocator(num_blocks=10, block_size=16)
    t = BlockTable(a)
    t.reserve(20)
    assert t.length == 0 and t.capacity == 32 and t.wasted_slots == 32 and t.version == 1
    t.append(20)                            # the reserved pages suffice
    assert t.blocks == [0, 1] and t.version == 1 and t.wasted_slots == 12
    t.reserve(12)
    assert t.version == 1 and t.capacity == 32
    t.reserve(13)
    assert t.version == 2 and t.capacity == 48 and t.length == 20


def _cache(batch=3, cap=100, layers=2):
    spec = KVCacheSpec(num_layers=layers, num_kv_heads=2, head_dim=128, max_batch_size=batch,
                       max_seq_len=cap, device="cpu")
    return PagedKVCache(spec)


def test_advance_keeps_persistent_capacity_width_buffers():
    c = _cache()
    c.advance(20, batch_size=2)
    bt, sl = c.block_tables_tensor(), c.seq_lens_tensor()
    base = c.inputs.tables.data_ptr()
    assert bt.shape == (2, 7) and sl.tolist() == [20, 20]
    assert bt.data_ptr() == base
    c.advance(1, slots=[1, 0])
    assert c.seq_lens_tensor().tolist() == [21, 21]
    assert c.block_tables_tensor().data_ptr() == base
    rows = c.block_tables_tensor()
    assert rows[0, :2].tolist() == c.tables[1].blocks and rows[1, :2].tolist() == c.tables[0].blocks
    assert c.write_slots(2).tolist() == [c.tables[1].slot(20), c.tables[0].slot(20)]
    assert c.write_slots(2).data_ptr() == c.inputs.vec["write_slot"].data_ptr()


def test_write_scatters_to_the_advanced_slots():
    c = _cache()
    c.advance(5, batch_size=2)
    rng = np.random.default_rng(0)
    k = torch.from_numpy(rng.standard_normal((2, 2, 5, 128)).astype(np.float16))
    v = torch.from_numpy(rng.standard_normal((2, 2, 5, 128)).astype(np.float16))
    c.write(1, k, v)
    for b in range(2):
        for p in range(5):
            s = c.tables[b].slot(p)
            assert torch.equal(c.k_pool[1].view(-1, 2, 128)[s], k[b, :, p])
            assert torch.equal(c.v_pool[1].view(-1, 2, 128)[s], v[b, :, p])
    assert c.k_pool[0].abs().sum() == 0


def test_table_rows_follow_slot_reuse_and_growth():
    """A row reassigned to another sequence is rewritten whole; a row whose
    sequence only grew gets its new entries; a freed-and-refilled slot is
    never served its old blocks."""
    c = _cache(batch=2, cap=200)
    c.advance(40, batch_size=2)                         # 3 pages each
    c.advance(1, slots=[1])                             # row 0 now holds slot 1
    assert c.block_tables_tensor(1)[0, :3].tolist() == c.tables[1].blocks
    c.free_sequence(0)
    c.advance(33, slots=[0])                            # slot 0 refilled: LIFO blocks
    assert c.block_tables_tensor(1)[0, :3].tolist() == c.tables[0].blocks
    for _ in range(20):                                 # grows by one page
        c.advance(1, slots=[0, 1])
    rows = c.block_tables_tensor(2)
    for r, s in enumerate([0, 1]):
        assert rows[r, :len(c.tables[s].blocks)].tolist() == c.tables[s].blocks
    assert c.seq_lens_tensor().tolist() == [53, 61]


def test_capacity_is_enforced_and_rewind_keeps_blocks():
    c = _cache(batch=1, cap=32)
    c.advance(30, batch_size=1)
    blocks = list(c.tables[0].blocks)
    c.rewind(10)
    assert c.seq_lens_tensor().tolist() == [10] and c.tables[0].blocks == blocks
    c.advance(22, batch_size=1)
    assert c.tables[0].blocks == blocks
    with pytest.raises(RuntimeError):
        c.advance(1, batch_size=1)          # 33 tokens need a third page: past capacity


def test_rope_tables_are_qwen2_rotary_embedding():
    """The decoder's cos / sin tables are transformers' Qwen2RotaryEmbedding
    (fp32 angles, cast to fp16) bit for bit."""
    import pytest
    qm = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    from transformers import Qwen2Config
    from latentserve_amd.runtime.qwen_decoder import DecoderConfig, Rope

    c = DecoderConfig()
    hf = qm.Qwen2RotaryEmbedding(Qwen2Config(
        hidden_size=c.hidden_size, num_attention_heads=c.num_heads,
        num_key_value_heads=c.num_kv_heads, rope_theta=c.rope_theta,
        max_position_embeddings=4096))
    cos, sin = hf(torch.zeros(1, dtype=torch.float16), torch.arange(4096)[None])
    r = Rope(c.head_dim, c.rope_theta, 4096, "cpu")
    assert torch.equal(cos[0], r.cos) and torch.equal(sin[0], r.sin)
