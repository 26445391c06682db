"""Paged KV cache bookkeeping for the HIP decode path.

The reference's cache layer (cache/block_allocator.py: BlockAllocator,
BlockTable, OutOfBlocks; cache/paged_cache.py: PagedKVCache) fixes what
the kernels read: per-layer pools ``[num_blocks, 16, H_kv, D]``, a block
table per sequence whose token p lives at flat slot ``blocks[p // 16] * 16
+ p % 16``, blocks handed out lowest id first and reused most recently
freed first.  Those rules are kept; the machinery is this build's own:

* ``StepInputs`` holds every per-step kernel input at a fixed device
  address (a captured graph reads them by pointer): the block-table rows
  at the cache's capacity width, the lengths, the decode token's write
  slot, and for the INT8 cache the residual row and index.  The per-step
  vectors live in one device buffer filled by ONE host-to-device copy from
  a double-buffered pinned staging area; a table row is uploaded only
  where it changed, and a row that only grew uploads just its new tail.
* The allocator keeps a reference count per block id in a flat list and
  the free ids on a stack.

Host-side Python, like the reference's: a decode step's bookkeeping is a
few list operations and one small copy.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Iterable, List, Optional, Sequence

import numpy as np
import torch


class OutOfBlocks(RuntimeError):
    """The pool cannot hold the requested blocks (cache/block_allocator.py:
    31-38): a scheduler's signal to wait or evict, not a crash."""


class BlockAllocator:
    """A fixed pool of equal blocks (cache/block_allocator.py:41-132).

    A fresh pool hands out 0, 1, 2, ...; a freed block is the next one
    handed out (most recently freed first).  Blocks are reference counted
    so a shared prefix can be held by several sequences.

    Three optional hooks let a prefix cache lend the pool the blocks only it
    still holds (cache/block_allocator.py:60-67, 100-103, 131-142):
    ``reclaimable()`` counts them (admission sees them as available),
    ``reclaimer(n)`` gives up to n of them back when an allocation comes up
    short, and ``on_ref_change(block, old, new)`` reports every count change.
    """

    def __init__(self, num_blocks: int, block_size: int):
        if num_blocks < 1 or block_size < 1:
            raise ValueError(f"a pool needs at least one block of at least one token "
                             f"(got {num_blocks} blocks of {block_size})")
        self.num_blocks = int(num_blocks)
        self.block_size = int(block_size)
        self._refs: List[int] = [0] * self.num_blocks
        self._stack: List[int] = []
        self.peak_used = 0
        self.alloc_calls = 0
        self.free_calls = 0
        self.reclaimer: Optional[Callable[[int], object]] = None
        self.reclaimable: Optional[Callable[[], int]] = None
        self.on_ref_change: Optional[Callable[[int, int, int], None]] = None
        self.reset()

    def reset(self) -> None:
        """Every block free again and the counters at zero: the pool as new."""
        self._refs = [0] * self.num_blocks
        self._stack = list(range(self.num_blocks - 1, -1, -1))   # top = lowest id
        self.peak_used = self.alloc_calls = self.free_calls = 0

    def stats(self) -> dict:
        """The pool's occupancy and traffic, under the reference's keys
        (cache/block_allocator.py:152-161)."""
        return {"num_blocks": self.num_blocks, "block_size": self.block_size,
                "blocks_used": self.num_used, "blocks_free": self.num_free,
                "block_utilization": self.utilization, "peak_blocks_used": self.peak_used,
                "alloc_calls": self.alloc_calls, "free_calls": self.free_calls}

    @property
    def num_free(self) -> int:
        return len(self._stack)

    @property
    def num_used(self) -> int:
        return self.num_blocks - len(self._stack)

    @property
    def utilization(self) -> float:
        return self.num_used / self.num_blocks

    def blocks_for_tokens(self, num_tokens: int) -> int:
        return -(-int(num_tokens) // self.block_size)

    @property
    def num_available(self) -> int:
        """What an allocation can get: free blocks, and blocks a prefix
        cache holds alone."""
        return len(self._stack) + (self.reclaimable() if self.reclaimable else 0)

    def allocate(self, count: int) -> List[int]:
        count = int(count)
        if count > len(self._stack) and self.reclaimer is not None:
            self.reclaimer(count - len(self._stack))
        if count > len(self._stack):
            raise OutOfBlocks(f"cannot allocate {count} blocks: only {len(self._stack)} of "
                              f"{self.num_blocks} are free")
        taken = self._stack[len(self._stack) - count:][::-1]
        del self._stack[len(self._stack) - count:]
        self.alloc_calls += 1
        for b in taken:
            self._refs[b] = 1
        self.peak_used = max(self.peak_used, self.num_used)
        return taken

    def incref(self, blocks: Iterable[int]) -> None:
        for b in blocks:
            if not 0 <= b < self.num_blocks or self._refs[b] == 0:
                raise ValueError(f"block {b} is free; only allocated blocks can be shared")
            self._refs[b] += 1
            if self.on_ref_change is not None:
                self.on_ref_change(b, self._refs[b] - 1, self._refs[b])

    def free(self, blocks: Iterable[int]) -> None:
        """Drop one reference to each block; a block whose count reaches
        zero goes back on the stack."""
        self.free_calls += 1
        for b in blocks:
            if not 0 <= b < self.num_blocks or self._refs[b] == 0:
                raise ValueError(f"block {b} is already free")
            self._refs[b] -= 1
            if self._refs[b] == 0:
                self._stack.append(b)
            if self.on_ref_change is not None:
                self.on_ref_change(b, self._refs[b] + 1, self._refs[b])

    def ref_count(self, block: int) -> int:
        return self._refs[block]

    refcount = ref_count


class BlockTable:
    """One sequence's pages (cache/block_allocator.py:165-229).

    ``blocks``: physical ids in logical order; ``length``: tokens written;
    ``version``: bumped whenever ``blocks`` changes (a new page, a free), so
    a mirror of the table knows to refresh.
    """

    def __init__(self, allocator: BlockAllocator):
        self.allocator = allocator
        self.blocks: List[int] = []
        self.length = 0
        self.version = 0
        # bumped when the block list is replaced rather than extended: a
        # mirror that saw an older lineage re-uploads the whole row
        self.lineage = 0

    @property
    def capacity(self) -> int:
        """Token slots of the table's pages."""
        return len(self.blocks) * self.allocator.block_size

    @property
    def wasted_slots(self) -> int:
        """Slots of the last page past the tokens written (internal
        fragmentation, under one page a sequence)."""
        return self.capacity - self.length

    def reserve(self, num_tokens: int) -> None:
        """Pages for length + num_tokens tokens, allocated as needed; the
        length is unchanged (cache/block_allocator.py:198-208)."""
        need = self.allocator.blocks_for_tokens(self.length + num_tokens) - len(self.blocks)
        if need > 0:
            self.blocks.extend(self.allocator.allocate(need))
            self.version += 1

    def append(self, num_tokens: int) -> None:
        """Make room for num_tokens more tokens (new pages as needed)."""
        self.reserve(num_tokens)
        self.length += num_tokens

    def slot(self, position: int) -> int:
        if not 0 <= position < self.length:
            raise IndexError(f"position {position} is outside the sequence (length "
                             f"{self.length})")
        page, off = divmod(position, self.allocator.block_size)
        return self.blocks[page] * self.allocator.block_size + off

    def slots(self, start: int = 0, end: Optional[int] = None) -> List[int]:
        end = self.length if end is None else end
        return [self.slot(p) for p in range(start, end)]

    def free(self) -> None:
        self.allocator.free(self.blocks)
        self.blocks = []
        self.length = 0
        self.version += 1
        self.lineage += 1


@dataclass
class KVCacheSpec:
    """Geometry of a cache (the fields of the reference's cache/kv_cache.py
    KVCacheSpec that a paged cache reads)."""

    num_layers: int
    num_kv_heads: int
    head_dim: int
    max_batch_size: int
    max_seq_len: int
    dtype: torch.dtype = torch.float16
    device: str = "cuda"


class StepInputs:
    """Per-step kernel inputs at fixed device addresses.

    ``tables`` [max_batch, capacity_pages] int32, and four vectors of
    max_batch entries carved from one device buffer: ``write_slot`` int64
    (the decode token's flat slot), ``res_index`` int64 (its row in the
    flattened INT8 residual), ``lens`` int32 and ``res_row`` int32 (each
    sequence's residual row).  ``publish`` writes the step's values into a
    pinned staging area and issues asynchronous copies: the changed table
    entries, then the whole vector buffer in one copy.  Two staging areas
    alternate; one is refilled only after the copies that last read it
    have run, so the host never waits for the step before.
    """

    _FIELDS = (("write_slot", np.int64), ("res_index", np.int64),
               ("lens", np.int32), ("res_row", np.int32))

    def __init__(self, max_batch: int, capacity_pages: int, block_size: int, device):
        self.max_batch = mb = int(max_batch)
        self.capacity_pages = cap = max(1, int(capacity_pages))
        self.block_size = int(block_size)
        self.device = torch.device(device)
        self.tables = torch.zeros((mb, cap), dtype=torch.int32, device=self.device)
        offs, pos = {}, 0
        for name, dt in self._FIELDS:
            offs[name] = (pos, pos + mb * np.dtype(dt).itemsize)
            pos = offs[name][1]
        self._dev = torch.zeros(pos, dtype=torch.uint8, device=self.device)
        self.vec = {name: self._dev[a:b].view(_TORCH[dt])
                    for (name, dt), (a, b) in zip(self._FIELDS, offs.values())}
        # the values of every field as last published (host copy)
        self._cur = np.zeros(pos, dtype=np.uint8)
        self._cur_views = {name: self._cur[a:b].view(dt)
                           for (name, dt), (a, b) in zip(self._FIELDS, offs.values())}
        self._async = self.device.type == "cuda"
        self._stage = []
        for _ in range(2 if self._async else 1):
            vec = torch.zeros(pos, dtype=torch.uint8, pin_memory=self._async)
            tab = torch.zeros((mb, cap), dtype=torch.int32, pin_memory=self._async)
            self._stage.append((vec, tab, torch.cuda.Event() if self._async else None))
        self._turn = 0
        # per table row: (sequence slot, its lineage, entries uploaded)
        self._row_state: List[Optional[tuple]] = [None] * mb

    def forget_rows(self) -> None:
        self._row_state = [None] * self.max_batch

    def publish(self, seqs: Sequence[int], tables: Sequence[BlockTable],
                **values: Sequence[int]) -> None:
        """Row r of the device table mirrors tables[seqs[r]].blocks; each
        vector given is set for rows 0..len-1 (vectors not given keep their
        last published values)."""
        if self._async:
            self._turn ^= 1
        vec, tab, ev = self._stage[self._turn]
        if ev is not None:
            ev.synchronize()                    # the copies that last read this area ran
        tab_np = tab.numpy()
        for row, s in enumerate(seqs):
            t = tables[s]
            n = len(t.blocks)
            if n > self.capacity_pages:
                raise RuntimeError(f"the sequence in slot {s} holds {n} pages; the cache was "
                                   f"sized for {self.capacity_pages}")
            st = self._row_state[row]
            first = st[2] if st is not None and st[0] == s and st[1] == t.lineage \
                and st[2] <= n else 0
            if first < n:
                tab_np[row, first:n] = t.blocks[first:n]
                self.tables[row, first:n].copy_(tab[row, first:n], non_blocking=self._async)
            self._row_state[row] = (s, t.lineage, n)
        for name, vals in values.items():
            self._cur_views[name][:len(vals)] = vals
        vec.numpy()[:] = self._cur
        self._dev.copy_(vec, non_blocking=self._async)
        if ev is not None:
            ev.record()


_TORCH = {np.int64: torch.int64, np.int32: torch.int32}


class _PagedBase:
    """Bookkeeping shared by the fp16 and INT8 paged caches: allocator,
    per-slot tables, the active set, and the kernel inputs."""

    def __init__(self, spec: KVCacheSpec, block_size: int, num_blocks: Optional[int]):
        if block_size != 16:
            raise ValueError(f"the HIP kernels read 16-token pages, not {block_size}")
        self.spec = spec
        self.block_size = block_size
        self.device = torch.device(spec.device)
        self.capacity_pages = -(-spec.max_seq_len // block_size)
        self.num_blocks = num_blocks or self.capacity_pages * spec.max_batch_size
        self.allocator = BlockAllocator(self.num_blocks, block_size)
        self.tables = [BlockTable(self.allocator) for _ in range(spec.max_batch_size)]
        self.inputs = StepInputs(spec.max_batch_size, self.capacity_pages, block_size,
                                 self.device)
        self._active: List[int] = list(range(spec.max_batch_size))
        self._batch = 0                       # rows published by the last advance()
        self._chunk_slots: Optional[torch.Tensor] = None    # multi-token write slots
        # When set (a graph runner's bucket), sparse selection is sized for it.
        self.sparse_context_hint: Optional[int] = None

    # ---- the active set ---------------------------------------------------
    @property
    def seq_lens(self) -> List[int]:
        return [self.tables[s].length for s in self._active]

    @property
    def max_len(self) -> int:
        return max((self.tables[s].length for s in self._active), default=0)

    @property
    def active_slots(self) -> List[int]:
        return list(self._active)

    def set_active(self, slots: Sequence[int]) -> None:
        self._active = list(slots)

    def can_admit(self, num_tokens: int) -> bool:
        """Whether a prompt of num_tokens fits now (blocks a prefix cache
        holds alone count: an allocation reclaims them)."""
        return self.allocator.blocks_for_tokens(num_tokens) <= self.allocator.num_available

    def free_sequence(self, index: int) -> None:
        self.tables[index].free()

    # ---- prefix sharing ---------------------------------------------------
    def attach_prefix(self, index: int, blocks: Sequence[int], num_tokens: int) -> None:
        """Start the empty slot `index` on `blocks`, whole pages already
        written by another sequence with the same first num_tokens tokens
        (cache/paged_cache.py:199-217).  The slot takes a reference to each;
        pages are append-only, so a shared page is never written again."""
        t = self.tables[index]
        if t.length or t.blocks:
            raise ValueError(f"slot {index} already holds a sequence")
        if num_tokens != len(blocks) * self.block_size:
            raise ValueError(f"a shared prefix is whole pages: {len(blocks)} pages hold "
                             f"{len(blocks) * self.block_size} tokens, not {num_tokens}")
        self.allocator.incref(blocks)
        t.blocks = list(blocks)
        t.length = int(num_tokens)
        t.version += 1
        t.lineage += 1

    def shareable_blocks(self, index: int) -> int:
        """Leading pages of slot `index` whose K/V in the pool is final, so a
        prefix cache may hand them to another sequence."""
        return self.tables[index].length // self.block_size

    def reset(self) -> None:
        """Forget every sequence; storage (and every address a graph holds)
        is kept."""
        for t in self.tables:
            if t.blocks:
                t.free()
        self.allocator.reset()
        self._active = list(range(self.spec.max_batch_size))
        self._batch = 0
        self._chunk_slots = None
        self.inputs.forget_rows()

    # ---- per-step inputs --------------------------------------------------
    def _grow(self, n: int, batch_size, slots) -> List[int]:
        """Extend the active sequences by n tokens; returns their old lengths."""
        if slots is not None:
            self.set_active(slots)
        elif batch_size is not None:
            self.set_active(range(batch_size))
        starts = [self.tables[s].length for s in self._active]
        for s in self._active:
            self.tables[s].append(n)
        return starts

    def _publish(self, n: int, starts: List[int], extra: Optional[dict] = None) -> None:
        seqs = self._active
        vals = {"lens": [self.tables[s].length for s in seqs]}
        if n == 1:
            vals["write_slot"] = [self.tables[s].slot(p) for s, p in zip(seqs, starts)]
            self._chunk_slots = None
        else:
            self._chunk_slots = torch.tensor(
                [self.tables[s].slots(p, p + n) for s, p in zip(seqs, starts)],
                dtype=torch.long, device=self.device).reshape(len(seqs), n)
        vals.update(extra or {})
        self.inputs.publish(seqs, self.tables, **vals)
        self._batch = len(seqs)

    def _need(self, b: Optional[int]) -> int:
        if self._batch == 0:
            raise RuntimeError("advance() the cache before asking for kernel inputs")
        b = self._batch if b is None else int(b)
        if b > self._batch:
            raise RuntimeError(f"{b} rows asked for, the last advance() published "
                               f"{self._batch}")
        return b

    def block_tables_tensor(self, batch_size: Optional[int] = None) -> torch.Tensor:
        """[B, capacity_pages] int32 rows of the active sequences (fixed address)."""
        return self.inputs.tables[:self._need(batch_size)]

    def seq_lens_tensor(self, batch_size: Optional[int] = None) -> torch.Tensor:
        return self.inputs.vec["lens"][:self._need(batch_size)]

    def write_slots(self, batch_size: int) -> torch.Tensor:
        """[B] int64 flat slot of each active sequence's decode token (after
        an advance(1)), at a fixed address."""
        if self._chunk_slots is not None:
            raise RuntimeError("the last advance() reserved several tokens; write_slots() "
                               "names the single decode token of an advance(1)")
        return self.inputs.vec["write_slot"][:self._need(batch_size)]

    def _slots_for_write(self, b: int, n: int) -> torch.Tensor:
        """[b, n] flat slots the last advance() reserved."""
        if n == 1 and self._chunk_slots is None:
            return self.inputs.vec["write_slot"][:self._need(b)].view(b, 1)
        if self._chunk_slots is None or self._chunk_slots.shape != (b, n):
            raise RuntimeError(f"advance({n}) for {b} sequences must precede this write")
        return self._chunk_slots


class PagedKVCache(_PagedBase):
    """fp16 paged KV storage (cache/paged_cache.py:63-506), decode side."""

    def __init__(self, spec: KVCacheSpec, block_size: int = 16, num_blocks: Optional[int] = None):
        super().__init__(spec, block_size, num_blocks)
        shape = (self.num_blocks, block_size, spec.num_kv_heads, spec.head_dim)
        self.k_pool = [torch.zeros(shape, dtype=spec.dtype, device=self.device)
                       for _ in range(spec.num_layers)]
        self.v_pool = [torch.zeros(shape, dtype=spec.dtype, device=self.device)
                       for _ in range(spec.num_layers)]
        self.kmin: Optional[List[torch.Tensor]] = None
        self.kmax: Optional[List[torch.Tensor]] = None

    def advance(self, n: int, batch_size: Optional[int] = None,
                slots: Optional[Sequence[int]] = None) -> None:
        """Reserve n more tokens for each active sequence (paged_cache.py:
        235-271) and publish the step's kernel inputs."""
        starts = self._grow(n, batch_size, slots)
        self._publish(n, starts)

    def rewind(self, length: int, slots: Optional[Sequence[int]] = None) -> None:
        """Shorten sequences to `length` tokens, keeping their pages
        (paged_cache.py:273-303): growing again lands on the same slots."""
        seqs = self._active if slots is None else list(slots)
        for s in seqs:
            t = self.tables[s]
            if not 0 <= length <= t.length:
                raise ValueError(f"slot {s} holds {t.length} tokens; cannot rewind it to "
                                 f"{length}")
        for s in seqs:
            self.tables[s].length = length
            if self.kmin is not None and length % self.block_size:
                self._bound_partial_page(s, length)
        self._publish(0, [self.tables[s].length for s in self._active])

    def write(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, start_pos: int = 0) -> None:
        """Store k, v [B, H_kv, n, D] at the slots the last advance(n) reserved."""
        b, h, n, d = k.shape
        flat = self._slots_for_write(b, n).reshape(-1)
        rows_k = k.transpose(1, 2).reshape(b * n, h, d)
        rows_v = v.transpose(1, 2).reshape(b * n, h, d)
        self.k_pool[layer_idx].view(-1, h, d).index_copy_(0, flat, rows_k)
        self.v_pool[layer_idx].view(-1, h, d).index_copy_(0, flat, rows_v)
        if self.kmin is not None:
            from latentserve_amd.kernels.hip import paged_sparse as ps
            if n == 1:
                ps.update_bounds(k[:, :, 0], flat, self.kmin[layer_idx], self.kmax[layer_idx])
            else:
                ps.rebuild_bounds(self.k_pool[layer_idx], self.kmin[layer_idx],
                                  self.kmax[layer_idx])

    def read(self, layer_idx: int, batch_size: int, length: Optional[int] = None):
        """[B, H_kv, L, D] K and V of the active sequences (the gather read,
        paged_cache.py:486-506), on the HIP gather kernel."""
        from latentserve_amd.kernels.hip import paged_gather as pg

        length = self.max_len if length is None else length
        return pg.read(self.k_pool[layer_idx], self.v_pool[layer_idx],
                       self.block_tables_tensor(batch_size), self.seq_lens_tensor(batch_size),
                       length)

    # ---- page bounds for the sparse indexer -------------------------------
    def enable_page_bounds(self) -> None:
        """Per-block per-channel K min / max per layer (paged_cache.py:422-445),
        built from the pools and kept current by every write."""
        if self.kmin is not None:
            return
        nb, _, h, d = self.k_pool[0].shape
        self.kmin = [torch.zeros(nb, h, d, dtype=self.spec.dtype, device=self.device)
                     for _ in self.k_pool]
        self.kmax = [torch.zeros_like(t) for t in self.kmin]
        from latentserve_amd.kernels.hip import paged_sparse as ps
        for layer, pool in enumerate(self.k_pool):
            ps.rebuild_bounds(pool, self.kmin[layer], self.kmax[layer])

    def page_bounds(self, layer_idx: int):
        if self.kmin is None:
            return None
        return self.kmin[layer_idx], self.kmax[layer_idx]

    def _bound_partial_page(self, seq: int, length: int) -> None:
        """Bounds of the page a rewind lands in, over its remaining rows."""
        t = self.tables[seq]
        page, rows = divmod(length, self.block_size)
        blk = t.blocks[page]
        for layer, pool in enumerate(self.k_pool):
            live = pool[blk, :rows]
            self.kmin[layer][blk] = live.amin(dim=0)
            self.kmax[layer][blk] = live.amax(dim=0)
