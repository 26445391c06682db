"""Paged KV cache bookkeeping: block allocator, block tables, fp16 pools.

Mirrors the reference's cache/block_allocator.py (BlockAllocator, BlockTable,
OutOfBlocks) and cache/paged_cache.py (PagedKVCache) on the decode path the
HIP kernels serve: per-layer pools [num_blocks, 16, H_kv, D], block tables
held at capacity width in persistent device buffers (so one captured graph
serves a growing sequence), `advance()` reserving each step's slots on the
host before the step runs, `write()` scattering the step's K/V, and the read
path and page bounds on the HIP kernels.  Host-side Python, as the
reference's is: the per-step work is a few small host-to-device copies.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterable, Optional, Sequence

import torch


class OutOfBlocks(RuntimeError):
    """The pool cannot satisfy an allocation (cache/block_allocator.py:31-38):
    backpressure for a scheduler, not a crash."""


@dataclass
class BlockAllocator:
    """Fixed pool of equal-sized blocks with a LIFO free list
    (cache/block_allocator.py:41-132): the free list starts descending, so
    the first allocation is block 0, 1, 2, ..., and freed blocks are reused
    most-recent first."""

    num_blocks: int
    block_size: int
    _free: list = field(default_factory=list, init=False)
    _ref_count: dict = field(default_factory=dict, init=False)
    alloc_calls: int = field(default=0, init=False)
    free_calls: int = field(default=0, init=False)
    peak_used: int = field(default=0, init=False)

    def __post_init__(self) -> None:
        if self.num_blocks <= 0 or self.block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self._free = list(range(self.num_blocks - 1, -1, -1))

    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def num_used(self) -> int:
        return self.num_blocks - len(self._free)

    @property
    def utilization(self) -> float:
        return self.num_used / self.num_blocks

    def blocks_for_tokens(self, num_tokens: int) -> int:
        return (num_tokens + self.block_size - 1) // self.block_size

    def allocate(self, num_blocks: int) -> list:
        if num_blocks > self.num_free:
            raise OutOfBlocks(f"requested {num_blocks} blocks, {self.num_free} free "
                              f"({self.num_used}/{self.num_blocks} in use)")
        self.alloc_calls += 1
        out = [self._free.pop() for _ in range(num_blocks)]
        for b in out:
            self._ref_count[b] = 1
        self.peak_used = max(self.peak_used, self.num_used)
        return out

    def incref(self, blocks: Iterable[int]) -> None:
        for b in blocks:
            if b not in self._ref_count:
                raise ValueError(f"block {b} is not allocated")
            self._ref_count[b] += 1

    def free(self, blocks: Iterable[int]) -> None:
        self.free_calls += 1
        for b in blocks:
            count = self._ref_count.get(b)
            if count is None:
                raise ValueError(f"freeing block {b} that is not allocated")
            if count > 1:
                self._ref_count[b] = count - 1
            else:
                del self._ref_count[b]
                self._free.append(b)

    def reset(self) -> None:
        self._free = list(range(self.num_blocks - 1, -1, -1))
        self._ref_count.clear()


@dataclass
class BlockTable:
    """One sequence's logical -> physical map (cache/block_allocator.py:
    180-229): token p lives at flat slot blocks[p // bs] * bs + p % bs."""

    allocator: BlockAllocator
    blocks: list = field(default_factory=list)
    length: int = 0
    version: int = 0

    def append(self, n: int) -> None:
        need = self.allocator.blocks_for_tokens(self.length + n) - len(self.blocks)
        if need > 0:
            self.blocks.extend(self.allocator.allocate(need))
            self.version += 1
        self.length += n

    def slot(self, position: int) -> int:
        if position >= self.length:
            raise IndexError(f"position {position} beyond length {self.length}")
        bs = self.allocator.block_size
        return self.blocks[position // bs] * bs + position % bs

    def slots(self, start: int = 0, end: Optional[int] = None) -> list:
        return [self.slot(p) for p in range(start, self.length if end is None else end)]

    def free(self) -> None:
        self.allocator.free(self.blocks)
        self.blocks = []
        self.length = 0
        self.version += 1


@dataclass
class KVCacheSpec:
    """The reference's KVCacheSpec (cache/kv_cache.py) fields the paged cache
    reads."""

    num_layers: int
    num_kv_heads: int
    head_dim: int
    max_batch_size: int
    max_seq_len: int
    dtype: torch.dtype = torch.float16
    device: str = "cuda"


class PagedKVCache:
    """Block-paged fp16 KV storage (cache/paged_cache.py:63-506), decode path."""

    def __init__(self, spec: KVCacheSpec, block_size: int = 16, num_blocks: Optional[int] = None):
        if block_size != 16:
            raise ValueError("the HIP kernels take 16-token pages")
        self.spec = spec
        self.block_size = block_size
        self.device = torch.device(spec.device)
        if num_blocks is None:
            num_blocks = -(-spec.max_seq_len // block_size) * spec.max_batch_size
        self.num_blocks = num_blocks
        self.allocator = BlockAllocator(num_blocks=num_blocks, block_size=block_size)
        self.tables = [BlockTable(self.allocator) for _ in range(spec.max_batch_size)]
        shape = (num_blocks, block_size, spec.num_kv_heads, spec.head_dim)
        self.k_pool = [torch.zeros(shape, dtype=spec.dtype, device=self.device)
                       for _ in range(spec.num_layers)]
        self.v_pool = [torch.zeros(shape, dtype=spec.dtype, device=self.device)
                       for _ in range(spec.num_layers)]
        self._flat_k = [t.view(-1, spec.num_kv_heads, spec.head_dim) for t in self.k_pool]
        self._flat_v = [t.view(-1, spec.num_kv_heads, spec.head_dim) for t in self.v_pool]
        # Persistent decode buffers at capacity width (graph-address stable).
        self._capacity_pages = -(-spec.max_seq_len // block_size)
        self._block_tables_buf = torch.zeros((spec.max_batch_size, max(1, self._capacity_pages)),
                                             dtype=torch.int32, device=self.device)
        self._seq_lens_buf = torch.zeros(spec.max_batch_size, dtype=torch.int32,
                                         device=self.device)
        self._write_slots_buf = torch.zeros((spec.max_batch_size, 1), dtype=torch.long,
                                            device=self.device)
        self._table_state: list = [None] * spec.max_batch_size
        # Host staging for the per-step copies: pinned and double-buffered,
        # so a step's slots and lengths go up asynchronously while the
        # previous step still runs (a pageable copy would wait for it).
        self._staging = None
        if self.device.type == "cuda":
            mb = spec.max_batch_size
            self._staging = [
                (torch.empty(mb, dtype=torch.long).pin_memory(),
                 torch.empty(mb, dtype=torch.int32).pin_memory(), torch.cuda.Event())
                for _ in range(2)]
            self._stage_i = 0
        self._write_slots: Optional[torch.Tensor] = None
        self._block_tables: Optional[torch.Tensor] = None
        self._seq_lens_tensor: Optional[torch.Tensor] = None
        self._active = list(range(spec.max_batch_size))
        self._bounds_on = False
        # When set (a graph runner's bucket), sparse selection is sized for it.
        self.sparse_context_hint: Optional[int] = None

    # ---- state ----------------------------------------------------------
    @property
    def seq_lens(self) -> list:
        return [self.tables[i].length for i in self._active]

    @property
    def max_len(self) -> int:
        return max((self.tables[i].length for i in self._active), default=0)

    @property
    def active_slots(self) -> list:
        return list(self._active)

    def set_active(self, slots: Sequence[int]) -> None:
        self._active = list(slots)

    def reset(self) -> None:
        for t in self.tables:
            if t.blocks:
                t.free()
        self.allocator.reset()
        self.tables = [BlockTable(self.allocator) for _ in range(self.spec.max_batch_size)]
        self._write_slots = self._block_tables = self._seq_lens_tensor = None
        self._block_tables_buf.zero_()
        self._seq_lens_buf.zero_()
        self._table_state = [None] * self.spec.max_batch_size
        self._active = list(range(self.spec.max_batch_size))

    def free_sequence(self, index: int) -> None:
        self.tables[index].free()

    def can_admit(self, num_tokens: int) -> bool:
        return self.allocator.blocks_for_tokens(num_tokens) <= self.allocator.num_free

    # ---- allocation -----------------------------------------------------
    def advance(self, n: int, batch_size: Optional[int] = None,
                slots: Optional[Sequence[int]] = None) -> None:
        """Reserve n more tokens for each active sequence (paged_cache.py:
        230-271) and refresh the kernel inputs in place."""
        if slots is not None:
            self.set_active(slots)
        elif batch_size is not None:
            self.set_active(range(batch_size))
        active = self._active
        starts = [self.tables[i].length for i in active]
        for i in active:
            self.tables[i].append(n)
        slots_now = [[self.tables[i].slot(p) for p in range(s, s + n)]
                     for i, s in zip(active, starts)]
        b = len(active)
        if n == 1 and self._staging is not None:
            pin_slots, pin_lens, ev = self._next_staging()
            pin_slots[:b] = torch.tensor([s[0] for s in slots_now], dtype=torch.long)
            self._write_slots_buf[:b, 0].copy_(pin_slots[:b], non_blocking=True)
            self._write_slots = self._write_slots_buf[:b]
            self._rebuild_kernel_inputs(pin_lens, ev)
            return
        if n == 1:
            self._write_slots_buf[:b].copy_(torch.tensor(slots_now, dtype=torch.long))
            self._write_slots = self._write_slots_buf[:b]
        else:
            self._write_slots = torch.tensor(slots_now, dtype=torch.long, device=self.device)
        self._rebuild_kernel_inputs()

    def _next_staging(self):
        """The pinned buffers not used by the previous step, once the copies
        that last read them have run."""
        self._stage_i ^= 1
        pin_slots, pin_lens, ev = self._staging[self._stage_i]
        ev.synchronize()
        return pin_slots, pin_lens, ev

    def rewind(self, length: int, slots: Optional[Sequence[int]] = None) -> None:
        """Shorten the active sequences to `length` tokens, keeping their
        blocks (paged_cache.py:273-303)."""
        for i in (self._active if slots is None else slots):
            t = self.tables[i]
            if not 0 <= length <= t.length:
                raise ValueError(f"cannot rewind slot {i} from {t.length} to {length}")
            t.length = length
        self._rebuild_kernel_inputs()

    def _rebuild_kernel_inputs(self, pin_lens: Optional[torch.Tensor] = None,
                               ev: Optional[torch.cuda.Event] = None) -> None:
        active = self._active
        b = len(active)
        for row, i in enumerate(active):
            blocks = self.tables[i].blocks
            state = (i, self.tables[i].version)
            if self._table_state[row] != state:
                if len(blocks) > self._capacity_pages:
                    raise RuntimeError(f"sequence in slot {i} needs {len(blocks)} pages, past "
                                       f"the capacity of {self._capacity_pages}")
                if blocks:
                    self._block_tables_buf[row, :len(blocks)].copy_(
                        torch.tensor(blocks, dtype=torch.int32))
                self._table_state[row] = state
        lens = torch.tensor([self.tables[i].length for i in active], dtype=torch.int32)
        if pin_lens is not None:
            pin_lens[:b] = lens
            self._seq_lens_buf[:b].copy_(pin_lens[:b], non_blocking=True)
            ev.record()
        else:
            self._seq_lens_buf[:b].copy_(lens)
        self._block_tables = self._block_tables_buf[:b]
        self._seq_lens_tensor = self._seq_lens_buf[:b]

    def block_tables_tensor(self, batch_size: Optional[int] = None) -> torch.Tensor:
        if self._block_tables is None:
            raise RuntimeError("call advance() before block_tables_tensor()")
        return self._block_tables if batch_size is None else self._block_tables[:batch_size]

    def seq_lens_tensor(self, batch_size: Optional[int] = None) -> torch.Tensor:
        if self._seq_lens_tensor is None:
            raise RuntimeError("call advance() before seq_lens_tensor()")
        return self._seq_lens_tensor if batch_size is None else self._seq_lens_tensor[:batch_size]

    # ---- read / write ---------------------------------------------------
    def write(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, start_pos: int = 0) -> None:
        """Scatter [B, H_kv, n, D] into the pool at the slots advance() chose."""
        b, h, n, d = k.shape
        slots = self._write_slots
        if slots is None or slots.shape[0] < b or slots.shape[1] != n:
            raise RuntimeError("call advance(n, batch_size) before write()")
        flat = slots[:b].reshape(-1)
        self._flat_k[layer_idx].index_copy_(0, flat, k.permute(0, 2, 1, 3).reshape(-1, h, d))
        self._flat_v[layer_idx].index_copy_(0, flat, v.permute(0, 2, 1, 3).reshape(-1, h, d))
        if self._bounds_on:
            from latentserve_amd.kernels.hip import paged_sparse as ps
            if n == 1:
                ps.update_bounds(k[:, :, 0], flat, self.kmin[layer_idx], self.kmax[layer_idx])
            else:
                self._recompute_bounds(layer_idx)

    def write_slots(self, batch_size: int) -> torch.Tensor:
        """[batch_size] int64 flat slots (block * page + offset) that advance(1)
        chose for the active sequences' new token, on the device, at a fixed
        address (a graph reads them by pointer)."""
        slots = self._write_slots
        if slots is None or slots.shape[0] < batch_size or slots.shape[1] != 1:
            raise RuntimeError("call advance(1, ...) before asking for the write slots")
        return slots[:batch_size].reshape(batch_size)

    def read(self, layer_idx: int, batch_size: int, length: Optional[int] = None):
        """[B, H_kv, L, D] K and V of the active sequences (the gather path,
        paged_cache.py:486-506), on the HIP gather kernel."""
        from latentserve_amd.kernels.hip import paged_gather as pg

        tables = self.block_tables_tensor(batch_size)
        lens = self.seq_lens_tensor(batch_size)
        length = self.max_len if length is None else length
        return pg.read(self.k_pool[layer_idx], self.v_pool[layer_idx], tables, lens, length)

    # ---- page bounds for the sparse indexer -------------------------------
    def enable_page_bounds(self) -> None:
        """Per-block per-channel K min / max per layer (paged_cache.py:422-445)."""
        if self._bounds_on:
            return
        nb, _, h, d = self.k_pool[0].shape
        self.kmin = [torch.zeros(nb, h, d, dtype=self.spec.dtype, device=self.device)
                     for _ in self.k_pool]
        self.kmax = [torch.zeros_like(t) for t in self.kmin]
        self._bounds_on = True
        for layer in range(len(self.k_pool)):
            self._recompute_bounds(layer)

    def page_bounds(self, layer_idx: int):
        if not self._bounds_on:
            return None
        return self.kmin[layer_idx], self.kmax[layer_idx]

    def _recompute_bounds(self, layer_idx: int) -> None:
        """Bounds of every block over all its rows (rebuild_bounds).  Rows a
        sequence has not written yet widen a partial page's bound; the
        decode-step update resets a page on its first token."""
        from latentserve_amd.kernels.hip import paged_sparse as ps
        ps.rebuild_bounds(self.k_pool[layer_idx], self.kmin[layer_idx], self.kmax[layer_idx])
