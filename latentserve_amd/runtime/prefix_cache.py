"""Prefix sharing: whole pages of a prompt prefix written once, reused.

Behaviour of the reference's cache/prefix_cache.py:39-137 (chained page
keys, verified matches, the cache's own reference on every recorded page,
least-recently-used eviction through the allocator's reclaim hooks, an O(1)
count of the pages only the cache holds); the design here is this build's:

* A page's key is a 16-byte BLAKE2b digest of its parent page's key and its
  tokens (as little-endian int64), so equal tokens after different prefixes
  get different keys and keys are stable across processes.  A match still
  compares the stored parent key and tokens, so even a digest collision can
  never hand out a page with other contents.
* ``entry[block] = (key, parent_key, tokens)``; ``by_key[key] = block``; an
  ``OrderedDict`` keeps the recorded pages oldest-used first.
* The allocator reports every reference-count change; a recorded page
  going from two holders to one (the last sequence let go) becomes
  reclaimable, from one to two it is in use again.  The page is recorded
  only after the cache's own reference is taken, and forgotten before that
  reference is dropped, so those two changes are never counted.
"""

from __future__ import annotations

import hashlib
from collections import OrderedDict
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from latentserve_amd.runtime.kv_cache import BlockAllocator

Key = bytes
Entry = Tuple[Key, Optional[Key], Tuple[int, ...]]


def _page_key(parent: Optional[Key], tokens: Sequence[int]) -> Key:
    h = hashlib.blake2b(digest_size=16)
    h.update(parent if parent is not None else b"\0" * 16)
    h.update(np.asarray(tokens, dtype="<i8").tobytes())
    return h.digest()


def block_keys(tokens: Sequence[int], block_size: int,
               num_blocks: Optional[int] = None) -> List[Entry]:
    """(key, parent key, tokens) of each full page of `tokens` (the first
    `num_blocks` of them when given), each key covering every token before
    its page's end."""
    count = len(tokens) // block_size if num_blocks is None else int(num_blocks)
    out: List[Entry] = []
    parent: Optional[Key] = None
    for i in range(count):
        page = tuple(int(t) for t in tokens[i * block_size:(i + 1) * block_size])
        key = _page_key(parent, page)
        out.append((key, parent, page))
        parent = key
    return out


class PrefixCache:
    """Pages of finished or running sequences, findable by their prefix."""

    def __init__(self, allocator: BlockAllocator, block_size: int):
        if block_size != allocator.block_size:
            raise ValueError(f"pages of {block_size} tokens in a pool of "
                             f"{allocator.block_size}-token blocks")
        self.allocator = allocator
        self.block_size = int(block_size)
        self.by_key: Dict[Key, int] = {}
        self.entry: Dict[int, Entry] = {}
        self.lru: "OrderedDict[int, None]" = OrderedDict()
        self.hits = 0
        self.lookups = 0
        self.evictions = 0
        self.peak_live = 0          # pages held by sequences (cache-only ones excluded)
        self._alone = 0             # recorded pages no sequence holds
        allocator.reclaimer = self.reclaim
        allocator.reclaimable = self.num_reclaimable
        allocator.on_ref_change = self._count_change

    # ---- the allocator's hooks -------------------------------------------
    def _count_change(self, block: int, old: int, new: int) -> None:
        live = self.allocator.num_used - self._alone
        self.peak_live = max(self.peak_live, live)
        if block in self.entry:
            if (old, new) == (2, 1):
                self._alone += 1
            elif (old, new) == (1, 2):
                self._alone -= 1

    def num_reclaimable(self) -> int:
        return self._alone

    def count_reclaimable_by_scan(self) -> int:
        """The definition of num_reclaimable(), by scanning (for tests)."""
        return sum(self.allocator.ref_count(b) == 1 for b in self.entry)

    # ---- lookup ----------------------------------------------------------
    def match(self, tokens: Sequence[int]) -> List[int]:
        """Recorded pages holding the longest prefix of `tokens`, whole
        pages, never the page of the last token (whose logits a prefill must
        still produce)."""
        usable = (len(tokens) - 1) // self.block_size
        found: List[int] = []
        for key, parent, page in block_keys(tokens, self.block_size, max(usable, 0)):
            blk = self.by_key.get(key)
            if blk is None:
                break
            _, stored_parent, stored_page = self.entry[blk]
            if stored_parent != parent or stored_page != page:
                break
            found.append(blk)
        self.lookups += 1
        if found:
            self.hits += 1
        for blk in found:
            self.lru.move_to_end(blk)
        return found

    # ---- recording -------------------------------------------------------
    def register(self, tokens: Sequence[int], blocks: Sequence[int]) -> int:
        """Record the full pages of a sequence whose tokens `tokens` are
        written in `blocks` (in order); pages already recorded stay as they
        are.  Returns how many pages were added."""
        added = 0
        for (key, parent, page), blk in zip(block_keys(tokens, self.block_size), blocks):
            held = self.by_key.get(key)
            if held is not None:
                if held == blk:
                    self.lru.move_to_end(blk)
                continue
            if blk in self.entry:
                continue                      # this page is recorded under another key
            self.allocator.incref([blk])      # the cache's reference first, then the entry
            self.by_key[key] = blk
            self.entry[blk] = (key, parent, page)
            self.lru[blk] = None
            added += 1
        return added

    # ---- eviction --------------------------------------------------------
    def reclaim(self, count: int) -> int:
        """Give back up to `count` pages only the cache holds, least recently
        used first.  Returns how many went back to the pool."""
        victims = []
        for blk in self.lru:
            if len(victims) >= count:
                break
            if self.allocator.ref_count(blk) == 1:
                victims.append(blk)
        for blk in victims:
            key = self.entry.pop(blk)[0]      # forgotten first, then the reference dropped
            del self.by_key[key]
            del self.lru[blk]
            self._alone -= 1
            self.allocator.free([blk])
            self.evictions += 1
        return len(victims)

    def stats(self) -> dict:
        return {"cached_blocks": len(self.entry), "reclaimable": self._alone,
                "peak_live": self.peak_live, "lookups": self.lookups, "hits": self.hits,
                "evictions": self.evictions}
