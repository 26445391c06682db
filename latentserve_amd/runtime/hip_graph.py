"""Decode steps captured in HIP graphs, keyed by (batch, context bucket, ratio).

Mirrors the reference's runtime/cuda_graph.py (GraphUnsupported,
check_capturable, CapturedDecode :123-222, GraphedDecoder :225-388) on the
HIP backend: torch.cuda.CUDAGraph is hipGraph on ROCm.  What a graph
freezes and how each is handled is the reference's design, kept because
the graph semantics force it:

* the cache's host bookkeeping (advance) runs before each replay and writes
  into persistent buffers the graph already points at;
* token ids and positions are copied into static input buffers;
* the block table is held at capacity width and the kernels mask by
  seq_lens, so one graph serves a growing sequence;
* the decode kernel's split count is pinned per graph (its grid is
  captured) -- the kernel re-derives pages per split on the device when a
  sequence outgrows the bucket's split, so a pinned count stays correct;
* RoPE tables are built to the cache capacity before any capture.

On MI355X the runner leans on one property of this build: every HIP entry
point allocates nothing and needs no host synchronisation, and the decode
kernels leave their arrival counters at zero, so a captured step needs no
memset node (which has given wrong results on replays here).
"""

from __future__ import annotations

import time
from collections import Counter
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from latentserve_amd.kernels import fused_elementwise as fe
from latentserve_amd.runtime.kv_cache import PagedKVCache

DEFAULT_BUCKETS = (1024, 2048, 4096, 8192, 16384, 32768)


class GraphUnsupported(RuntimeError):
    """A configuration a graph cannot capture correctly (the serving engine
    falls back to eager)."""


def check_capturable(model) -> None:
    cache = model.cache
    if cache is None:
        raise GraphUnsupported("allocate the cache before capturing")
    if not isinstance(cache, PagedKVCache):
        raise GraphUnsupported("graph capture needs the paged cache")
    if model.rope is None:
        raise GraphUnsupported("graph capture needs RoPE tables")
    if model.device.type != "cuda":
        raise GraphUnsupported(
            f"the model is on {model.device}; a graph records only GPU kernels, so capturing "
            "a CPU model records nothing and every replay is a no-op")


@dataclass
class CapturedDecode:
    """One graph for a fixed (batch size, context bucket)."""

    model: object
    batch_size: int
    bucket_tokens: int
    num_splits: int
    warmup: int = 3
    greedy: bool = False

    static_ids: torch.Tensor = field(init=False)
    static_pos: torch.Tensor = field(init=False)
    static_logits: Optional[torch.Tensor] = field(init=False, default=None)
    static_next: Optional[torch.Tensor] = field(init=False, default=None)
    graph: Optional[torch.cuda.CUDAGraph] = field(init=False, default=None)
    replays: int = field(init=False, default=0)

    def __post_init__(self) -> None:
        dev = self.model.device
        self.static_ids = torch.zeros(self.batch_size, 1, dtype=torch.long, device=dev)
        self.static_pos = torch.zeros(self.batch_size, 1, dtype=torch.long, device=dev)

    def _set_splits(self, value: Optional[int]) -> None:
        for layer in self.model.layers:
            layer.attn.num_splits = value

    def _run(self):
        logits = self.model.decode_forward_static(self.static_ids, self.static_pos,
                                                  max_position=self.bucket_tokens - 1)
        if not self.greedy:
            return logits, None
        return logits, fe.argmax_rows(logits[:, -1, :])

    def load(self, token_ids: torch.Tensor, positions: torch.Tensor) -> None:
        """Copy this step's inputs into the buffers the graph reads."""
        self.static_ids.copy_(token_ids)
        self.static_pos.copy_(positions)

    def capture(self, pool=None) -> None:
        """Record the step (the cache is advanced and load() called with this
        step's real inputs: the K/V write is idempotent, so warm-up and
        capture may run it)."""
        self._set_splits(self.num_splits)
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(self.warmup):
                    self._run()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                self.static_logits, self.static_next = self._run()
            self.graph = graph
        finally:
            self._set_splits(None)

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        self.replays += 1
        return self.static_logits


class GraphedDecoder:
    """Decode steps through captured graphs, eager where none applies.

        logits = decoder.step(token_ids, positions, slots)

    The returned tensor is the graph's static output, overwritten by the
    next replay of the same graph.
    """

    def __init__(self, model, buckets: Sequence[int] = DEFAULT_BUCKETS,
                 num_splits: Optional[dict] = None, enabled: bool = True, greedy: bool = False,
                 policy=None):
        self.model = model
        self.policy = policy
        self.ratio_steps: Counter = Counter()
        self.ratio_tokens: Counter = Counter()
        self.batch_tokens: Counter = Counter()
        self.capture_s = 0.0
        self.num_splits_override = num_splits or {}
        self.enabled = enabled and torch.cuda.is_available() and model.device.type == "cuda"
        self.graphs: dict = {}
        self._last_graph: Optional[CapturedDecode] = None
        self.greedy = greedy
        self.eager_steps = 0
        self.graph_steps = 0
        self.captures = 0
        self._pool = None
        self.last_host_ms = 0.0
        if self.enabled:
            check_capturable(model)
        capacity = model.cache.spec.max_seq_len
        self.buckets = tuple(sorted({b for b in buckets if b < capacity} | {capacity}))
        if model.rope is not None and model.rope.max_seq_len < capacity:
            model.rope._build_tables(capacity)

    def bucket_for(self, length: int) -> Optional[int]:
        for b in self.buckets:
            if length <= b:
                return b
        return None

    def _splits_for(self, batch: int, bucket: int) -> int:
        if (batch, bucket) in self.num_splits_override:
            return self.num_splits_override[(batch, bucket)]
        from latentserve_amd.kernels.gqa.paged_decode import choose_num_splits

        cache = self.model.cache
        return choose_num_splits(batch, cache.spec.num_kv_heads, bucket, cache.block_size,
                                 self.model.device)

    @torch.no_grad()
    def step_greedy(self, token_ids: torch.Tensor, positions: torch.Tensor,
                    slots: Sequence[int]) -> torch.Tensor:
        """The greedy next tokens as a device [B, 1] tensor (the captured
        argmax's output under a graph)."""
        if not self.greedy:
            raise RuntimeError("construct GraphedDecoder(greedy=True) to use step_greedy")
        logits = self.step(token_ids, positions, slots)
        if self._last_graph is not None:
            return self._last_graph.static_next
        return fe.argmax_rows(logits[:, -1, :])

    @torch.no_grad()
    def step(self, token_ids: torch.Tensor, positions: torch.Tensor,
             slots: Sequence[int]) -> torch.Tensor:
        t0 = time.perf_counter()
        self._last_graph = None
        cache = self.model.cache
        cache.advance(1, slots=list(slots))
        batch = len(slots)
        bucket = self.bucket_for(cache.max_len)
        rope_limit = self.model.rope.max_seq_len
        if self.policy is not None:
            mean_ctx = sum(cache.tables[s].length for s in slots) / max(1, batch)
            ratio = self.policy.choose(batch, mean_ctx)
            if ratio != getattr(self.model, "sparse_ratio", None):
                self.model.set_sparse(ratio, recent=self.model.layers[0].attn.sparse_recent)
        else:
            ratio = getattr(self.model, "sparse_ratio", None)
        self.ratio_steps[ratio] += 1
        self.ratio_tokens[ratio] += batch
        self.batch_tokens[(batch, ratio)] += batch

        if not self.enabled or bucket is None or bucket > rope_limit:
            self.eager_steps += 1
            out = self.model.decode_forward_static(token_ids, positions, max_position=cache.max_len)
            self.last_host_ms = (time.perf_counter() - t0) * 1000
            return out

        key = (batch, bucket, ratio)
        graph = self.graphs.get(key)
        if graph is None:
            graph = CapturedDecode(self.model, batch, bucket, self._splits_for(batch, bucket),
                                   greedy=self.greedy)
            graph.load(token_ids, positions)
            cache.sparse_context_hint = bucket
            t_cap = time.perf_counter()
            try:
                graph.capture(pool=self._pool)
            finally:
                cache.sparse_context_hint = None
                self.capture_s += time.perf_counter() - t_cap
            if self._pool is None:
                self._pool = graph.graph.pool()
            self.graphs[key] = graph
            self.captures += 1
        else:
            graph.load(token_ids, positions)
        self.graph_steps += 1
        out = graph.replay()
        self._last_graph = graph
        self.last_host_ms = (time.perf_counter() - t0) * 1000
        return out

    def stats(self) -> dict:
        return {
            "ratio_tokens": {("dense" if k is None else k): v for k, v in self.ratio_tokens.items()},
            "graphs": len(self.graphs),
            "captures": self.captures,
            "graph_steps": self.graph_steps,
            "eager_steps": self.eager_steps,
            "keys": sorted(self.graphs, key=lambda k: (k[0], k[1], -1 if k[2] is None else k[2])),
        }
