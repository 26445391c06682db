"""Decode steps replayed from HIP graphs (the role of the reference's
runtime/cuda_graph.py: GraphUnsupported, check_capturable, CapturedDecode,
GraphedDecoder).

What a replay may rely on, and how this runner provides it:

* Addresses, not values, are frozen.  Every tensor a step reads lives at a
  fixed address: the caches publish tables, lengths and write slots into
  their ``StepInputs`` buffers (kv_cache.py) in ``advance()``, which the
  runner calls before every replay; token ids and positions are copied into
  the graph's own input buffers; RoPE tables are built to the cache's
  capacity before the first capture; the decode kernels' split workspaces
  are persistent per shape.
* Shapes are frozen.  A graph serves one (batch size, context bucket,
  sparse ratio); tables are held at capacity width and the kernels mask by
  length, so one graph serves a sequence as it grows through its bucket.
  The split count is pinned per graph (the kernels re-derive each split's
  pages on the device).
* Nothing in a step allocates, synchronises with the host or needs a
  memset node (the HIP entry points leave their counters at zero).  The
  INT8 cache quantizes a page only in ``advance()`` (outside the graph);
  inside, its decode write goes to fixed indices, so capture and warm-up
  may run the step (writing the same values to the same places).
* A step the runner cannot replay (no bucket covers the length, graphs
  disabled, a model on the CPU) runs eagerly; ``GraphUnsupported`` marks a
  configuration that can never be captured.
"""

from __future__ import annotations

import contextlib
import time
from collections import Counter
from typing import Dict, Optional, Sequence, Tuple

import torch

from latentserve_amd.kernels import fused_elementwise as fe

DEFAULT_BUCKETS = (1024, 2048, 4096, 8192, 16384, 32768)


class GraphUnsupported(RuntimeError):
    """A configuration no graph can capture correctly; callers fall back to
    eager steps."""


def check_capturable(model) -> None:
    """Raise GraphUnsupported unless the model's decode step is capturable."""
    from latentserve_amd.runtime.int8_cache import Int8PagedKVCache
    from latentserve_amd.runtime.kv_cache import PagedKVCache

    if model.cache is None:
        raise GraphUnsupported("no cache: allocate it before capturing")
    if not isinstance(model.cache, (PagedKVCache, Int8PagedKVCache)):
        raise GraphUnsupported(f"{type(model.cache).__name__} has no fixed-address step "
                               "inputs; only the paged caches can be captured")
    if model.rope is None:
        raise GraphUnsupported("RoPE tables must exist (and cover the capacity) before capture")
    if model.device.type != "cuda":
        raise GraphUnsupported(f"a graph records GPU work only; the model is on {model.device}")


@contextlib.contextmanager
def _pinned_splits(model, splits: Optional[int]):
    """Every layer's decode split count set to `splits` for the duration."""
    saved = [layer.attn.num_splits for layer in model.layers]
    for layer in model.layers:
        layer.attn.num_splits = splits
    try:
        yield
    finally:
        for layer, s in zip(model.layers, saved):
            layer.attn.num_splits = s


class CapturedDecode:
    """One recorded decode step for a fixed (batch, bucket, ratio)."""

    WARMUP_RUNS = 2

    def __init__(self, model, batch_size: int, bucket_tokens: int, num_splits: int,
                 greedy: bool = False):
        self.model = model
        self.batch_size = batch_size
        self.bucket_tokens = bucket_tokens
        self.num_splits = num_splits
        self.greedy = greedy
        dev = model.device
        self.ids = torch.zeros(batch_size, 1, dtype=torch.long, device=dev)
        self.positions = torch.zeros(batch_size, 1, dtype=torch.long, device=dev)
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.logits_buf: Optional[torch.Tensor] = None
        self.next_buf: Optional[torch.Tensor] = None
        self.replays = 0

    def _forward(self):
        logits = self.model.decode_forward_static(self.ids, self.positions,
                                                  max_position=self.bucket_tokens - 1)
        nxt = fe.argmax_rows(logits[:, -1, :]) if self.greedy else None
        return logits, nxt

    def set_inputs(self, token_ids: torch.Tensor, positions: torch.Tensor) -> None:
        self.ids.copy_(token_ids)
        self.positions.copy_(positions)

    def record(self, pool=None) -> None:
        """Warm up on a side stream, then capture one step (the inputs set
        and the cache advanced for a real step: the recording does not run,
        the first replay does)."""
        with _pinned_splits(self.model, self.num_splits):
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(self.WARMUP_RUNS):
                    self._forward()
            torch.cuda.current_stream().wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self.logits_buf, self.next_buf = self._forward()
        self.graph = g

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        self.replays += 1
        return self.logits_buf


class GraphedDecoder:
    """Decode steps through bucketed graphs:

        logits = runner.step(token_ids, positions, slots)

    `slots` names the cache rows (sequences) of this step; the cache is
    advanced by one token for each.  The returned logits of a graphed step
    are the graph's static buffer, valid until that graph's next replay.
    """

    def __init__(self, model, buckets: Sequence[int] = DEFAULT_BUCKETS,
                 num_splits: Optional[Dict[Tuple[int, int], int]] = None,
                 enabled: bool = True, greedy: bool = False, policy=None):
        self.model = model
        self.greedy = greedy
        self.policy = policy
        self.split_overrides = dict(num_splits or {})
        self.enabled = bool(enabled) and torch.cuda.is_available() \
            and model.device.type == "cuda"
        if self.enabled:
            check_capturable(model)
        cap = model.cache.spec.max_seq_len
        # the capacity closes the list, so every reachable length has a bucket
        self.buckets = tuple(sorted({int(b) for b in buckets if b < cap} | {cap}))
        if model.rope is not None and model.rope.max_seq_len < cap:
            model.rope._build_tables(cap)         # never rebuilt (reallocated) after a capture
        self.graphs: Dict[tuple, CapturedDecode] = {}
        self._pool = None
        self._last_graph: Optional[CapturedDecode] = None
        self._tokens_by_ratio: Counter = Counter()
        self.graph_steps = self.eager_steps = self.captures = 0
        self.capture_seconds = 0.0
        self.last_host_ms = 0.0

    def bucket_for(self, length: int) -> Optional[int]:
        """The smallest bucket holding `length` tokens (None: past capacity)."""
        return next((b for b in self.buckets if length <= b), None)

    def _splits(self, batch: int, bucket: int) -> int:
        if (batch, bucket) in self.split_overrides:
            return self.split_overrides[(batch, bucket)]
        from latentserve_amd.kernels.gqa.paged_decode import choose_num_splits

        c = self.model.cache
        return choose_num_splits(batch, c.spec.num_kv_heads, bucket, c.block_size,
                                 self.model.device, int8=c.k_pool[0].dtype == torch.int8)

    def _ratio_for_step(self, slots: Sequence[int]) -> Optional[float]:
        """The sparse ratio of this step: the policy's choice at the batch's
        mean context (applied to the model), else the model's own."""
        model = self.model
        if self.policy is None:
            return getattr(model, "sparse_ratio", None)
        lens = [model.cache.tables[s].length for s in slots]
        ratio = self.policy.choose(len(slots), sum(lens) / max(1, len(lens)))
        if ratio != getattr(model, "sparse_ratio", None):
            model.set_sparse(ratio, recent=model.layers[0].attn.sparse_recent)
        return ratio

    @torch.no_grad()
    def step(self, token_ids: torch.Tensor, positions: torch.Tensor,
             slots: Sequence[int]) -> torch.Tensor:
        t0 = time.perf_counter()
        self._last_graph = None
        cache = self.model.cache
        cache.advance(1, slots=list(slots))
        batch = len(slots)
        ratio = self._ratio_for_step(slots)
        self._tokens_by_ratio[ratio] += batch
        bucket = self.bucket_for(cache.max_len)
        if not self.enabled or bucket is None or bucket > self.model.rope.max_seq_len:
            self.eager_steps += 1
            out = self.model.decode_forward_static(token_ids, positions,
                                                   max_position=cache.max_len)
            self.last_host_ms = (time.perf_counter() - t0) * 1e3
            return out
        key = (batch, bucket, ratio)
        g = self.graphs.get(key)
        if g is None:
            g = CapturedDecode(self.model, batch, bucket, self._splits(batch, bucket),
                               greedy=self.greedy)
            g.set_inputs(token_ids, positions)
            t_cap = time.perf_counter()
            cache.sparse_context_hint = bucket      # selection sized for the bucket's top
            try:
                g.record(self._pool)
            finally:
                cache.sparse_context_hint = None
                self.capture_seconds += time.perf_counter() - t_cap
            self._pool = self._pool or g.graph.pool()
            self.graphs[key] = g
            self.captures += 1
        else:
            g.set_inputs(token_ids, positions)
        out = g.replay()
        self.graph_steps += 1
        self._last_graph = g
        self.last_host_ms = (time.perf_counter() - t0) * 1e3
        return out

    @torch.no_grad()
    def step_greedy(self, token_ids: torch.Tensor, positions: torch.Tensor,
                    slots: Sequence[int]) -> torch.Tensor:
        """The next tokens [B, 1] (int64, on the device): under a graph the
        captured argmax's buffer, fit to feed back as the next token_ids."""
        if not self.greedy:
            raise RuntimeError("greedy steps need GraphedDecoder(..., greedy=True)")
        logits = self.step(token_ids, positions, slots)
        if self._last_graph is not None:
            return self._last_graph.next_buf
        return fe.argmax_rows(logits[:, -1, :])

    def stats(self) -> dict:
        def order(k):
            return (k[0], k[1], -1.0 if k[2] is None else k[2])

        return {
            "ratio_tokens": {("dense" if r is None else r): n
                             for r, n in self._tokens_by_ratio.items()},
            "graphs": len(self.graphs),
            "captures": self.captures,
            "graph_steps": self.graph_steps,
            "eager_steps": self.eager_steps,
            "keys": sorted(self.graphs, key=order),
        }
