"""INT8 paged KV cache for the HIP decode path.

The reference's Int8PagedKVCache (cache/int8_paged_cache.py:143-758) fixes
the storage the INT8 kernel reads, and this class keeps it:

* K and V pools ``[num_blocks, 16, H_kv, D]`` int8; K one fp32 step per
  (block, head, channel) (``k_scale_pool [nb, H_kv, D]``), V one per
  (block, token, head) (``v_scale_pool [nb, 16, H_kv]``); zero points of
  the same shapes when asymmetric (codes shifted by 2^(bits-1), the shift
  folded into the zero point, :191-214).
* A K step covers a whole page, so a page's K can only be quantized once
  the page is full.  Each sequence's LAST page of K is kept exact in an
  fp16 residual row ``residual(layer) [max_batch, 16, H_kv, D]`` (row =
  the sequence's slot), and the kernel reads that page's K from there
  (``k_residual`` / ``res_rows``); every earlier page is in the pool
  (:283-298).  V's scale is per token, so V is quantized as it is written.

How the invariant is kept is this build's own design, one rule for every
write: a page is quantized into the pool exactly when it stops being its
sequence's last page.

* ``advance(n)`` first quantizes, in every layer, each active sequence's
  last page if it is full (the write about to happen starts a new page),
  from the residual, with ``ls_int8_finalize_blocks``; then it reserves the
  tokens and publishes the step's inputs (tables, lengths, the decode
  token's V slot, its residual index ``slot * 16 + offset``, residual rows).
  It runs outside any captured graph, so a graphed decode step only ever
  writes at fixed indices: that is what makes the INT8 step capturable
  (the reference's deferred finalize, :514-580).
* ``write`` of one token (decode) is one ``ls_int8_decode_write`` launch:
  V quantized into the pool, K into the residual row.
* ``write`` of n > 1 tokens (a prefill chunk) quantizes V the same way; K
  is assembled page by page (the residual's rows for a page the chunk
  continues), the pages that are complete and not last are quantized into
  the pool in one launch, and the new last page goes to the residual.

Quantization runs on the HIP kernels only (bit-exact with the reference's
torch ops, tests/test_gpu_int8_write.py); there is no CPU path.
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import torch

from latentserve_amd.runtime.kv_cache import KVCacheSpec, _PagedBase

EPS = 1e-8


class Int8PagedKVCache(_PagedBase):
    """INT8 paged KV storage with the fp16 last-page K residual."""

    def __init__(self, spec: KVCacheSpec, block_size: int = 16, num_blocks: Optional[int] = None,
                 k_bits: int = 8, v_bits: int = 8, asymmetric: bool = False,
                 exact_division: bool = False):
        super().__init__(spec, block_size, num_blocks)
        for bits in (k_bits, v_bits):
            if not 2 <= bits <= 8:
                raise ValueError(f"bit widths must be in [2, 8] (an int8 pool), got {bits}")
        self.asymmetric = bool(asymmetric)
        # (eps, qmax, levels, offset) of K and V: symmetric codes lie in
        # [-qmax, qmax]; asymmetric in [0, levels] shifted down by offset
        self.k_quant = (EPS, float(2 ** (k_bits - 1) - 1), float(2 ** k_bits - 1),
                        float(2 ** (k_bits - 1)))
        self.v_quant = (EPS, float(2 ** (v_bits - 1) - 1), float(2 ** v_bits - 1),
                        float(2 ** (v_bits - 1)))
        self.exact_division = exact_division
        nb, bs, h, d = self.num_blocks, block_size, spec.num_kv_heads, spec.head_dim
        dev = self.device

        def per_layer(make):
            return [make() for _ in range(spec.num_layers)]

        self.k_pool = per_layer(lambda: torch.zeros(nb, bs, h, d, dtype=torch.int8, device=dev))
        self.v_pool = per_layer(lambda: torch.zeros(nb, bs, h, d, dtype=torch.int8, device=dev))
        self.k_scale_pool = per_layer(lambda: torch.ones(nb, h, d, dtype=torch.float32,
                                                         device=dev))
        self.v_scale_pool = per_layer(lambda: torch.ones(nb, bs, h, dtype=torch.float32,
                                                         device=dev))
        self.k_zero_pool = per_layer(lambda: torch.zeros(nb, h, d, dtype=torch.float32,
                                                         device=dev)) if asymmetric else []
        self.v_zero_pool = per_layer(lambda: torch.zeros(nb, bs, h, dtype=torch.float32,
                                                         device=dev)) if asymmetric else []
        self._residual = per_layer(lambda: torch.zeros(spec.max_batch_size, bs, h, d,
                                                       dtype=spec.dtype, device=dev))
        # pages of each slot's sequence whose K is in the pool, per layer
        self._pooled: List[List[int]] = [[0] * spec.max_batch_size
                                         for _ in range(spec.num_layers)]
        self._starts: List[int] = []

    # ---- API of the reference cache ----------------------------------------
    def enable_deferred_finalize(self) -> None:
        """A page is always quantized when it stops being the last page
        (in advance()); kept so callers of the reference's API work."""

    def residual(self, layer_idx: int) -> torch.Tensor:
        """[max_batch, 16, H_kv, D] fp16: each slot's last page of K."""
        return self._residual[layer_idx]

    def residual_rows_tensor(self, batch_size: Optional[int] = None) -> torch.Tensor:
        """[B] int32 residual row (= slot) of each active sequence."""
        return self.inputs.vec["res_row"][:self._need(batch_size)]

    def pooled_pages(self, slot: int) -> int:
        """Pages of slot's sequence whose K is quantized in every layer."""
        return min(layer[slot] for layer in self._pooled)

    def free_sequence(self, index: int) -> None:
        super().free_sequence(index)
        for layer in self._pooled:
            layer[index] = 0

    def shareable_blocks(self, index: int) -> int:
        """Full pages whose K is quantized in the pool in every layer (a full
        last page still has its K only in this slot's residual:
        cache/int8_paged_cache.py:385-396)."""
        return min(super().shareable_blocks(index), self.pooled_pages(index))

    def attach_prefix(self, index: int, blocks: Sequence[int], num_tokens: int) -> None:
        """As the fp16 cache; the attached pages are quantized (a prefix cache
        only records shareable pages), so the slot's residual starts empty:
        its next token opens a new page (cache/int8_paged_cache.py:398-413)."""
        super().attach_prefix(index, blocks, num_tokens)
        for layer in self._pooled:
            layer[index] = len(blocks)

    def reset(self) -> None:
        super().reset()
        for layer in self._pooled:
            layer[:] = [0] * len(layer)
        for r in self._residual:
            r.zero_()

    # ---- steps ----------------------------------------------------------------
    def advance(self, n: int, batch_size: Optional[int] = None,
                slots: Optional[Sequence[int]] = None) -> None:
        if slots is not None:
            self.set_active(slots)
        elif batch_size is not None:
            self.set_active(range(batch_size))
        if n > 0:
            self._pool_full_last_pages(self._active)
        starts = self._grow(n, None, None)
        self._starts = starts
        bs = self.block_size
        extra = {"res_row": list(self._active)}
        if n == 1:
            extra["res_index"] = [s * bs + p % bs for s, p in zip(self._active, starts)]
        self._publish(n, starts, extra)

    def _pool_full_last_pages(self, seqs: Sequence[int]) -> None:
        """Quantize each sequence's full last page from the residual (it is
        about to stop being the last page), in every layer where it is not
        pooled yet."""
        bs = self.block_size
        for li in range(self.spec.num_layers):
            rows, ids = [], []
            for s in seqs:
                t = self.tables[s]
                if t.length == 0 or t.length % bs:
                    continue
                page = t.length // bs - 1
                if self._pooled[li][s] > page:
                    continue
                if self._pooled[li][s] < page:
                    raise RuntimeError(f"slot {s}, layer {li}: pages {self._pooled[li][s]}.."
                                       f"{page - 1} were never quantized (a write was skipped)")
                rows.append(s)
                ids.append(t.blocks[page])
                self._pooled[li][s] = page + 1
            if rows:
                idx = torch.tensor(rows, dtype=torch.long, device=self.device)
                self._quantize_k(li, self._residual[li].index_select(0, idx),
                                 torch.tensor(ids, dtype=torch.long, device=self.device))

    def _quantize_k(self, layer: int, data: torch.Tensor, ids: torch.Tensor) -> None:
        from latentserve_amd.kernels.hip import int8_write as iw

        eps, qmax, levels, offset = self.k_quant
        iw.finalize_blocks(data, ids, self.k_pool[layer], self.k_scale_pool[layer],
                           self.k_zero_pool[layer] if self.asymmetric else None,
                           asym=self.asymmetric, eps=eps, qmax=qmax, levels=levels,
                           offset=offset, exact_division=self.exact_division)

    def _quantize_v_and_residual(self, layer: int, k_rows: torch.Tensor, v_rows: torch.Tensor,
                                 slots: torch.Tensor, res_index: torch.Tensor) -> None:
        """V rows quantized into the pool at flat `slots`; K rows copied to
        the flattened residual at `res_index` (-1: not copied)."""
        from latentserve_amd.kernels.hip import int8_write as iw

        h, d = self.spec.num_kv_heads, self.spec.head_dim
        eps, qmax, levels, offset = self.v_quant
        iw.decode_write(k_rows, v_rows, slots, res_index, self.v_pool[layer].view(-1, h, d),
                        self.v_scale_pool[layer].view(-1, h),
                        self.v_zero_pool[layer].view(-1, h) if self.asymmetric else None,
                        self._residual[layer].view(-1, h, d), asym=self.asymmetric, eps=eps,
                        qmax=qmax, levels=levels, offset=offset,
                        exact_division=self.exact_division)

    def write(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, start_pos: int = 0) -> None:
        """Store k, v [B, H_kv, n, D] fp16 at the tokens the last advance(n)
        reserved."""
        b, h, n, d = k.shape
        if not k.is_cuda:
            raise ValueError("the INT8 cache quantizes on the HIP kernels: k and v must be on "
                             "a GPU")
        slots = self._slots_for_write(b, n)
        if n == 1:
            self._quantize_v_and_residual(layer_idx, k, v, slots.view(b),
                                          self.inputs.vec["res_index"][:b])
            return
        # V of every token, no K copy
        k_tok = k.transpose(1, 2).reshape(b * n, h, 1, d)
        v_tok = v.transpose(1, 2).reshape(b * n, h, 1, d)
        skip = torch.full((b * n,), -1, dtype=torch.long, device=k.device)
        self._quantize_v_and_residual(layer_idx, k_tok, v_tok, slots.reshape(-1), skip)
        # K page by page
        bs = self.block_size
        res = self._residual[layer_idx]
        full_data, full_ids = [], []
        for row, s in enumerate(self._active[:b]):
            start = self._starts[row]
            first_page, off = divmod(start, bs)
            end = start + n
            last_page = (end - 1) // bs
            pages = last_page - first_page + 1
            stage = torch.zeros(pages * bs, h, d, dtype=k.dtype, device=k.device)
            if off:
                stage[:off] = res[s, :off]
            stage[off:off + n] = k[row].transpose(0, 1)
            stage = stage.view(pages, bs, h, d)
            blocks = self.tables[s].blocks
            if pages > 1:
                full_data.append(stage[:pages - 1])
                full_ids.extend(blocks[first_page:last_page])
            res[s] = stage[pages - 1]
            self._pooled[layer_idx][s] = last_page
        if full_ids:
            self._quantize_k(layer_idx, torch.cat(full_data),
                             torch.tensor(full_ids, dtype=torch.long, device=k.device))
