"""A Qwen2.5-1.5B-geometry decoder for the graph runner and the full-step
benchmark: random-init fp16 weights, the paged cache, and the HIP paged
decode attention in every layer.

The reference's model/ stack (model/qwen.py, model/attention/gqa.py) is not
rebuilt: this is the minimum that gives the decode-attention path its real
surroundings (28 layers, hidden 1536, 12 query / 2 KV heads, MLP 8960,
vocab 151936, tied embeddings, RoPE theta 1e6, q/k/v biases) so a captured
decode step can be timed as BASELINE's configuration 5 asks.  GEMMs and the
elementwise glue are torch ops (hipBLASLt); the attention is the HIP kernel
behind the reference's own entry point, reached as GQAAttention.forward's
decode branch reaches it (model/attention/gqa.py:283-344: q [B, 12, 1, D]
folded to [B, 2, 6, D], the new K/V written first, then attention over the
pool).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

from latentserve_amd.kernels.gqa import paged_decode as pd
from latentserve_amd.runtime.kv_cache import KVCacheSpec, PagedKVCache


@dataclass
class DecoderConfig:
    """Qwen/Qwen2.5-1.5B-Instruct's geometry."""

    vocab_size: int = 151936
    hidden_size: int = 1536
    intermediate_size: int = 8960
    num_layers: int = 28
    num_heads: int = 12
    num_kv_heads: int = 2
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = True


class Rope:
    """cos / sin tables to a fixed bound (no rebuild inside a graph)."""

    def __init__(self, head_dim: int, theta: float, max_seq_len: int, device):
        self.head_dim, self.theta, self.device = head_dim, theta, device
        self.max_seq_len = 0
        self._build_tables(max_seq_len)

    def _build_tables(self, n: int) -> None:
        inv = 1.0 / (self.theta ** (torch.arange(0, self.head_dim, 2, dtype=torch.float64)
                                    / self.head_dim))
        t = torch.arange(n, dtype=torch.float64)
        freqs = torch.outer(t, inv)
        emb = torch.cat([freqs, freqs], dim=-1)
        self.cos = emb.cos().to(torch.float32).to(self.device)
        self.sin = emb.sin().to(torch.float32).to(self.device)
        self.max_seq_len = n

    def apply(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """x [B, n_heads, 1, D] fp16, pos [B, 1] int64 -> rotated, fp16."""
        cos = self.cos[pos][:, None]          # [B, 1, 1, D]
        sin = self.sin[pos][:, None]
        xf = x.float()
        half = self.head_dim // 2
        rot = torch.cat([-xf[..., half:], xf[..., :half]], dim=-1)
        return (xf * cos + rot * sin).to(x.dtype)


class _Attn:
    def __init__(self):
        self.num_splits: Optional[int] = None
        self.sparse_recent = 2


class _Layer:
    def __init__(self, cfg: DecoderConfig, gen: torch.Generator, device, std: float):
        h, kvd = cfg.hidden_size, cfg.num_kv_heads * cfg.head_dim
        qd = cfg.num_heads * cfg.head_dim

        def w(*shape):
            return (torch.randn(*shape, generator=gen, device=device, dtype=torch.float32)
                    * std).to(torch.float16)

        self.attn = _Attn()
        self.w_qkv = w(qd + 2 * kvd, h)
        self.b_qkv = w(qd + 2 * kvd)
        self.w_o = w(h, qd)
        self.w_gate_up = w(2 * cfg.intermediate_size, h)
        self.w_down = w(h, cfg.intermediate_size)
        self.norm1 = torch.ones(h, dtype=torch.float16, device=device)
        self.norm2 = torch.ones(h, dtype=torch.float16, device=device)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w


class QwenDecoder:
    """Decode-only model over a PagedKVCache; random weights, fixed seed."""

    def __init__(self, cfg: DecoderConfig = DecoderConfig(), device="cuda", seed: int = 0,
                 std: float = 0.02):
        self.cfg = cfg
        self.device = torch.device(device)
        gen = torch.Generator(device=self.device).manual_seed(seed)
        self.embed = (torch.randn(cfg.vocab_size, cfg.hidden_size, generator=gen,
                                  device=self.device) * std).to(torch.float16)
        self.layers = [_Layer(cfg, gen, self.device, std) for _ in range(cfg.num_layers)]
        self.norm = torch.ones(cfg.hidden_size, dtype=torch.float16, device=self.device)
        self.lm_head = self.embed if cfg.tie_word_embeddings else (
            torch.randn(cfg.vocab_size, cfg.hidden_size, generator=gen, device=self.device)
            * std).to(torch.float16)
        self.cache: Optional[PagedKVCache] = None
        self.rope: Optional[Rope] = None
        self.sparse_ratio: Optional[float] = None
        self.scale = 1.0 / math.sqrt(cfg.head_dim)

    def allocate_cache(self, max_batch_size: int, max_seq_len: int,
                       num_blocks: Optional[int] = None) -> PagedKVCache:
        spec = KVCacheSpec(num_layers=self.cfg.num_layers, num_kv_heads=self.cfg.num_kv_heads,
                           head_dim=self.cfg.head_dim, max_batch_size=max_batch_size,
                           max_seq_len=max_seq_len, device=str(self.device))
        self.cache = PagedKVCache(spec, num_blocks=num_blocks)
        self.rope = Rope(self.cfg.head_dim, self.cfg.rope_theta, max_seq_len, self.device)
        return self.cache

    def set_sparse(self, ratio: Optional[float], recent: int = 2) -> None:
        """Sparse decode attention over a page budget (None: dense)."""
        if ratio is not None:
            self.cache.enable_page_bounds()
        self.sparse_ratio = ratio
        for layer in self.layers:
            layer.attn.sparse_recent = recent

    @torch.no_grad()
    def decode_forward_static(self, token_ids: torch.Tensor, positions: torch.Tensor,
                              max_position: int) -> torch.Tensor:
        """One decode step for the active sequences: token_ids / positions
        [B, 1] int64 -> logits [B, 1, vocab].  The cache has already been
        advanced; `max_position` bounds every position (a graph bucket)."""
        cfg, cache = self.cfg, self.cache
        b = token_ids.shape[0]
        qd, kvd, hd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim, cfg.head_dim
        n_rep = cfg.num_heads // cfg.num_kv_heads
        tables = cache.block_tables_tensor(b)
        lens = cache.seq_lens_tensor(b)
        x = F.embedding(token_ids, self.embed)                     # [B, 1, hidden]
        for li, layer in enumerate(self.layers):
            h = rms_norm(x, layer.norm1, cfg.rms_norm_eps)
            qkv = F.linear(h, layer.w_qkv, layer.b_qkv)            # [B, 1, qd + 2 kvd]
            q = qkv[..., :qd].view(b, 1, cfg.num_heads, hd).transpose(1, 2)
            k = qkv[..., qd:qd + kvd].view(b, 1, cfg.num_kv_heads, hd).transpose(1, 2)
            v = qkv[..., qd + kvd:].view(b, 1, cfg.num_kv_heads, hd).transpose(1, 2)
            q = self.rope.apply(q, positions)
            k = self.rope.apply(k, positions)
            cache.write(li, k, v)
            qg = q.reshape(b, cfg.num_kv_heads, n_rep, hd)          # query head i -> kv head i // 6
            if self.sparse_ratio is None:
                o = pd.paged_decode_attention(qg, cache.k_pool[li], cache.v_pool[li], tables, lens,
                                              num_splits=layer.attn.num_splits,
                                              softmax_scale=self.scale,
                                              max_seq_len=max_position + 1)
            else:
                from latentserve_amd.kernels.hip import paged_sparse as ps
                kmin, kmax = cache.page_bounds(li)
                ctx = cache.sparse_context_hint or max_position + 1
                o = ps.sparse_attention(qg, cache.k_pool[li], cache.v_pool[li], tables, lens,
                                        kmin, kmax, ratio=self.sparse_ratio,
                                        recent=layer.attn.sparse_recent, max_seq_len=ctx,
                                        softmax_scale=self.scale)
            x = x + F.linear(o.reshape(b, 1, qd), layer.w_o)
            h = rms_norm(x, layer.norm2, cfg.rms_norm_eps)
            gu = F.linear(h, layer.w_gate_up)
            g, u = gu.chunk(2, dim=-1)
            x = x + F.linear(F.silu(g) * u, layer.w_down)
        x = rms_norm(x, self.norm, cfg.rms_norm_eps)
        return F.linear(x, self.lm_head)
