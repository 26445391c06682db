"""A Qwen2.5-1.5B-geometry decoder for the graph runner and the full-step
benchmark: random-init fp16 weights, the paged cache, and the HIP paged
decode attention in every layer.

The reference's model/ stack (model/qwen.py, model/attention/gqa.py) is not
rebuilt: this is the minimum that gives the decode-attention path its real
surroundings (28 layers, hidden 1536, 12 query / 2 KV heads, MLP 8960,
vocab 151936, tied embeddings, RoPE theta 1e6, q/k/v biases) so a captured
decode step can be timed on the reference's full-step configuration.  The
projections run on the HIP weight-streaming GEMM with packed weights up to
16 rows (hipBLASLt, through torch, above that, where it is faster); the
MLP activation is in the gate/up GEMM's epilogue, and RoPE + the K/V store
+ the query fold (GQAAttention.forward's decode branch,
model/attention/gqa.py:283-344: q [B, 12, 1, D] folded to [B, 2, 6, D],
the new K/V written first) in the q/k/v GEMM's.  Everything else is HIP
as well: the embedding lookup inside the first norm, per layer the fused
norms (residual add folded in) and the paged decode attention, writing
straight into the output projection's input.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

from latentserve_amd.kernels import decode_gemm as dg
from latentserve_amd.kernels import fused_elementwise as fe
from latentserve_amd.kernels.hip import paged_decode_hip as pdh
from latentserve_amd.kernels.hip import paged_sparse as ps
from latentserve_amd.runtime.int8_cache import Int8PagedKVCache
from latentserve_amd.runtime.kv_cache import KVCacheSpec, PagedKVCache


# Rows up to which the projections take the HIP GEMM (measured: at 1 and 16
# rows it streams the weights 1.3-2.7x faster than hipBLASLt; at 64 rows
# hipBLASLt is faster).
HIP_GEMM_MAX_ROWS = 16


def _pack(w: torch.Tensor, kind: str, head_dim: int = 128):
    """The weight packed for its HIP GEMM launch (GPU weights only)."""
    return dg.PackedWeight(w, kind, head_dim) if w.is_cuda else None


def _linear(x: torch.Tensor, w: torch.Tensor, pw=None,
            b: Optional[torch.Tensor] = None) -> torch.Tensor:
    wk = pw if pw is not None else w
    if x.shape[0] <= HIP_GEMM_MAX_ROWS and dg.supports(x, wk):
        return dg.linear(x, wk, b)
    return F.linear(x, w, b)


def _norm_folds(x: torch.Tensor, pw) -> bool:
    """Whether the RMSNorm before the projection with packed weight pw can
    run in its prologue: at most 16 rows and K not split over workgroups."""
    if pw is None or x.shape[0] > 16 or not dg.supports(x, pw):
        return False
    n = pw.shape[0]
    return dg.workspace_bytes(x.shape[0], n, pw.shape[1]) == 0


def _gate_up_silu(x: torch.Tensor, w: torch.Tensor, pw=None) -> torch.Tensor:
    wk = pw if pw is not None else w
    if x.shape[0] <= HIP_GEMM_MAX_ROWS and dg.supports(x, wk):
        return dg.gate_up_silu(x, wk)                # SiLU in the GEMM's epilogue
    return fe.silu_and_mul(F.linear(x, w))


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
    """Hugging Face's Qwen2 rotary tables (transformers' Qwen2RotaryEmbedding:
    fp32 inverse frequencies and angles, cos / sin cast to the model's fp16),
    built to a fixed bound so that nothing is rebuilt inside a graph."""

    def __init__(self, head_dim: int, theta: float, max_seq_len: int, device):
        self.head_dim, self.theta, self.device = head_dim, theta, device
        self.max_seq_len = 0
        self._build_tables(max_seq_len)

    def _build_tables(self, n: int) -> None:
        inv = 1.0 / (self.theta ** (torch.arange(0, self.head_dim, 2, dtype=torch.int64).float()
                                    / self.head_dim))
        freqs = torch.outer(torch.arange(n, dtype=torch.int64).float(), inv)
        emb = torch.cat([freqs, freqs], dim=-1)
        self.cos = emb.cos().to(torch.float16).to(self.device)
        self.sin = emb.sin().to(torch.float16).to(self.device)
        self.max_seq_len = n


class _Attn:
    def __init__(self):
        self.num_splits: Optional[int] = None
        self.sparse_recent = 2
        self.sparse_scoring = "bounds"


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
        # packed copies for the decode GEMMs (every weight load 1 KiB contiguous)
        self.p_qkv = _pack(self.w_qkv, "qkv", cfg.head_dim)
        self.p_o = _pack(self.w_o, "plain")
        self.p_gate_up = _pack(self.w_gate_up, "gate_up")
        self.p_down = _pack(self.w_down, "plain")


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
        self.p_lm_head = _pack(self.lm_head, "plain")
        self.cache = None
        self._stage = None
        self.rope: Optional[Rope] = None
        self.sparse_ratio: Optional[float] = None
        self.scale = 1.0 / math.sqrt(cfg.head_dim)

    def allocate_cache(self, max_batch_size: int, max_seq_len: int,
                       num_blocks: Optional[int] = None, kv_dtype: str = "fp16",
                       asymmetric: bool = False):
        """A paged cache for this model: fp16 (PagedKVCache) or INT8
        (Int8PagedKVCache: int8 pools, fp32 scales, the fp16 last-page K
        residual)."""
        spec = KVCacheSpec(num_layers=self.cfg.num_layers, num_kv_heads=self.cfg.num_kv_heads,
                           head_dim=self.cfg.head_dim, max_batch_size=max_batch_size,
                           max_seq_len=max_seq_len, device=str(self.device))
        if kv_dtype == "fp16":
            self.cache = PagedKVCache(spec, num_blocks=num_blocks)
            self._stage = None
        elif kv_dtype == "int8":
            self.cache = Int8PagedKVCache(spec, num_blocks=num_blocks, asymmetric=asymmetric)
            # the decode token's rotated K and its V are stored here by the
            # q/k/v launch (one 16-row block per sequence, row 0), then
            # quantized into the cache by its write
            hk, hd = self.cfg.num_kv_heads, self.cfg.head_dim
            self._stage = (
                torch.zeros(max_batch_size, 16, hk, hd, dtype=torch.float16, device=self.device),
                torch.zeros(max_batch_size, 16, hk, hd, dtype=torch.float16, device=self.device),
                torch.arange(max_batch_size, dtype=torch.long, device=self.device) * 16)
        else:
            raise ValueError(f"kv_dtype must be 'fp16' or 'int8', got {kv_dtype!r}")
        self.rope = Rope(self.cfg.head_dim, self.cfg.rope_theta, max_seq_len, self.device)
        return self.cache

    def set_sparse(self, ratio: Optional[float], recent: int = 2,
                   scoring: Optional[str] = None) -> None:
        """Sparse decode attention over a page budget (None: dense), pages
        ranked by their Quest bound ("bounds") or summed estimated mass
        ("mass"; unchanged when None)."""
        if ratio is not None:
            if isinstance(self.cache, Int8PagedKVCache):
                raise ValueError("sparse decode reads fp16 pools; this cache is INT8")
            self.cache.enable_page_bounds()
        self.sparse_ratio = ratio
        for layer in self.layers:
            layer.attn.sparse_recent = recent
            if scoring is not None:
                layer.attn.sparse_scoring = scoring

    @torch.no_grad()
    def decode_forward_static(self, token_ids: torch.Tensor, positions: torch.Tensor,
                              max_position: int) -> torch.Tensor:
        """One decode step for the active sequences: token_ids / positions
        [B, 1] int64 -> logits [B, 1, vocab].  The cache has already been
        advanced; `max_position` bounds every position (a graph bucket)."""
        cfg, cache = self.cfg, self.cache
        b = token_ids.shape[0]
        hq, hk, hd = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        eps = cfg.rms_norm_eps
        tables = cache.block_tables_tensor(b)
        lens = cache.seq_lens_tensor(b)
        int8 = self._stage is not None
        if int8:
            stage_k, stage_v, stage_slots = self._stage
            slots = stage_slots[:b]
            res_rows = cache.residual_rows_tensor(b)
        else:
            slots = cache.write_slots(b)
        pos = positions.reshape(b)
        q = torch.empty((b, hk, hq // hk, hd), dtype=torch.float16, device=self.device)
        o = torch.empty_like(q)                                    # = [B, hq * hd], contiguous
        # The token embedding lookup and the first norm are one launch; the
        # residual is carried into the next norm, which adds and normalises
        # in one launch (the reference's _run_layers_fused,
        # model/latentserve_qwen.py:425-450); the last add goes into the
        # final norm.
        h, residual = fe.embed_rms_norm(self.embed, token_ids.reshape(b), self.layers[0].norm1,
                                        eps)
        x = None
        for li, layer in enumerate(self.layers):
            # with packed weights at decode batch sizes the norm before a
            # projection runs in that projection's prologue (x + residual is
            # written to a new buffer: it may not alias its inputs)
            fold1 = li > 0 and _norm_folds(x, layer.p_qkv)
            if li > 0 and not fold1:
                h, residual = fe.fused_add_rms_norm(x, residual, layer.norm1, eps)
            kmin = kmax = None
            if self.sparse_ratio is not None:
                kmin, kmax = cache.page_bounds(li)
            # the q/k/v projection, RoPE, the K/V store at this step's slots
            # (and the page bounds) and q folded to [B, hk, n_rep, hd]: one
            # launch at decode batch sizes (the projection's epilogue)
            wq = layer.p_qkv if layer.p_qkv is not None else layer.w_qkv
            kdst, vdst = (stage_k, stage_v) if int8 else (cache.k_pool[li], cache.v_pool[li])
            if fold1:
                _, residual = dg.qkv_rope_write(
                    x, wq, layer.b_qkv, pos, self.rope.cos, self.rope.sin, slots,
                    kdst, vdst, hq, hk, q_out=q, kmin=kmin, kmax=kmax,
                    residual=residual, norm_weight=layer.norm1, eps=eps)
            elif b <= HIP_GEMM_MAX_ROWS and dg.supports(h, wq):
                dg.qkv_rope_write(h, wq, layer.b_qkv, pos, self.rope.cos, self.rope.sin,
                                  slots, kdst, vdst, hq, hk, q_out=q, kmin=kmin, kmax=kmax)
            else:
                qkv = F.linear(h, layer.w_qkv, layer.b_qkv)       # [B, (hq + 2 hk) hd]
                fe.rope_write_decode(qkv, pos, self.rope.cos, self.rope.sin, slots,
                                     kdst, vdst, hq, hk, q_out=q, kmin=kmin, kmax=kmax)
            if int8:
                # V quantized into the pool, K into the sequence's residual row
                cache.write(li, stage_k[:b, :1].transpose(1, 2), stage_v[:b, :1].transpose(1, 2))
                pdh.paged_decode_hip(
                    q, cache.k_pool[li], cache.v_pool[li], tables, lens,
                    max_seq_len=max_position + 1, num_splits=layer.attn.num_splits,
                    softmax_scale=self.scale, k_scale=cache.k_scale_pool[li],
                    v_scale=cache.v_scale_pool[li],
                    k_zero=cache.k_zero_pool[li] if cache.asymmetric else None,
                    v_zero=cache.v_zero_pool[li] if cache.asymmetric else None,
                    k_residual=cache.residual(li), res_rows=res_rows, out=o)
            elif self.sparse_ratio is None:
                pdh.paged_decode_hip(q, cache.k_pool[li], cache.v_pool[li], tables, lens,
                                     max_seq_len=max_position + 1,
                                     num_splits=layer.attn.num_splits,
                                     softmax_scale=self.scale, out=o)
            else:
                ctx = cache.sparse_context_hint or max_position + 1
                ps.sparse_attention(q, cache.k_pool[li], cache.v_pool[li], tables, lens, kmin,
                                    kmax, ratio=self.sparse_ratio,
                                    recent=layer.attn.sparse_recent, max_seq_len=ctx,
                                    softmax_scale=self.scale, out=o,
                                    scoring=layer.attn.sparse_scoring)
            x = _linear(o.view(b, hq * hd), layer.w_o, layer.p_o)
            # (the gate/up projection keeps its norm launch: over its 1120
            # workgroups the prologue costs more than the launch it saves)
            h, residual = fe.fused_add_rms_norm(x, residual, layer.norm2, eps)
            x = _linear(_gate_up_silu(h, layer.w_gate_up, layer.p_gate_up), layer.w_down,
                        layer.p_down)
        if _norm_folds(x, self.p_lm_head):
            logits, _ = dg.linear(x, self.p_lm_head, residual=residual, norm_weight=self.norm,
                                  eps=eps)
            return logits.view(b, 1, -1)
        h, _ = fe.fused_add_rms_norm(x, residual, self.norm, eps)
        return _linear(h, self.lm_head, self.p_lm_head).view(b, 1, -1)
