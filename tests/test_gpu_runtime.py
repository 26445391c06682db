"""The decoder glue and the HIP-graph runner, on an MI355X.

* A small Qwen-geometry decoder (2 layers, the real attention geometry) run
  step by step through the paged cache and the HIP decode kernel agrees with
  a from-scratch fp32 forward over the whole sequence (causal attention by
  torch ops, same weights).
* GraphedDecoder: graph steps agree with eager steps from the same state,
  a sequence crossing a bucket boundary captures a second graph, replays
  of one graph across growing lengths stay correct (the reference's
  tests/test_phase13_graph.py checks the same three).
"""

from __future__ import annotations

import math

import pytest

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def small_cfg():
    from latentserve_amd.runtime.qwen_decoder import DecoderConfig
    return DecoderConfig(vocab_size=512, intermediate_size=384, num_layers=2)


def make_model(cap=256, batch=3, seed=0):
    from latentserve_amd.runtime.qwen_decoder import QwenDecoder
    m = QwenDecoder(small_cfg(), seed=seed, std=0.05)
    m.allocate_cache(batch, cap)
    return m


def reference_logits(model, ids):
    """fp32 forward of sequences ids [B, T] from scratch -> last logits [B, V]."""
    cfg = model.cfg
    b, t = ids.shape
    x = model.embed[ids].float()
    pos = torch.arange(t, device=ids.device)
    cos, sin = model.rope.cos[pos], model.rope.sin[pos]             # [T, D]
    half = cfg.head_dim // 2

    def rope(z):                                                   # [B, H, T, D]
        rot = torch.cat([-z[..., half:], z[..., :half]], dim=-1)
        return z * cos + rot * sin

    def norm(z, w):
        return z * torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + cfg.rms_norm_eps) * w.float()

    qd, kvd, hd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim, cfg.head_dim
    mask = torch.full((t, t), float("-inf"), device=ids.device).triu(1)
    for layer in model.layers:
        h = norm(x, layer.norm1)
        qkv = h @ layer.w_qkv.float().T + layer.b_qkv.float()
        q = rope(qkv[..., :qd].view(b, t, cfg.num_heads, hd).transpose(1, 2))
        k = rope(qkv[..., qd:qd + kvd].view(b, t, cfg.num_kv_heads, hd).transpose(1, 2))
        v = qkv[..., qd + kvd:].view(b, t, cfg.num_kv_heads, hd).transpose(1, 2)
        rep = cfg.num_heads // cfg.num_kv_heads
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
        att = torch.softmax(q @ k.transpose(-1, -2) / math.sqrt(hd) + mask, dim=-1) @ v
        x = x + att.transpose(1, 2).reshape(b, t, qd) @ layer.w_o.float().T
        h = norm(x, layer.norm2)
        g, u = (h @ layer.w_gate_up.float().T).chunk(2, dim=-1)
        x = x + (torch.nn.functional.silu(g) * u) @ layer.w_down.float().T
    x = norm(x, model.norm)
    return x[:, -1] @ model.lm_head.float().T


def test_decode_steps_match_a_from_scratch_fp32_forward():
    torch.manual_seed(0)
    m = make_model(cap=256, batch=3)
    steps = 70
    ids = torch.randint(0, m.cfg.vocab_size, (3, steps), device="cuda")
    for t in range(steps):
        m.cache.advance(1, batch_size=3)
        pos = torch.full((3, 1), t, dtype=torch.long, device="cuda")
        logits = m.decode_forward_static(ids[:, t:t + 1], pos, max_position=t)
    want = reference_logits(m, ids)
    got = logits[:, -1].float()
    err = (got - want).abs().max().item()
    assert err <= 2e-2 * want.abs().max().item() + 1e-3, err
    assert torch.equal(got.argmax(-1), want.argmax(-1))


def test_graph_steps_match_eager_steps_and_buckets_capture_once():
    from latentserve_amd.runtime.hip_graph import GraphedDecoder

    torch.manual_seed(1)
    runs = {}
    for enabled in (True, False):
        m = make_model(cap=256, batch=2, seed=3)
        dec = GraphedDecoder(m, buckets=(64, 128), enabled=enabled)
        ids = torch.randint(0, m.cfg.vocab_size, (2, 140), generator=torch.Generator().manual_seed(5))
        ids = ids.cuda()
        out = []
        for t in range(140):                       # crosses 64 and 128
            pos = torch.full((2, 1), t, dtype=torch.long, device="cuda")
            out.append(dec.step(ids[:, t:t + 1], pos, slots=[0, 1]).clone())
        runs[enabled] = (torch.stack(out), dec.stats())
    # eager picks its split count from the current length, a graph pins the
    # bucket's: a different summation order, a few fp16 ulps on the logits
    g, e = runs[True][0].float(), runs[False][0].float()
    assert (g - e).abs().max().item() <= 3e-3 * e.abs().max().item() + 1e-4
    stats = runs[True][1]
    assert stats["captures"] == 3 and stats["graph_steps"] == 140
    assert [k[:2] for k in stats["keys"]] == [(2, 64), (2, 128), (2, 256)]
    assert runs[False][1]["eager_steps"] == 140


def test_greedy_step_is_the_captured_argmax():
    from latentserve_amd.runtime.hip_graph import GraphedDecoder

    m = make_model(cap=128, batch=2, seed=7)
    dec = GraphedDecoder(m, buckets=(128,), greedy=True)
    tok = torch.zeros(2, 1, dtype=torch.long, device="cuda")
    for t in range(5):
        pos = torch.full((2, 1), t, dtype=torch.long, device="cuda")
        nxt = dec.step_greedy(tok, pos, slots=[0, 1])
        logits = dec._last_graph.logits_buf
        assert torch.equal(nxt, logits[:, -1].argmax(-1, keepdim=True))
        tok = nxt.clone()


def test_sparse_full_ratio_step_matches_dense():
    """ratio 1.0 runs index -> select -> sparse attend and must equal dense."""
    torch.manual_seed(2)
    outs = []
    for ratio in (None, 1.0):
        m = make_model(cap=128, batch=2, seed=9)
        if ratio is not None:
            m.set_sparse(ratio)
        ids = torch.randint(0, m.cfg.vocab_size, (2, 50), generator=torch.Generator().manual_seed(3))
        ids = ids.cuda()
        for t in range(50):
            m.cache.advance(1, batch_size=2)
            pos = torch.full((2, 1), t, dtype=torch.long, device="cuda")
            logits = m.decode_forward_static(ids[:, t:t + 1], pos, max_position=127)
        outs.append(logits.float())
    assert (outs[0] - outs[1]).abs().max().item() <= 1e-3 * outs[0].abs().max().item() + 1e-4
