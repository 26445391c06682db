"""The decode kernel's page compute alone, MFMA against VALU (measurement).

``run(mode, groups, items)`` launches ls_compute_probe: groups x 8 waves,
each applying one register-resident page (16 tokens, 6 query rows, 128
channels, synthetic values exact in fp16) ``items`` times to its
online-softmax state.  Mode 0 is the decode kernel's own compute_page (QK and
PV on v_mfma_f32_16x16x16f16), mode 1 a VALU formulation of the same page.
``reference()`` is the same page's attention in fp32 torch: every wave's
output equals it whatever ``items`` is (the page repeats, so its softmax
weights do not change).
"""

from __future__ import annotations

import math

import torch

from latentserve_amd import _lib

ROWS, TOKENS, D, WAVES = 6, 16, 128, 8
MODES = {"mfma": 0, "valu": 1}


def synthetic():
    """(q [6, 128], K [16, 128], V [16, 128]) fp32, the probe's values."""
    t = torch.arange(TOKENS).view(-1, 1)
    r = torch.arange(ROWS).view(-1, 1)
    ch = torch.arange(D).view(1, -1)
    k = ((t * 7 + ch * 3) % 17 - 8).float() * 0.0625
    v = ((t * 5 + ch * 11) % 13 - 6).float() * 0.125
    q = ((r * 13 + ch * 5) % 11 - 5).float() * 0.125
    return q, k, v


def reference(scale: float = 1.0 / math.sqrt(D)) -> torch.Tensor:
    q, k, v = synthetic()
    return torch.softmax((q @ k.t()) * scale, dim=-1) @ v


def run(mode: str, groups: int, items: int, scale: float = 1.0 / math.sqrt(D),
        out: torch.Tensor = None) -> torch.Tensor:
    """[groups * 8, 6, 128] fp32 outputs of every wave."""
    if out is None:
        out = torch.empty(groups * WAVES, ROWS, D, dtype=torch.float32, device="cuda")
    rc = _lib.lib().ls_compute_probe(MODES[mode], groups, items, float(scale), out.data_ptr(),
                                     torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "ls_compute_probe")
    return out
