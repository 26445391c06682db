"""The page-compute probe: both formulations compute the page's attention.

The MFMA mode is the decode kernel's own compute_page, so this is also a
unit test of it on known values; the VALU mode is the alternative it is
timed against.  Held to the attention tolerance of fp16 inputs with fp32
sums (max-abs 2e-3) against fp32 torch.
"""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


@pytest.mark.parametrize("mode", ["mfma", "valu"])
@pytest.mark.parametrize("items", [1, 37])
def test_probe_modes_compute_the_page_attention(mode, items):
    from latentserve_amd.kernels.hip import compute_probe as cp
    out = cp.run(mode, groups=3, items=items)
    torch.cuda.synchronize()
    want = cp.reference().cuda()
    assert (out - want).abs().max().item() < 2e-3
    assert torch.equal(out[0], out[-1])             # every wave computes the same page
