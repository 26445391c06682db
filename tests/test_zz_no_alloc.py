"""ls_paged_decode_fp16_noalloc against ls_paged_decode_fp16, on an MI355X.

The no-allocation entry point runs the same kernel with its split records
and arrival counters in the library's fixed device array; its output must
match the workspace entry point's within the path's fp16 tolerance (the
same kernel and split count; the waves of a workgroup claim pages
dynamically, so the order of the sums, and the last bit, can differ
between any two calls).  Two calls in a row, the second smaller (the array keeps the first
call's records; the counters must be back at zero), then sizes past the
array's limit are refused.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from tests.cases import assert_close, paged_case

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def _call_noalloc(q, k, v, t, l, splits, max_len, out):
    from latentserve_amd import _lib
    P, S = _lib.ptr, _lib.strides
    b, h, n_rep, d = q.shape
    return _lib.lib().ls_paged_decode_fp16_noalloc(
        P(q), S(q, 3), P(k), P(v), S(k, 3), k.shape[0], P(t), t.stride(0), t.shape[1], P(l),
        P(out), S(out, 3), b, h, n_rep, d, k.shape[1], splits, max_len,
        1.0 / math.sqrt(d), _lib.stream_of(q.device))


@pytest.mark.parametrize("splits", [1, 16])
def test_noalloc_equals_the_workspace_entry_point(splits):
    from latentserve_amd import _lib
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh

    for lens, seed in (([4096, 3000, 17, 1024, 777, 0, 2048, 64], 1), ([500, 33], 2)):
        print(f"noalloc splits={splits} lens={lens}", flush=True)
        case = paged_case(lens, seed=seed)
        q, k, v, t, l = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in case]
        max_len = int(max(lens)) or 1
        want = pdh.paged_decode_hip(q, k, v, t, l, max_len, num_splits=splits).clone()
        out = torch.full_like(q, float("nan"))
        rc = _call_noalloc(q, k, v, t, l, splits, max_len, out)
        assert rc == 0, _lib.lib().ls_last_error()
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), want.float().cpu().numpy(), 2e-3, 1e-2,
                     f"noalloc against ls_paged_decode_fp16, splits={splits}")
        assert_close(out.float().cpu().numpy(), oracle.paged_decode(*case), 2e-3, 1e-2,
                     f"noalloc splits={splits}")


def test_noalloc_refuses_sizes_past_its_scratch():
    from latentserve_amd import _lib

    case = paged_case([64, 64], seed=3)
    q, k, v, t, l = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in case]
    out = torch.empty_like(q)
    # 2 x 2 x 100000 records of 800 floats: far past 16 MiB
    rc = _call_noalloc(q, k, v, t, l, 100000, 64, out)
    assert rc == 1
    assert b"exceed" in _lib.lib().ls_last_error()
