"""ls_paged_decode_fp16_noalloc against ls_paged_decode_fp16, on an MI355X.

The no-allocation entry point runs the same kernel with its split records
and arrival counters in the library's fixed device array; its output must
match the workspace entry point's within the path's fp16 tolerance (the
same kernel and split count; the waves of a workgroup claim pages
dynamically, so the order of the sums, and the last bit, can differ
between any two calls).  Two calls in a row, the second smaller (the array keeps the first
call's records; the counters must be back at zero), then sizes past the
array's limit are refused (the counter limit, 2048 (sequence, KV head)
pairs, is refused before any device call: tests/test_abi.py).  Captured
in a HIP graph and replayed, also when the process's first call is the
captured one (a child process).
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


def _graph_replays_match(first_call_captured: bool):
    """Capture one noalloc call, replay it three times with eager work and
    synchronisations between the replays, and compare every replay with the
    workspace entry point's output."""
    from latentserve_amd import _lib
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh

    lens = [3000, 17, 1024, 2048]
    case = paged_case(lens, seed=7)
    q, k, v, t, l = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in case]
    out = torch.full_like(q, float("nan"))
    if not first_call_captured:
        assert _call_noalloc(q, k, v, t, l, 16, 3000, out) == 0
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            rc = _call_noalloc(q, k, v, t, l, 16, 3000, out)
    assert rc == 0, _lib.lib().ls_last_error()
    torch.cuda.synchronize()
    want = pdh.paged_decode_hip(q, k, v, t, l, 3000, num_splits=16).float().cpu().numpy()
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), want, 2e-3, 1e-2, f"replay {rep}")
        _ = (q.float() * 2).sum().item()               # eager work between replays


def test_noalloc_under_graph_capture_and_replay():
    print("noalloc captured, replayed 3x", flush=True)
    _graph_replays_match(first_call_captured=False)


def test_noalloc_first_call_captured_in_a_fresh_process():
    """The library's first noalloc call on the device made under capture (a
    child process, so no earlier call has set the array up)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path.insert(0, %r); "
            "from tests.test_zz_no_alloc import _graph_replays_match; "
            "_graph_replays_match(first_call_captured=True); print('ok')") % root
    print("noalloc first call captured, child process", flush=True)
    r = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout[-2000:] + r.stderr[-2000:]

