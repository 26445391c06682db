"""HIP block-table gather against the CPU oracle, on an MI355X: bit-exact.

oracle.gather restates the reference's read path (cache/paged_cache.py:
486-506 with the zero-padded slot table of :305-323) and is pinned in
tests/test_oracle.py by the slot rule written out in numpy.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.cases import paged_case

torch = pytest.importorskip("torch")

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def pg():
    from latentserve_amd.kernels.hip import paged_gather
    return paged_gather


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("lengths", [[40, 17, 0], [1, 16, 15, 33], [300]])
def test_gather_fp16_is_bit_exact(lengths):
    q, k, v, t, l = paged_case(lengths, seed=len(lengths))
    lmax = t.shape[1] * 16
    got = pg().gather(dev(k), dev(t), dev(l), lmax).cpu().numpy()
    want = oracle.gather(k, t, l, lmax)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def test_gather_int8_and_a_shorter_window():
    rng = np.random.default_rng(3)
    _, k, _, t, l = paged_case([70, 5], seed=4)
    k8 = rng.integers(-128, 128, size=k.shape, dtype=np.int8)
    got = pg().gather(dev(k8), dev(t), dev(l), 48).cpu().numpy()
    np.testing.assert_array_equal(got, oracle.gather(k8, t, l, 48))


def test_read_returns_the_reference_layout():
    q, k, v, t, l = paged_case([33, 64], seed=5)
    K, V = pg().read(dev(k), dev(v), dev(t), dev(l), 64)
    assert K.shape == (2, 2, 64, 128) and K.stride() == (64 * 2 * 128, 128, 2 * 128, 1)
    np.testing.assert_array_equal(V.cpu().numpy().view(np.uint16),
                                  oracle.gather(v, t, l, 64).view(np.uint16))


def test_block_ids_outside_the_pool_read_slot_0():
    _, k, _, t, l = paged_case([32], seed=6)
    t = t.copy()
    t[0, 1] = 10 ** 6
    got = pg().gather(dev(k), dev(t), dev(l), 32).cpu().numpy()
    np.testing.assert_array_equal(got[0, :, 16:].view(np.uint16),
                                  np.broadcast_to(k.reshape(-1, 2, 128)[0][:, None],
                                                  (2, 16, 128)).view(np.uint16))
