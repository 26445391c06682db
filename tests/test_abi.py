"""The C ABI, checked without a GPU: the library loads, exports every entry
point include/latentserve_amd.h declares, and rejects bad arguments before
any launch (argument checks need no device)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "latentserve_amd.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ls_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from latentserve_amd import _lib
    return _lib.lib()


def test_library_exports_every_declared_symbol(lib):
    names = declared()
    assert "ls_paged_decode_fp16" in names and "ls_paged_decode_int8" in names
    for n in names:
        assert hasattr(lib, n), n


def test_python_binding_covers_the_header():
    from latentserve_amd import _lib
    assert set(declared()) == set(_lib.exported_symbols())


def test_abi_version(lib):
    assert lib.ls_abi_version() == 19


def test_workspace_size(lib):
    assert lib.ls_decode_workspace_bytes(16, 2, 6, 1) == 0
    assert lib.ls_decode_counter_ints(16, 2) == 16 * 2 * 32
    assert lib.ls_decode_counter_ints(0, 2) == 0
    assert lib.ls_decode_workspace_bytes(16, 2, 6, 8) == 16 * 2 * 8 * (6 * 128 + 32) * 4


def _strides(*v):
    return (ctypes.c_int64 * len(v))(*v)


def _call_fp16(lib, **over):
    args = dict(q=1024, qs=_strides(1536, 768, 128), k=4096, v=8192,
                kvs=_strides(4096, 256, 128), nb=10, bt=16, bts=4, mp=4, sl=32, out=64,
                outs=_strides(1536, 768, 128), work=None, cnt=64,
                B=2, H=2, NR=6, D=128, P=16, S=1, msl=0, scale=0.088)
    args.update(over)
    a = args
    return lib.ls_paged_decode_fp16(a["q"], a["qs"], a["k"], a["v"], a["kvs"], a["nb"], a["bt"],
                                    a["bts"], a["mp"], a["sl"], a["out"], a["outs"], a["work"],
                                    a["cnt"], a["B"], a["H"], a["NR"], a["D"], a["P"], a["S"],
                                    a["msl"], a["scale"], None)


@pytest.mark.parametrize("over,needle", [
    (dict(D=64), "head_dim"),
    (dict(P=32), "page"),
    (dict(NR=17), "n_rep"),
    (dict(q=None), "null"),
    (dict(q=1026), "aligned"),
    (dict(cnt=None), "counters is required"),
    (dict(S=4, cnt=64), "num_splits > 1 needs"),
    (dict(S=4, work=4096 + 64, cnt=64), "256-byte"),
    (dict(kvs=_strides(4096, 256, 127)), "aligned"),
])
def test_bad_arguments_are_rejected_before_launch(lib, over, needle):
    rc = _call_fp16(lib, **over)
    assert rc == 1
    assert needle in lib.ls_last_error().decode()


def test_zero_batch_is_a_no_op(lib):
    assert _call_fp16(lib, B=0) == 0


def test_noalloc_refuses_more_pairs_than_its_counters(lib):
    """The fixed scratch holds 65536 counter ints, one 128-byte line (32
    ints) per (sequence, KV head): 2048 pairs; more are refused before any
    device call."""
    assert lib.ls_decode_counter_ints(2048, 1) == 65536
    rc = lib.ls_paged_decode_fp16_noalloc(1024, _strides(1536, 768, 128), 4096, 8192,
                                          _strides(4096, 256, 128), 10, 16, 4, 4, 32, 64,
                                          _strides(1536, 768, 128), 1025, 2, 6, 128, 16, 1, 0,
                                          0.088, None)
    assert rc == 1
    assert "arrival counters" in lib.ls_last_error().decode()


def test_kernel_resources_rejects_unknown_names_and_bad_shapes(lib):
    """Argument checks of ls_kernel_resources, before any device call."""
    from latentserve_amd import _lib
    r = _lib.KernelResources()
    assert lib.ls_kernel_resources(b"no_such_kernel", 2, 6, 0, 0, ctypes.byref(r)) == 1
    assert "unknown kernel" in lib.ls_last_error().decode()
    assert lib.ls_kernel_resources(b"paged_decode_fp16", 0, 6, 0, 0, ctypes.byref(r)) == 1
    assert lib.ls_kernel_resources(b"page_index", 2, 17, 0, 0, ctypes.byref(r)) == 1
    assert lib.ls_kernel_resources(b"page_index", 2, 6, 0, 0, None) == 1

