"""ctypes binding of liblatentserve_hip.so (the C ABI in include/latentserve_amd.h).

The library is built in-tree by ``python -m latentserve_amd.csrc.build``.
There is no fallback: if it is missing or fails to load, every entry point
raises, so a GPU run can never silently take another path.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
# LATENTSERVE_HIP_LIB points at another build of the same ABI (A/B runs).
LIB_PATH = os.environ.get("LATENTSERVE_HIP_LIB") or os.path.join(HERE, "liblatentserve_hip.so")

_VP = ctypes.c_void_p
_I64P = ctypes.POINTER(ctypes.c_int64)
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

LS_ERR_INVALID = 1
LS_ERR_HIP = 2
# The ABI this binding is written for (include/latentserve_amd.h); a library
# built from other sources is refused rather than called with wrong arguments.
ABI_VERSION = 19

# name -> argtypes, mirroring include/latentserve_amd.h
_SIGNATURES = {
    "ls_abi_version": [],
    "ls_kernel_resources": [ctypes.c_char_p, _I32, _I32, _I32, _I32, _VP],
    "ls_last_error": [],
    "ls_decode_workspace_bytes": [_I32, _I32, _I32, _I32],
    "ls_decode_counter_ints": [_I32, _I32],
    "ls_paged_decode_fp16": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _I64P,
        _VP, _VP, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _VP],
    "ls_paged_decode_fp16_noalloc": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _I64P,
        _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _VP],
    "ls_page_mass_workspace_bytes": [_I32, _I32, _I32, _I32],
    "ls_set_coop_wait_ticks": [ctypes.c_uint64],
    "ls_page_scores_mass": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _VP, _I64P, _I32, _I32,
        _I32, _I32, _I32, _I32, _F32, _VP],
    "ls_sparse_attention_bounds_fp16": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _VP, _I64P, _VP, _I64P,
        _I32, _F32, _I32, _VP, _I64P, _VP, _VP, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32,
        _VP],
    "ls_paged_decode_int8": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64P, _VP, _I64P, _VP, _VP,
        _VP, _I64P, _I32, _VP, _VP, _I64, _I32, _VP, _VP, _I64P,
        _VP, _VP, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _VP],
    "ls_paged_sparse_fp16": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _I64P,
        _I32, _F32, _I32, _VP, _I64P, _VP, _VP,
        _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _VP],
    "ls_sparse_attention_fp16": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _I64P, _I32, _I32, _F32,
        _I32, _VP, _I64P, _VP, _VP, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _VP],
    "ls_page_scores": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _I64P,
        _I32, _I32, _I32, _I32, _I32, _I32, _VP],
    "ls_sparse_index": [
        _VP, _I64P, _VP, _VP, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _I64P,
        _VP, _I32, _F32, _I32, _VP, _I64P, _I32, _I32, _I32, _I32, _I32, _VP],
    "ls_page_select": [
        _VP, _I64P, _VP, _I32, _I32, _I32, _I32, _F32, _I32, _I32, _VP, _I64P, _VP],
    "ls_page_bounds_update": [
        _VP, _I64P, _VP, _VP, _VP, _I64P, _I32, _I32, _I32, _I32, _I32, _VP],
    "ls_page_bounds_rebuild": [
        _VP, _I64P, _I32, _VP, _VP, _I64P, _I32, _I32, _I32, _VP],
    "ls_int8_decode_write": [
        _VP, _I64P, _VP, _I64P, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I32, _I32, _I32,
        _I32, _F32, _F32, _F32, _F32, _I32, _VP],
    "ls_int8_finalize_blocks": [
        _VP, _I64P, _VP, _I32, _VP, _I64P, _VP, _VP, _I64P, _I64, _I32, _I32, _I32, _I32,
        _F32, _F32, _F32, _F32, _I32, _VP],
    "ls_paged_gather": [
        _VP, _I32, _I64P, _I32, _VP, _I64, _I32, _VP, _VP, _I64P, _I32, _I32, _I32, _I32, _I32,
        _VP],
    "ls_rms_norm": [
        _VP, _I64, _VP, _I64, _VP, _VP, _I64, _VP, _I64, _I32, _I32, _F32, _VP],
    "ls_silu_and_mul": [_VP, _I64, _VP, _I64, _I32, _I32, _VP],
    "ls_rope_qk": [
        _VP, _I64, _VP, _I64, _VP, _I64, _VP, _I64, _VP, _I64, _VP, _I64, _I32, _I32, _I32, _I32,
        _VP],
    "ls_rope_write_decode": [
        _VP, _I64, _VP, _VP, _VP, _I64, _I32, _VP, _VP, _VP, _I64P, _I32, _I32, _VP, _I64P, _VP,
        _VP, _I64P, _I32, _I32, _I32, _I32, _VP],
    "ls_decode_qkv_rope_write": [
        _VP, _I64, _VP, _I64, _I32, _VP, _I32, _VP, _VP, _VP, _I64, _I32, _VP, _VP, _VP, _I64P, _I32,
        _I32, _VP, _I64P, _VP, _VP, _I64P, _I32, _I32, _I32, _I32,
        _VP, _I64, _VP, _F32, _VP, _I64, _VP],
    "ls_embed_rms_norm": [
        _VP, _I64, _I64, _VP, _VP, _VP, _I64, _VP, _I64, _I32, _I32, _F32, _VP],
    "ls_argmax_workspace_bytes": [_I32, _I32],
    "ls_argmax_rows": [_VP, _I64, _VP, _I32, _I32, _VP, _SZ, _VP],
    "ls_decode_gemm": [_VP, _I64, _VP, _I64, _I32, _VP, _VP, _I64, _I32, _I32, _I32, _VP, _SZ,
                       _VP, _I64, _VP, _F32, _VP, _I64, _VP],
    "ls_gemm_packed_bytes": [_I32, _I32, _I32, _I32],
    "ls_pack_gemm_weight": [_VP, _I64, _I32, _I32, _I32, _I32, _VP, _VP],
    "ls_decode_gemm_workspace_bytes": [_I32, _I32, _I32],
    "ls_decode_gate_up_silu": [_VP, _I64, _VP, _I64, _I32, _VP, _VP, _I64, _I32, _I32, _I32,
                               _VP, _I64, _VP, _F32, _VP, _I64, _VP],
    "ls_combine_splits": [
        _VP, _I64P, _VP, _VP, _I64P, _VP, _I32, _I64P, _I32, _I32, _I32, _I32, _I32, _VP],
}

_lib: Optional[ctypes.CDLL] = None


class HipLibraryMissing(RuntimeError):
    pass


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """Load the library (once). Raises HipLibraryMissing if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m latentserve_amd.csrc.build` "
                "(the HIP backend has no fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = {"ls_last_error": ctypes.c_char_p,
                          "ls_decode_workspace_bytes": ctypes.c_size_t,
                          "ls_decode_counter_ints": ctypes.c_size_t,
                          "ls_decode_gemm_workspace_bytes": ctypes.c_size_t,
                          "ls_argmax_workspace_bytes": ctypes.c_size_t,
                          "ls_page_mass_workspace_bytes": ctypes.c_size_t,
                          "ls_gemm_packed_bytes": ctypes.c_size_t}.get(name, ctypes.c_int)
        got = handle.ls_abi_version()
        if got != ABI_VERSION:
            raise HipLibraryMissing(
                f"{LIB_PATH} has ABI {got}, this binding expects {ABI_VERSION}: rebuild it with "
                "`python -m latentserve_amd.csrc.build`")
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    msg = lib().ls_last_error().decode(errors="replace")
    if rc == LS_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else _VP(t.data_ptr())


def strides(t: Optional[torch.Tensor], n: int):
    if t is None:
        return None
    return (ctypes.c_int64 * n)(*t.stride()[:n])


class KernelResources(ctypes.Structure):
    """LsKernelResources (include/latentserve_amd.h)."""
    _fields_ = [("regs", ctypes.c_int), ("local_bytes", ctypes.c_int),
                ("shared_bytes", ctypes.c_int), ("threads", ctypes.c_int),
                ("groups_per_cu", ctypes.c_int)]


def kernel_resources(kernel: str, device: Optional[torch.device] = None, kv_heads: int = 2,
                     n_rep: int = 6, asym: bool = False, has_res: bool = False) -> dict:
    """ls_kernel_resources for one kernel, as a dict, on `device` (default:
    the current one)."""
    r = KernelResources()
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    with torch.cuda.device(dev):
        rc = lib().ls_kernel_resources(kernel.encode(), int(kv_heads), int(n_rep), int(asym),
                                       int(has_res), ctypes.byref(r))
    check(rc, "ls_kernel_resources")
    return {name: int(getattr(r, name)) for name, _ in KernelResources._fields_}


def stream_of(device: torch.device):
    """torch's current stream on `device` as a hipStream_t."""
    return _VP(torch.cuda.current_stream(device).cuda_stream)
