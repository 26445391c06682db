"""Compile the HIP sources into latentserve_amd/liblatentserve_hip.so (in-tree).

    python -m latentserve_amd.csrc.build
    python -m latentserve_amd.csrc.build --diagnostics PATH   (measurement build)
    python -m latentserve_amd.csrc.build --stamps PATH        (timeline build)

Cross-compiles for gfx950 with hipcc; no GPU is needed. Object files go to
latentserve_amd/csrc/_build/ (git-ignored). The library links the HIP runtime
by soname, so inside a PyTorch process it binds to the runtime torch already
loaded.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB = os.path.join(PKG, "liblatentserve_hip.so")
SOURCES = ["ls_abi.hip", "ls_decode.hip", "ls_sparse_index.hip", "ls_int8_write.hip",
           "ls_gather.hip", "ls_elementwise.hip", "ls_gemm.hip"]
ARCH = os.environ.get("LS_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU forms are disabled for every device pass; fp32 division
# stays IEEE (no fast-math), which the INT8 quantizers rely on.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-fast-math", "-fhip-fp32-correctly-rounded-divide-sqrt", "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built here")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that line is noise.
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False, diagnostics: bool = False, out: str = LIB,
          stamps: bool = False) -> str:
    """Compile and link the library to `out`.  ``diagnostics`` adds
    -DLS_DIAGNOSTICS (ablation variants selected by an environment
    variable, the page-compute probe); ``stamps`` adds -DLS_STAMPS (each
    decode workgroup records the clock at numbered points, read back by
    ls_diag_read_stamps): separate measurement builds, never the shipped
    library."""
    cc = hipcc()
    flags = HIP_FLAGS + (["-DLS_DIAGNOSTICS"] if diagnostics else []) + \
        (["-DLS_STAMPS"] if stamps else [])
    obj_dir = os.path.join(HERE, "_build_diag" if diagnostics else
                           "_build_stamps" if stamps else "_build")
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, s.replace(".hip", ".o")) for s in SOURCES]
    cmds = [[cc, *flags, "-c", os.path.join(HERE, s), "-o", o] for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        for log in ex.map(_run, cmds):
            if verbose and log.strip():
                print(log)
    tmp = out + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    if "--diagnostics" in sys.argv:
        print(build(verbose="-v" in sys.argv, diagnostics=True,
                    out=sys.argv[sys.argv.index("--diagnostics") + 1]))
    elif "--stamps" in sys.argv:
        print(build(verbose="-v" in sys.argv, stamps=True,
                    out=sys.argv[sys.argv.index("--stamps") + 1]))
    else:
        print(build(verbose="-v" in sys.argv))
