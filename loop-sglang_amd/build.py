"""Build recipe for libloopsgl_tok.so (HIP, gfx950).

Each translation unit is compiled separately because the exit-gate kernels need
``-ffp-contract=off`` (the cumulative exit probability is three separately
rounded fp32 operations), while the sampler may contract to FMA.  The shared
library lands next to this file so it travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB_NAME = "libloopsgl_tok.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
STAMPS_LIB_PATH = os.path.join(HERE, "libloopsgl_tok_stamps.so")
ARCH = os.environ.get("LSG_OFFLOAD_ARCH", "gfx950")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Never emit packed-fp32 VALU ops (v_pk_add/mul/fma_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

SOURCES = {
    "sample.hip": ["-ffp-contract=fast"],
    "sample_quad.hip": ["-ffp-contract=fast"],
    "exit_gate.hip": ["-ffp-contract=off"],
    "lm_head.hip": [],
    "capi.hip": [],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libloopsgl_tok.so)")


def build(verbose: bool = False, stamps: bool = False) -> str:
    """Compile every HIP source and link libloopsgl_tok.so; returns its path.

    stamps=True builds the profiling variant instead, libloopsgl_tok_stamps.so:
    the sampler records per-workgroup phase timestamps (-DLSG_PHASE_STAMPS),
    read back by phase_stamps.py.  The product library is left untouched.
    """
    bdir = os.path.join(BUILD, "stamps") if stamps else BUILD
    lib_path = STAMPS_LIB_PATH if stamps else LIB_PATH
    os.makedirs(bdir, exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src, extra in SOURCES.items():
        obj = os.path.join(bdir, src.replace(".hip", ".o"))
        objs.append(obj)
        flags = [*extra, "-DLSG_PHASE_STAMPS"] if stamps else extra
        cmd = [cc, *COMMON, *flags, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        # hipcc's host pass does not know the packed-fp32 feature; that warning is harmless.
        lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
        if p.returncode != 0:
            failed.append((src, "\n".join(lines)))
        elif verbose and lines:
            print("\n".join(lines))
    if failed:
        msg = "\n".join(f"--- {s}\n{t}" for s, t in failed)
        raise RuntimeError(f"HIP build failed:\n{msg}")
    tmp = lib_path + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, lib_path)
    return lib_path


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, stamps="--stamps" in sys.argv))
