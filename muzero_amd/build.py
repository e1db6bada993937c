"""Build libmuzero_hip.so in-tree with hipcc for gfx950.

Usage: ``python -m muzero_amd.build`` (also called by ``__graft_entry__.build``).
The library is written next to this file (``muzero_amd/libmuzero_hip.so``) so
it travels with the source tree; it is never installed elsewhere.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmuzero_hip.so")
SOURCES = ["quantize.hip", "decode.hip", "decode_fold.hip", "decode_cb.hip", "decode_twopass.hip", "prologue.hip", "qk_av.hip", "stream.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # the reference evaluates every elementwise op separately: no FMA contraction
    "-ffp-contract=off",
    # no packed-FP32 instructions (v_pk_*_f32) anywhere in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm 7.x expected under /opt/rocm)")


def build(verbose: bool = True) -> str:
    """Compile every HIP source into one shared library (always rebuilds).

    Each source compiles to an object in its own hipcc process (in parallel),
    then one link step writes the library."""
    inc = ["-I", os.path.join(ROOT, "include")]
    with tempfile.TemporaryDirectory(prefix="muzero_build_") as tmpdir:
        procs = []
        for src in SOURCES:
            obj = os.path.join(tmpdir, os.path.splitext(src)[0] + ".o")
            cmd = [hipcc(), *HIPCC_FLAGS, *inc, "-c", os.path.join(CSRC, src), "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((cmd, obj, subprocess.Popen(cmd)))
        failed = [cmd for cmd, _, p in procs if p.wait() != 0]
        if failed:
            raise subprocess.CalledProcessError(1, failed[0])
        tmp = LIB + ".tmp"
        link = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *[o for _, o, _ in procs], "-o", tmp]
        if verbose:
            print(" ".join(link), flush=True)
        subprocess.run(link, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
