"""Build libwh_sample.so (the gfx950 token-selection library) in-tree.

    python -m whallm_amd.build

Compiles every HIP source under whallm_amd/csrc with hipcc for gfx950 into
whallm_amd/libwh_sample.so.  Flags: -ffp-contract=off keeps float32
arithmetic in the exact operation order the CPU oracle uses (no fused
multiply-adds the source does not write); packed-fp32 instructions are
disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libwh_sample.so")
SOURCES = ["wh_sample.hip", "wh_verify.hip", "wh_fast.hip", "wh_draft.hip", "wh_logprobs.hip", "wh_history.hip", "wh_lmhead.hip", "wh_wide.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # leading scalar kernel arguments arrive in SGPRs at wave launch
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libwh_sample.so")


def source_digest() -> str:
    """sha256 over the library's sources (every file under csrc, the public
    header) and its compiler flags: what a profile was measured on."""
    import hashlib

    h = hashlib.sha256()
    files = sorted(os.listdir(CSRC))
    for name in files:
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            with open(os.path.join(CSRC, name), "rb") as f:
                h.update(f.read())
    with open(os.path.join(ROOT, "include", "wh_sample.h"), "rb") as f:
        h.update(f.read())
    h.update(" ".join(SOURCES + HIPCC_FLAGS).encode())
    return h.hexdigest()


def build(verbose: bool = False) -> str:
    missing = [s for s in SOURCES if not os.path.exists(os.path.join(CSRC, s))]
    if missing:
        raise RuntimeError(f"library sources missing: {missing}")
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd))
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libwh_sample.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
