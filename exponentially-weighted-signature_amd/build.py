"""Build recipe of libews_mi355x.so: hipcc for gfx950, in-tree (the .so sits beside the Python package)."""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
SOURCES = ["ews_diag.hip", "ews_pairs.hip", "ews_seq.hip", "ews_jordan.hip", "ews_dense.hip", "ews_log.hip", "ews_mixer.hip", "ews_front.hip"]
OUT = os.path.join(HERE, "ews_mi355x", "libews_mi355x.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed FP32 instructions stay off: ordinary float code only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def command(out=OUT):
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    return [hipcc, *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC,
            *[os.path.join(CSRC, s) for s in SOURCES], "-o", out]


def build(out=OUT, verbose=True):
    cmd = command(out)
    if verbose:
        print(" ".join(cmd), flush=True)
    tmp = out + ".tmp"
    cmd[-1] = tmp
    subprocess.check_call(cmd)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    build(sys.argv[1] if len(sys.argv) > 1 else OUT)
