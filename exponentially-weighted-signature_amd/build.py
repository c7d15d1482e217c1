"""Build recipe of libews_mi355x.so: hipcc for gfx950, in-tree (the .so sits beside the Python package).

Each source compiles to its own object in parallel (one hipcc per file, `EWS_BUILD_JOBS` at once, default the
CPU count capped at 16), then one hipcc line links the shared library."""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
SOURCES = ["ews_diag.hip", "ews_pairs.hip", "ews_seq.hip", "ews_jordan.hip", "ews_chain.hip", "ews_token1.hip", "ews_dense.hip", "ews_wide.hip", "ews_log.hip", "ews_mixer.hip", "ews_front.hip"]
OUT = os.path.join(HERE, "ews_mi355x", "libews_mi355x.so")
OBJ_DIR = os.path.join(HERE, "_build")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed FP32 instructions stay off: ordinary float code only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc():
    return os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def compile_command(src, obj):
    return [_hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-c",
            os.path.join(CSRC, src), "-o", obj]


def link_command(objs, out=OUT):
    return [_hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", out]


def build(out=OUT, verbose=True, sources=None):
    """Compile every source (or only `sources`, reusing the other objects) and link `out`."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs = [os.path.join(OBJ_DIR, s.replace(".hip", ".o")) for s in SOURCES]
    todo = [(s, o) for s, o in zip(SOURCES, objs) if sources is None or s in sources or not os.path.exists(o)]
    jobs = int(os.environ.get("EWS_BUILD_JOBS", min(16, os.cpu_count() or 1)))

    def run(so):
        cmd = compile_command(*so)
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.check_call(cmd)

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(run, todo))
    tmp = out + ".tmp"
    cmd = link_command(objs, tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.check_call(cmd)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    args = sys.argv[1:]
    build(sources=args or None)
