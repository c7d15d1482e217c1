"""Build recipe of the oracle's C restatement (test infrastructure; outputs stay under oracle/_build/).

The reference is pure Python/JAX (no C/C++ sources), so there is no reference build under oracle/_ref/."""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
SRC = os.path.join(HERE, "cpu_scan.c")


def lib_path(kind="f64"):
    return os.path.join(OUT_DIR, f"libcpu_scan_{kind}.so")


def build(verbose=True):
    if not os.path.exists(SRC):
        return None
    os.makedirs(OUT_DIR, exist_ok=True)
    outs = []
    for kind, real in (("f64", "double"), ("f32", "float")):
        out = lib_path(kind)
        cmd = ["gcc", "-O3", "-march=x86-64-v2", "-fopenmp", "-shared", "-fPIC", f"-DREAL={real}", SRC, "-lm",
               "-o", out]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.check_call(cmd)
        outs.append(out)
    return outs
