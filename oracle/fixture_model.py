"""The reference's pinned classifier, rebuilt for checking against ``reference_kernel_outputs.npz``.

TEST INFRASTRUCTURE ONLY (the product never imports ``oracle/``).

``tests/test_kernel_outputs_pinned.py:26-74`` (reference) builds ``experiments/uea/train.py:159-305``'s
``PathLabelModel`` from ``PRNGKey(0)`` with: general A (variance 1), lift B (out_dim 5, first channel kept,
``ews/params.py:1166-1217``), depth 2, M = 4, exact expms, an MLP head with one hidden layer of 16
(equinox's ``MLP``: ReLU hidden, identity out, ``Linear`` weights U(-1/sqrt(in), 1/sqrt(in))), a learned-gain
feature norm initialised to ones (``ews/norms.py:148-235``). Inputs: ``RandomState(0)``,
``cumsum(0.1 randn(4, 9, 3))``, clock ``linspace(0, 1, 9)``, all float32.

The draws come from ``oracle/jax_prng.py``. The model's forward (B lift, EWS, norm, head) is restated here;
the EWS itself is supplied by the caller, so the same harness pins both the float64 oracle and the GPU path.
"""

from __future__ import annotations

import numpy as np

from . import jax_prng as P

B_, L_, D_, NCLASS = 4, 9, 3, 3


def fixture_inputs():
    """tests/test_kernel_outputs_pinned.py:26-29 (reference)."""
    rng = np.random.RandomState(0)
    paths = np.cumsum(0.1 * rng.randn(B_, L_, D_).astype("float32"), axis=1)
    clocks = np.broadcast_to(np.linspace(0, 1, L_, dtype="float32"), (B_, L_)).copy()
    return paths.astype(np.float32), clocks


def fixture_params(d_in=D_, feature="signature", w=5, N=2):
    """(A (w,w) f32, B (w-1, d_in-1) f32, head [(W0, b0), (W1, b1)] f64) from PRNGKey(0), in the split order
    of experiments/uea/train.py:159-230 and ews/params.py:1195-1217."""
    key = P.prng_key(0)
    key, sub = P.split(key)
    key_a, key_b = P.split(sub, 2)
    A = P.normal(key_a, (w, w), np.float32)
    Bm = P.normal(key_b, (w - 1, d_in - 1), np.float32)
    key, sub = P.split(key)
    if feature == "signature":
        feat_dim = 1 + sum(w**k for k in range(1, N + 1))
    else:
        from .ews_oracle import lyndon_words

        feat_dim = sum(len(x) for x in lyndon_words(N, w))
    hidden, out = 16, NCLASS
    k0, k1 = P.split(sub, 2)
    head = []
    for lk, (fi, fo) in zip((k0, k1), ((feat_dim, hidden), (hidden, out))):
        wk, bk = P.split(lk, 2)
        lim = 1.0 / np.sqrt(fi)
        head.append((P.uniform(wk, (fo, fi), np.float64, -lim, lim), P.uniform(bk, (fo,), np.float64, -lim, lim)))
    return A, Bm, head


def lift(paths, Bm):
    """B with the first channel preserved (ews/params.py:1181-1190)."""
    t = paths[..., :1]
    return np.concatenate([t, paths[..., 1:] @ Bm.T], -1).astype(np.float32)


def head_apply(features, head):
    """eqx.nn.MLP(depth=1): Linear -> ReLU -> Linear, float64 weights."""
    x = np.asarray(features, np.float64)
    (W0, b0), (W1, b1) = head
    hdn = np.maximum(x @ W0.T + b0, 0.0)
    return hdn @ W1.T + b1


def combinations():
    """tests/test_kernel_outputs_pinned.py:55-68 (reference): name -> (mode, readout, terminal_reduce, feature)."""
    out = {}
    for mode in ["displacement", "displacement_uniform", "displacement_uniform_basepoint"]:
        for reduce in ["tree", "assoc"]:
            out[f"{mode}|terminal|{reduce}"] = (mode, "terminal", reduce, "signature")
        for readout in ["mean", "max"]:
            out[f"{mode}|{readout}|-"] = (mode, readout, "tree", "signature")
    out["displacement|terminal|tree|log"] = ("displacement", "terminal", "tree", "logsignature")
    return out
