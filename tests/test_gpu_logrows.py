"""GPU parity of the LogEWS prefix rows written by the chunk kernels' output pass (rotation planes, and real
diagonals off the sequential kernels: an explicit chunk length or cached flows): the compressed log of every prefix
row (ews/layer.py:488-517, restated in oracle/ews_oracle.py log_ews_single and pinned to the reference's golden
`log` logit in tests/test_oracle_golden.py) straight from the scan, and its backward through the log cotangent
turned into a flat-row cotangent. Against the float64 oracle (forward <= 1e-5, gradients of path, clock and A
<= 1e-4, metric max|a-b| / max|b|) and against the rows-then-log route on the same GPU (ops.log_rows after the flat
prefix rows).
"""

import numpy as np
import pytest
import torch

import ews_mi355x as E
from ews_mi355x import ops
from oracle import ews_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def relerr(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _data(B, L, d, seed, uniform):
    rng = np.random.default_rng(seed)
    path = np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1)
    if uniform:
        clock = np.broadcast_to(np.linspace(0.0, 1.0, L), (B, L)).copy()
    else:
        clock = np.cumsum(rng.lognormal(-3.0, 0.3, size=(B, L)), 1)
    return torch.tensor(path, dtype=torch.float32), torch.tensor(clock, dtype=torch.float32)


def _params(structure, K, seed):
    rng = np.random.default_rng(seed + 100)
    if structure == "planes":
        v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
        u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
        return (E.AParamDampedRotation(v.clone(), u.clone(), 2 * K, omega_scale=3.0).to(DEV),
                E.AParamDampedRotation(v.double(), u.double(), 2 * K, omega_scale=3.0))
    th = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    return E.AParamEFM(th.clone()).to(DEV), E.AParamEFM(th.double())


CASES = [
    # structure, K, B, L, uniform clock, reweighting mode
    ("planes", 8, 2, 150, False, "displacement"),           # d = 16: the generic kernels (no pair-group log)
    ("planes", 3, 2, 90, True, "displacement_uniform"),     # cached flows
    ("planes", 12, 2, 70, False, "displacement"),           # d = 24: 1,024-lane workgroups
    ("real", 8, 3, 120, False, "displacement_uniform_basepoint"),
    ("real", 5, 2, 65, True, "displacement_uniform"),
    # a few long samples of a real diagonal with per-interval flows: the default plan takes the chunk kernels (the
    # per-sample sequential kernels are for B >= 128 and L <= 1025), whose output pass writes the log rows
    ("real", 8, 2, 5000, False, "displacement"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-K{c[1]}-L{c[3]}-{c[5]}" for c in CASES])
def test_log_rows_from_chunk_kernels_match_oracle(case):
    structure, K, B, L, uniform, mode = case
    d = 2 * K if structure == "planes" else K
    seed = 7 * K + L
    path, clock = _data(B, L, d, seed, uniform)
    gpu, ref = _params(structure, K, seed)
    kw = dict(leaf="plane_closed") if structure == "planes" else dict(leaf="series", series_q=24)
    layer = E.LogEWS(gpu, N=2, reweighting_mode=mode, **kw)
    print(f"log rows {structure} K={K} B={B} L={L} {mode}", flush=True)
    p = path.to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    out = layer(p, c, readout="prefix")
    ev[1].record()
    torch.cuda.synchronize()
    print(f"  forward {ev[0].elapsed_time(ev[1]):.3f} ms (first call)", flush=True)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    A = ref()
    oleaf = "plane_closed" if structure == "planes" else "series"
    want = torch.stack([O.log_ews_single(pr[b], cr[b], A, 2, "prefix", leaf=oleaf, series_q=24,
                                         reweighting_mode=mode, chen_expm="exact") for b in range(B)])
    assert out.shape == want.shape, (out.shape, want.shape)
    e = relerr(out, want)
    w = torch.tensor(np.random.default_rng(seed).normal(size=tuple(want.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (want * w).sum().backward()
    errs = [relerr(p.grad, pr.grad), relerr(c.grad, cr.grad)]
    errs += [relerr(g, h) for g, h in zip([q.grad for q in gpu.parameters()], [q.grad for q in ref.parameters()])]
    print(f"  forward {e:.2e}, gradients {['%.2e' % x for x in errs]}", flush=True)
    assert e < 1e-5, e
    assert max(errs) < 1e-4, errs


def test_log_rows_equal_rows_then_log():
    """c2's planes (d = 16) at B = 4, L = 3,000 and a real diagonal on explicit 32-step chunks: the fused log rows
    against the flat prefix rows followed by the separate log pass (ops.log_rows), forward and gradients."""
    for structure, K, chunk in (("planes", 8, 0), ("real_diag", 12, 32)):
        d = 2 * K if structure == "planes" else K
        path, clock = _data(4, 3000, d, 11, False)
        params = (torch.tensor(np.random.default_rng(5).uniform(0.1, 2.0, size=(K, 2)), dtype=torch.float32)
                  if structure == "planes" else
                  torch.tensor(np.random.default_rng(5).uniform(0.1, 2.0, size=K), dtype=torch.float32))
        outs, grads = [], []
        for fused in (True, False):
            p = path.to(DEV).requires_grad_(True)
            c = clock.to(DEV).requires_grad_(True)
            lam = params.to(DEV).requires_grad_(True)
            if fused:
                o = ops.diag_scan(p, c, lam, 2, structure, "per_interval", "log_prefix", False, chunk=chunk)
            else:
                rows = ops.diag_scan(p, c, lam, 2, structure, "per_interval", "prefix", True, chunk=chunk)
                o = ops.log_rows(rows, d, 2, True, "prefix")
            g = torch.tensor(np.random.default_rng(9).normal(size=tuple(o.shape)), dtype=torch.float32, device=DEV)
            (o * g).sum().backward()
            outs.append(o.detach())
            grads.append((p.grad, c.grad, lam.grad))
        e = relerr(outs[0], outs[1])
        errs = [relerr(a, b) for a, b in zip(grads[0], grads[1])]
        print(f"{structure} fused vs rows-then-log: forward {e:.2e}, gradients {['%.2e' % x for x in errs]}",
              flush=True)
        assert e < 1e-5 and max(errs) < 1e-4, (e, errs)
