"""GPU parity of the fused diagonal / rotation-plane scan against the float64 oracle.

Bars: forward max relative error <= 1e-5, gradients <= 1e-4, with the
reference's metric max|a-b| / max|b| (tests/test_engines.py:31-33). Cases mirror the reference's engine gates
(tests/test_engines.py:227-358): rotation planes and real diagonals, depths 1-2, every readout, the three
reweighting modes, both terminal reductions, single- and multi-chunk lengths, uniform clocks (first-order
coefficient models) and irregular clocks (exact per-step coefficients), float32 and bfloat16 paths.
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


def _planes_param(K, seed, scale=1.0):
    rng = np.random.default_rng(seed + 100)
    v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    return v, u, scale


def _layers(structure, K_or_d, N, seed, **kw):
    if structure == "planes":
        v, u, sc = _planes_param(K_or_d, seed)
        gpu = E.AParamDampedRotation(v.clone(), u.clone(), 2 * K_or_d, omega_scale=3.0).to(DEV)
        ref = E.AParamDampedRotation(v.double(), u.double(), 2 * K_or_d, omega_scale=3.0)
        leaf = "plane_closed"
        oleaf = "plane_closed"
    else:
        rng = np.random.default_rng(seed + 200)
        th = torch.tensor(rng.normal(size=K_or_d), dtype=torch.float32)
        gpu = E.AParamEFM(th.clone()).to(DEV)
        ref = E.AParamEFM(th.double())
        leaf = "series"
        oleaf = "series"  # the oracle's series leaf at the same order (q = 24)
    kwg = dict(kw)
    if leaf == "series":
        kwg["series_q"] = 24
    layer = E.EWS(gpu, N=N, leaf=leaf, **kwg)
    return layer, ref, oleaf


def _oracle(ref_param, path, clock, N, readout, oleaf, mode, terminal_reduce):
    A = ref_param()
    return O.ews(path, clock, A, N, readout, leaf=oleaf, reweighting_mode=mode, terminal_reduce=terminal_reduce,
                 chen_expm="exact", series_q=24)


CASES = [
    # structure, K/d, N, B, L, uniform
    ("planes", 3, 2, 2, 37, False),
    ("planes", 3, 2, 2, 300, True),
    ("planes", 8, 2, 2, 150, False),
    ("planes", 2, 1, 3, 90, True),
    ("real", 5, 2, 2, 160, False),
    ("real", 6, 1, 2, 40, True),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-K{c[1]}-N{c[2]}-L{c[4]}-{'u' if c[5] else 'nu'}" for c in CASES])
@pytest.mark.parametrize("readout", ["prefix", "terminal", "mean", "max"])
def test_forward_and_grads_match_oracle(case, readout):
    structure, K, N, B, L, uniform = case
    d = 2 * K if structure == "planes" else K
    seed = hash((structure, K, N, L, readout)) % 1000
    path, clock = _data(B, L, d, seed, uniform)
    layer, ref_param, oleaf = _layers(structure, K, N, seed, combine="block_kernel" if structure == "planes" else "assoc")
    p = path.to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    out = layer(p, c, readout=readout)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    ref = _oracle(ref_param, pr, cr, N, readout, oleaf, "displacement", "assoc")
    assert out.shape == ref.shape
    e = relerr(out, ref)
    assert e < 1e-5, f"forward relerr {e:.2e}"
    w = torch.tensor(np.random.default_rng(3).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    gp = relerr(p.grad, pr.grad)
    gc = relerr(c.grad, cr.grad)
    assert gp < 1e-4, f"path grad relerr {gp:.2e}"
    assert gc < 1e-4, f"clock grad relerr {gc:.2e}"
    for g_gpu, g_ref in zip([q.grad for q in layer.A_param.parameters()], [q.grad for q in ref_param.parameters()]):
        ga = relerr(g_gpu, g_ref)
        assert ga < 1e-4, f"A-param grad relerr {ga:.2e}"


@pytest.mark.parametrize("structure,K,steps", [("real", 32, "unit"), ("real", 32, "uniform"), ("real", 16, "unit"),
                                               ("planes", 16, "uniform"), ("planes", 16, "unit"),
                                               ("planes", 12, "uniform"), ("planes", 12, "unit")])
@pytest.mark.parametrize("readout", ["prefix", "mean"])
def test_wide_states(structure, K, steps, readout):
    """The widths of BASELINE.json configs[3] (d = 32 real diagonal) and configs[4] (d = 24, 12 planes) at depth 2,
    and 16 diagonal entries or planes (K = 32 runs the lane all-reduce of the row and column sums, K = 16 and 12 the
    LDS partial sums).
    Unit clock steps (the block default clock arange(L)) contract a chunk too much to invert its steps, so the
    adjoint recomputes the states from checkpoints; at d = 32 the plan shortens the checkpoint block to fit LDS."""
    N, B, L = 2, 2, 70
    d = 2 * K if structure == "planes" else K
    path, clock = _data(B, L, d, 21 + K, True)
    if steps == "unit":
        clock = torch.arange(L, dtype=torch.float32).expand(B, L).contiguous()
    layer, ref_param, oleaf = _layers(structure, K, N, 9, combine="block_kernel" if structure == "planes" else "assoc")
    p = path.to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    out = layer(p, c, readout=readout)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    ref = _oracle(ref_param, pr, cr, N, readout, oleaf, "displacement", "assoc")
    e = relerr(out, ref)
    assert e < 1e-5, f"forward relerr {e:.2e}"
    w = torch.tensor(np.random.default_rng(8).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    assert relerr(p.grad, pr.grad) < 1e-4, relerr(p.grad, pr.grad)
    assert relerr(c.grad, cr.grad) < 1e-4, relerr(c.grad, cr.grad)
    for g_gpu, g_ref in zip([q.grad for q in layer.A_param.parameters()], [q.grad for q in ref_param.parameters()]):
        assert relerr(g_gpu, g_ref) < 1e-4, relerr(g_gpu, g_ref)


@pytest.mark.parametrize("mode", ["displacement_uniform", "displacement_uniform_basepoint"])
@pytest.mark.parametrize("readout,reduce", [("prefix", "assoc"), ("terminal", "tree"), ("terminal", "assoc"),
                                            ("mean", "tree")])
def test_reweighting_modes(mode, readout, reduce):
    K, N, B, L = 3, 2, 2, 140
    path, clock = _data(B, L, 2 * K, 11, True)
    if mode.endswith("basepoint"):
        clock[:, 1:] = clock[:, :-1].clone()  # clock[0] == clock[1]: a dt = 0 basepoint interval
        path[:, 0] = path[:, 1]
    layer, ref_param, oleaf = _layers("planes", K, N, 5, reweighting_mode=mode, terminal_reduce=reduce)
    p = path.to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    out = layer(p, c, readout=readout)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    ref = _oracle(ref_param, pr, cr, N, readout, oleaf, mode, reduce)
    assert relerr(out, ref) < 1e-5
    w = torch.tensor(np.random.default_rng(4).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    assert relerr(p.grad, pr.grad) < 1e-4
    assert relerr(c.grad, cr.grad) < 1e-4
    for g_gpu, g_ref in zip([q.grad for q in layer.A_param.parameters()], [q.grad for q in ref_param.parameters()]):
        assert relerr(g_gpu, g_ref) < 1e-4


def test_list_output_and_single_path():
    K, N, L = 2, 2, 50
    path, clock = _data(1, L, 2 * K, 2, False)
    layer, ref_param, oleaf = _layers("planes", K, N, 1)
    lv = layer(path[0].to(DEV), clock[0].to(DEV), readout="prefix", output_format="list")
    ref = O.ews_single(path[0].double(), clock[0].double(), ref_param().detach(), N, "prefix", leaf=oleaf,
                       output_format="list")
    assert [tuple(x.shape) for x in lv] == [(L - 1, 2 * K), (L - 1, 2 * K, 2 * K)]
    for a, b in zip(lv, ref):
        assert relerr(a, b) < 1e-5
    term = layer(path[0].to(DEV), clock[0].to(DEV))  # default readout: terminal, flat with level 0
    assert term.shape == (1 + 2 * K + 4 * K * K,) and float(term[0]) == 1.0


def test_bf16_path_input():
    K, N, B, L = 4, 2, 2, 120
    path, clock = _data(B, L, 2 * K, 9, True)
    pb = path.to(torch.bfloat16)
    layer, ref_param, oleaf = _layers("planes", K, N, 2)
    out = layer(pb.to(DEV), clock.to(DEV), readout="prefix")
    ref = _oracle(ref_param, pb.double(), clock.double(), N, "prefix", oleaf, "displacement", "assoc")
    assert relerr(out, ref) < 1e-5  # same bf16 inputs upcast on both sides


def test_log_ews_depth2():
    K, B, L = 3, 2, 80
    path, clock = _data(B, L, 2 * K, 21, False)
    v, u, _ = _planes_param(K, 21)
    A = E.AParamDampedRotation(v.clone(), u.clone(), 2 * K).to(DEV)
    log_layer = E.LogEWS(A, N=2, leaf="plane_closed")
    Aref = E.AParamDampedRotation(v.double(), u.double(), 2 * K)().detach()
    for readout in ("terminal", "prefix", "mean", "max"):
        got = log_layer(path.to(DEV), clock.to(DEV), readout=readout)
        ref = torch.stack([O.log_ews_single(path[b].double(), clock[b].double(), Aref, 2, readout,
                                            leaf="plane_closed") for b in range(B)])
        assert got.shape == ref.shape
        assert relerr(got, ref) < 1e-5, readout


def test_forward_graph_replay_matches_eager():
    """The forward passes captured as a HIP graph (torch.cuda.CUDAGraph over the library's launches) and replayed
    several times, with eager work and synchronisations in between: every replay equals the eager result exactly
    (the kernels record no memset and no host synchronisation)."""
    B, L, d = 8, 1024, 8
    rng = np.random.default_rng(31)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.05, 1), dtype=torch.float32, device=DEV)
    clock = torch.tensor(np.broadcast_to(np.arange(L) / L, (B, L)).copy(), dtype=torch.float32, device=DEV)
    lam = torch.tensor(rng.uniform(0.1, 2.0, d), dtype=torch.float32, device=DEV)
    eager = ops.diag_scan(path, clock, lam, 2, "real_diag", "per_interval", "prefix", True)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm up on a side stream, as graph capture asks
        ops.diag_scan(path, clock, lam, 2, "real_diag", "per_interval", "prefix", True)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.diag_scan(path, clock, lam, 2, "real_diag", "per_interval", "prefix", True)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        _ = (path * 2.0).sum().item()  # eager work between the replays
