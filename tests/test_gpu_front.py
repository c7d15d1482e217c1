"""GPU parity of the block-front kernels (csrc/ews_front.hip: clocks and lift) against the float64 oracle
(oracle/front_oracle.py, pinned in tests/test_oracle_front.py to the reference's clock and path tests).

Bars: forward max relative error <= 1e-5, gradients <= 1e-4, metric max|a-b| / max|b|
(the reference's tests/test_engines.py:31-33). Cases cover the six clock modes, every scaling and normalisation,
time denominators, learned alpha at an interior point and at a bound (the half derivative of jnp.clip), both
alpha parametrisations, masks of different lengths per sample (including a sample with one real row and one with
none), increment drivers, the basepoint copy, chunk edges (L = 1, 2, 256, 257) and a long sample (L = 49,920)
for the float64 chunk carries; the lift with and without B, the preserved first channel, the appended clock
channel, the increment path, the forward fill and the basepoint row; and the chain front -> EWS scan with
gradients to the block inputs, B and the clock parameters.
"""

import numpy as np
import pytest
import torch

import ews_mi355x as E
from oracle import ews_oracle as O
from oracle import front_oracle as FO

pytestmark = pytest.mark.gpu

DEV = "cuda"
DT = torch.float64


def relerr(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-300))


def _mask(B, L, lens):
    m = torch.zeros(B, L, dtype=torch.bool)
    for i, n in enumerate(lens):
        m[i, :n] = True
    return m


def _oracle_theta(clk, t, x, mask, increment, basepoint, w=None, b=None, araw=None):
    s = clk.spec
    drv = FO.increment_path(x, mask) if increment else x
    if s.mode in ("token_gated", "clamped_gate"):
        th = FO.gated_clock(drv, s.mode, w, b, s.norm_constant, in_scale=s.gate_in_scale, mask=mask)
    else:
        alpha = FO.learned_alpha(araw, s.alpha_parametrisation) if s.mode == "blended_learn" else s.alpha
        mode = "blended_variation" if s.mode == "blended_learn" else s.mode
        th = FO.build_clock(t, drv, mode, alpha, s.scaling, mask=mask, normalize=s.normalize,
                            norm_constant=s.norm_constant, time_denominator=s.time_denominator,
                            variation_eps=s.variation_eps)
    if basepoint:
        th = torch.cat([th[:, :1], th], 1)
    return th


CLOCKS = [
    # name, spec kwargs, c
    ("time01", dict(mode="time"), 3),
    ("time-sym-tden", dict(mode="time", scaling="[-1,1]", time_denominator=37.0), 3),
    ("time-steps", dict(mode="time", scaling="steps"), 3),
    ("var01", dict(mode="blended_variation", alpha=0.3), 6),
    ("var-none", dict(mode="blended_variation", alpha=0.0, scaling="none"), 6),
    ("var-sym", dict(mode="blended_variation", alpha=0.6, scaling="[-1,1]"), 5),
    ("var-const", dict(mode="blended_variation", alpha=0.5, normalize="constant", norm_constant=7.0,
                       time_denominator=300.0), 8),
    ("quad01", dict(mode="blended_quad_variation", alpha=0.25), 4),
    ("quad-const-sym", dict(mode="blended_quad_variation", alpha=0.2, scaling="[-1,1]", normalize="constant",
                            norm_constant=50.0), 16),
    ("learn-clip", dict(mode="blended_learn", alpha=0.4), 6),
    ("learn-clip-bound", dict(mode="blended_learn", alpha=1.0), 6),
    ("learn-sigmoid", dict(mode="blended_learn", alpha=0.7, alpha_parametrisation="sigmoid"), 3),
    ("token", dict(mode="token_gated", scaling="none", normalize="constant", norm_constant=4.0,
                   gate_init_bias=0.1, gate_in_scale=2.0), 6),
    ("clamped", dict(mode="clamped_gate", scaling="none", normalize="constant", norm_constant=3.0,
                     gate_init_bias=(-0.2, 0.1, 0.4)), 5),
    ("clamped-wide", dict(mode="clamped_gate", scaling="none", normalize="constant", norm_constant=8.0,
                          gate_K=8, gate_init_bias=0.05), 40),
]

SETTINGS = [
    # B, L, mask lengths (None: no mask), increment driver, basepoint
    (3, 700, None, False, False),
    (3, 700, (700, 401, 1), False, True),
    (3, 513, (513, 300, 0), True, False),
    (2, 257, (257, 256), True, True),
]


@pytest.mark.parametrize("setting", SETTINGS, ids=[f"B{s[0]}-L{s[1]}-{'mask' if s[2] else 'nomask'}-"
                                                   f"{'incr' if s[3] else 'value'}-{'bp' if s[4] else 'nobp'}"
                                                   for s in SETTINGS])
@pytest.mark.parametrize("case", CLOCKS, ids=[c[0] for c in CLOCKS])
def test_clock_forward_and_grads_match_oracle(case, setting):
    name, kw, c = case
    B, L, lens, incr, bp = setting
    rng = np.random.default_rng(sum(map(ord, name)) * 1000 + L)
    clk = E.make_clock(E.ClockSpec(**kw), dim=c, key=5)
    x = torch.tensor(rng.normal(size=(B, L, c)) * 0.3, dtype=torch.float32)
    t = torch.tensor(np.cumsum(rng.uniform(0.5, 1.5, size=L)), dtype=torch.float32)
    mask = None if lens is None else _mask(B, L, lens)
    clk = clk.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    th = clk(t.to(DEV), xg, None if mask is None else mask.to(DEV), increment_driver=incr, basepoint=bp)
    assert th.shape == (B, L + int(bp))
    xr = x.double().requires_grad_(True)
    w = b = araw = None
    if kw["mode"] in ("token_gated", "clamped_gate"):
        w = clk.w.detach().cpu().double().requires_grad_(True)
        b = clk.b.detach().cpu().double().requires_grad_(True)
    if kw["mode"] == "blended_learn":
        araw = clk.alpha_raw.detach().cpu().double().requires_grad_(True)
    ref = _oracle_theta(clk, t.double(), xr, mask, incr, bp, w, b, araw)
    e = relerr(th, ref)
    assert e < 1e-5, f"theta relerr {e:.2e}"
    if kw["mode"] == "time":
        return
    cot = torch.tensor(np.random.default_rng(3).normal(size=tuple(ref.shape)))
    (th * cot.to(DEV, torch.float32)).sum().backward()
    (ref * cot).sum().backward()
    ex = relerr(xg.grad, xr.grad)
    assert ex < 1e-4, f"driver grad relerr {ex:.2e}"
    if w is not None:
        assert relerr(clk.w.grad, w.grad) < 1e-4, relerr(clk.w.grad, w.grad)
        assert relerr(clk.b.grad, b.grad) < 1e-4, relerr(clk.b.grad, b.grad)
    if araw is not None:
        assert relerr(clk.alpha_raw.grad, araw.grad) < 1e-4, (float(clk.alpha_raw.grad), float(araw.grad))


def test_clock_long_sample_and_short_edges():
    """L = 49,920 (195 chunks: float64 carries) with a mask, and L = 1, 2 (no or one increment)."""
    for L, lens in ((49920, (49920, 31111)), (1, (1, 0)), (2, (2, 1))):
        rng = np.random.default_rng(L)
        clk = E.make_clock(E.ClockSpec(mode="blended_variation", alpha=0.2), dim=6).to(DEV)
        x = torch.tensor(rng.normal(size=(2, L, 6)) * 0.05, dtype=torch.float32)
        t = torch.linspace(0.0, 1.0, L) if L > 1 else torch.zeros(1)
        mask = _mask(2, L, lens)
        xg = x.to(DEV).requires_grad_(True)
        th = clk(t.to(DEV), xg, mask.to(DEV))
        xr = x.double().requires_grad_(True)
        ref = _oracle_theta(clk, t.double(), xr, mask, False, False)
        assert relerr(th, ref) < 1e-5, (L, relerr(th, ref))
        cot = torch.tensor(np.random.default_rng(4).normal(size=tuple(ref.shape)))
        (th * cot.to(DEV, torch.float32)).sum().backward()
        (ref * cot).sum().backward()
        if float(xr.grad.abs().max()) > 0:
            assert relerr(xg.grad, xr.grad) < 1e-4, (L, relerr(xg.grad, xr.grad))
        else:
            assert float(xg.grad.abs().max()) == 0.0


LIFTS = [
    # H, append, out (None: no B), preserve, increment, mask lengths, basepoint
    (6, False, 16, False, False, None, False),
    (6, False, 16, False, True, (300, 177, 0), True),
    (5, True, 9, True, False, (300, 120, 1), False),
    (8, True, 17, True, True, (300, 300, 64), True),
    (32, False, 32, False, True, (300, 290, 5), False),
    (64, True, 64, True, False, None, True),
    (3, True, None, False, False, (300, 150, 2), True),
    (12, False, 20, False, False, (300, 129, 128), False),
]


@pytest.mark.parametrize("case", LIFTS, ids=[f"H{c[0]}-{'app' if c[1] else 'noapp'}-w{c[2]}-"
                                             f"{'pres' if c[3] else 'full'}-{'incr' if c[4] else 'value'}-"
                                             f"{'mask' if c[5] else 'nomask'}-{'bp' if c[6] else 'nobp'}"
                                             for c in LIFTS])
def test_lift_forward_and_grads_match_oracle(case):
    H, app, out, pres, incr, lens, bp = case
    B, L = 3, 300
    rng = np.random.default_rng(H * 7 + int(app))
    Hin = H + int(app)
    layer = None
    M = None
    if out is not None:
        M = torch.tensor(rng.normal(size=(out - 1, Hin - 1) if pres else (out, Hin)) / np.sqrt(Hin),
                         dtype=torch.float32)
        layer = E.B(M, preserve_first_channel=pres).to(DEV)
    br = torch.tensor(rng.normal(size=(B, L, H)), dtype=torch.float32)
    tha = torch.tensor(np.cumsum(rng.uniform(size=(B, L)), 1) / L, dtype=torch.float32) if app else None
    mask = None if lens is None else _mask(B, L, lens)
    bg = br.to(DEV).requires_grad_(True)
    tg = tha.to(DEV).requires_grad_(True) if app else None
    p = E.lift_path(bg, tg, layer, None if mask is None else mask.to(DEV), increment=incr, basepoint=bp)
    brr = br.double().requires_grad_(True)
    thr = tha.double().requires_grad_(True) if app else None
    Mr = M.double().requires_grad_(True) if M is not None else None
    ref, _ = FO.block_front(brr, torch.zeros(B, L, dtype=DT), thr, mask, Mr, pres, incr, bp)
    assert p.shape == ref.shape
    assert relerr(p, ref) < 1e-5, relerr(p, ref)
    cot = torch.tensor(np.random.default_rng(9).normal(size=tuple(ref.shape)))
    (p * cot.to(DEV, torch.float32)).sum().backward()
    (ref * cot).sum().backward()
    assert relerr(bg.grad, brr.grad) < 1e-4, relerr(bg.grad, brr.grad)
    if app:
        assert relerr(tg.grad, thr.grad) < 1e-4, relerr(tg.grad, thr.grad)
    if M is not None:
        assert relerr(layer.matrix.grad, Mr.grad) < 1e-4, relerr(layer.matrix.grad, Mr.grad)


def test_front_then_scan_chain():
    """BlockFront (gated clock on the increment driver, appended time clock, B with the preserved clock channel,
    mask, basepoint) into the EWS scan (rotation planes, d = 16, depth 2), gradients to the branch, the driver, B
    and the gate, against the oracle front followed by the oracle scan."""
    B, L, H, K = 2, 200, 6, 8
    rng = np.random.default_rng(21)
    clock = E.make_clock(E.ClockSpec(mode="token_gated", scaling="none", normalize="constant", norm_constant=2.0,
                                     gate_init_bias=-0.3), dim=H, key=3)
    app = E.make_clock(E.ClockSpec(mode="time", scaling="[0,1]"), dim=H)
    M = torch.tensor(rng.normal(size=(2 * K - 1, H)) / np.sqrt(H), dtype=torch.float32)
    front = E.BlockFront(clock, E.B(M, preserve_first_channel=True), app, path_mode="increment",
                         basepoint=True).to(DEV)
    v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    layer = E.EWS(E.AParamDampedRotation(v.clone(), u.clone(), 2 * K, omega_scale=3.0), N=2,
                  leaf="plane_closed").to(DEV)
    x = torch.tensor(rng.normal(size=(B, L, H)) * 0.2, dtype=torch.float32)
    mask = _mask(B, L, (L, 150))
    xg = x.to(DEV).requires_grad_(True)
    path, theta = front(xg, xg, mask=mask.to(DEV))
    out = layer(path, theta, readout="prefix")
    # oracle
    xr = x.double().requires_grad_(True)
    w = clock.w.detach().cpu().double().requires_grad_(True)
    b = clock.b.detach().cpu().double().requires_grad_(True)
    Mr = M.double().requires_grad_(True)
    t = torch.arange(L, dtype=DT)
    drv = FO.increment_path(xr, mask)
    th = FO.gated_clock(drv, "token_gated", w, b, 2.0, mask=mask)
    tha = FO.build_clock(t, drv, "time", 1.0, "[0,1]", mask=mask)
    pin, thin = FO.block_front(xr, th, tha, mask, Mr, True, True, True)
    assert relerr(path, pin) < 1e-5 and relerr(theta, thin) < 1e-5
    ref_param = E.AParamDampedRotation(v.double(), u.double(), 2 * K, omega_scale=3.0)
    ref = O.ews(pin, thin, ref_param(), 2, "prefix", leaf="plane_closed", reweighting_mode="displacement",
                terminal_reduce="assoc", chen_expm="exact")
    assert relerr(out, ref) < 1e-5, relerr(out, ref)
    cot = torch.tensor(np.random.default_rng(2).normal(size=tuple(ref.shape)))
    (out * cot.to(DEV, torch.float32)).sum().backward()
    (ref * cot).sum().backward()
    assert relerr(xg.grad, xr.grad) < 1e-4, relerr(xg.grad, xr.grad)
    assert relerr(front.b_layer.matrix.grad, Mr.grad) < 1e-4, relerr(front.b_layer.matrix.grad, Mr.grad)
    assert relerr(clock.w.grad, w.grad) < 1e-4 and relerr(clock.b.grad, b.grad) < 1e-4
