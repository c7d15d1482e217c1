"""CPU pins of the block-front oracle (oracle/front_oracle.py): the clocks, the increment path, the lift and the
forward fill, against the reference's own clock and path tests (tests/test_clocks.py, tests/test_block.py:130-265,
tests/test_paths.py:72-85). Expected values are built by an independent route in numpy (np.diff / np.cumsum on
the real segment, the reference's numpy builder restated below, per-token closed forms), not by the oracle's
formulas."""

import numpy as np
import pytest
import torch

from oracle import front_oracle as FO

DT = torch.float64


def _rand(shape, seed):
    return np.random.default_rng(seed).normal(size=shape)


def _np_builder(t, p, mode, alpha, scaling):
    """The reference's numpy clock (ews/clocks.py:311-345 build_clock_np): per-sample scaling of each component,
    no epsilon, no mask. Written here as a second route to check the oracle against."""

    def sc(c):
        if scaling == "none":
            return c
        z = (c - c[0]) / ((c[-1] - c[0]) + 1e-12)
        return z if scaling == "[0,1]" else 2.0 * z - 1.0

    if mode == "time":
        return sc(np.asarray(t, float))
    dx = np.diff(p, axis=0)
    incr = np.sqrt((dx**2).sum(1)) if mode == "blended_variation" else (dx**2).sum(1)
    V = np.concatenate([[0.0], np.cumsum(incr)])
    return alpha * sc(np.asarray(t, float)) + (1.0 - alpha) * sc(V)


def _padded_driver(L_real, L_pad, c=2, seed=9, pad_value=5.0):
    real = _rand((L_real, c), seed)
    driver = np.concatenate([real, np.full((L_pad - L_real, c), pad_value)], 0)
    mask = np.zeros(L_pad, dtype=bool)
    mask[:L_real] = True
    return real, driver, mask


def _clock(t, driver, mode, alpha, scaling, mask=None, **kw):
    th = FO.build_clock(torch.tensor(t, dtype=DT), torch.tensor(driver, dtype=DT)[None], mode, alpha, scaling,
                        mask=None if mask is None else torch.tensor(mask)[None], **kw)
    return th[0].numpy()


@pytest.mark.parametrize("mode", ["time", "blended_variation", "blended_quad_variation"])
@pytest.mark.parametrize("scaling", ["none", "[0,1]", "[-1,1]"])
def test_builder_matches_numpy_route(mode, scaling):
    """tests/test_clocks.py:37-42 and tests/test_block.py:98-111: the numpy and jnp builders agree (eps = 0)."""
    t = np.arange(9.0)
    d = _rand((9, 3), 0)
    got = _clock(t, d, mode, 0.3, scaling, variation_eps=0.0)
    np.testing.assert_allclose(got, _np_builder(t, d, mode, 0.3, scaling), rtol=1e-12, atol=1e-12)


def test_mask_gating_hand_computed():
    """tests/test_block.py:203-232: quadratic variation on the real segment, the pad jump excluded, frozen pads."""
    L_real, L_pad, C, T = 4, 9, 3.0, 10.0
    real, driver, mask = _padded_driver(L_real, L_pad)
    times = np.arange(L_pad, dtype=float)
    got = _clock(times, driver, "blended_quad_variation", 0.5, "[0,1]", mask=mask, normalize="constant",
                 norm_constant=C, time_denominator=T)
    Q = np.concatenate([[0.0], np.cumsum((np.diff(real, axis=0) ** 2).sum(1))])
    np.testing.assert_allclose(got[:L_real], 0.5 * times[:L_real] / T + 0.5 * Q / C, rtol=1e-12)
    assert np.all(got[L_real:] == got[L_real - 1])


def test_per_sample_padded_matches_truncated():
    """tests/test_block.py:235-258: the masked clock on a padded sample equals the clock of the truncated one."""
    L_real, L_pad = 6, 13
    real, driver, mask = _padded_driver(L_real, L_pad, seed=10)
    truncated = _np_builder(np.arange(L_real, dtype=float), real, "blended_variation", 0.5, "[0,1]")
    padded = _clock(np.arange(L_pad, dtype=float), driver, "blended_variation", 0.5, "[0,1]", mask=mask,
                    variation_eps=0.0, time_denominator=float(L_real - 1))
    np.testing.assert_allclose(padded[:L_real], truncated, rtol=1e-10)
    np.testing.assert_allclose(padded[L_real:], np.full(L_pad - L_real, truncated[-1]), rtol=1e-10)


def test_time_mode_frozen_beyond_true_end():
    """tests/test_block.py:261-276."""
    _, driver, mask = _padded_driver(5, 12, seed=11)
    got = _clock(np.arange(12.0), driver, "time", 1.0, "[0,1]", mask=mask)
    assert np.all(got[5:] == got[4]) and np.all(np.diff(got[:5]) > 0)


def test_constant_dispatch_is_linear_in_the_constant():
    """tests/test_block.py:283-296: halving the variation's denominator doubles the variation part."""
    L = 9
    d = _rand((L, 2), 12)
    kw = dict(normalize="constant", time_denominator=float(L - 1))
    th1 = _clock(np.arange(L, dtype=float), d, "blended_variation", 0.5, "[0,1]", norm_constant=2.0, **kw)
    th2 = _clock(np.arange(L, dtype=float), d, "blended_variation", 0.5, "[0,1]", norm_constant=4.0, **kw)
    ts = np.arange(L) / (L - 1)
    np.testing.assert_allclose(th1 - 0.5 * ts, 2.0 * (th2 - 0.5 * ts), rtol=1e-10)


def test_steps_scaling_and_saturated_gate_are_the_sample_counter():
    """tests/test_clocks.py:127-151: scaling 'steps' is theta_i = i, and a clamped gate with every gate at its
    ceiling (w = 0, b = -2, K gates, norm_constant K) is the same clock."""
    t = np.linspace(0.0, 1.0, 7)
    assert np.array_equal(_clock(t, _rand((7, 3), 0), "time", 1.0, "steps"), np.arange(7.0))
    th = FO.gated_clock(torch.tensor(_rand((7, 3), 0))[None], "clamped_gate", torch.zeros(4, 3, dtype=DT),
                        torch.full((4,), -2.0, dtype=DT), 4.0)
    assert np.array_equal(th[0].numpy(), np.arange(7.0))


def test_gated_clock_formula_mask_and_monotone():
    """tests/test_clocks.py:45-64: relu(dx . w - b) cumulated over norm_constant; frozen pads; monotone."""
    rng = np.random.default_rng(1)
    d = _rand((9, 3), 0)
    w, b = rng.normal(size=3) / np.sqrt(3), -0.5
    got = FO.gated_clock(torch.tensor(d)[None], "token_gated", torch.tensor(w), torch.tensor(b), 4.0)[0].numpy()
    incr = np.maximum(np.diff(d, axis=0) @ w - b, 0.0)
    np.testing.assert_allclose(got, np.concatenate([[0.0], np.cumsum(incr)]) / 4.0, rtol=1e-12)
    mask = torch.arange(9) < 6
    th = FO.gated_clock(torch.tensor(d)[None], "token_gated", torch.tensor(w), torch.tensor(b), 4.0,
                        mask=mask[None])[0].numpy()
    assert np.all(th[6:] == th[5]) and np.all(np.diff(th) >= 0)
    # the driver is scaled before the difference (in_scale): same as scaling w in exact arithmetic
    th2 = FO.gated_clock(torch.tensor(d)[None], "token_gated", torch.tensor(w) * 3.0, torch.tensor(b), 4.0)
    th3 = FO.gated_clock(torch.tensor(d)[None], "token_gated", torch.tensor(w), torch.tensor(b), 4.0, in_scale=3.0)
    np.testing.assert_allclose(th2.numpy(), th3.numpy(), rtol=1e-12)


def test_per_token_increment_matches_increment_stream():
    """tests/test_clocks.py:81-96: on an increment stream of token rows, diff(theta) is each token's
    sqrt(|e|^2 + eps) / norm_constant."""
    embeds = _rand((5, 4), 3)
    ids = np.array([2, 0, 3, 3, 1])
    path = np.cumsum(embeds[ids], axis=0)
    th = _clock(np.arange(5.0), path, "blended_variation", 0.0, "none", normalize="constant", norm_constant=3.0)
    per_tok = np.sqrt((embeds**2).sum(1) + 1e-8) / 3.0
    np.testing.assert_allclose(np.diff(th), per_tok[ids[1:]], rtol=1e-9)


def test_variation_eps_gradient_guard_and_stop_gradient():
    """tests/test_block.py:150-188: zero increments give finite gradients with eps > 0 and non-finite ones with
    eps = 0; stop_gradient detaches the clock."""
    flat = torch.zeros((1, 5, 3), dtype=DT, requires_grad=True)
    t = torch.arange(5, dtype=DT)
    th = FO.build_clock(t, flat, "blended_variation", 0.5, "[0,1]", normalize="constant", norm_constant=1.0,
                        variation_eps=1e-8)
    (g,) = torch.autograd.grad(th.sum(), flat)
    assert torch.isfinite(g).all()
    th0 = FO.build_clock(t, flat, "blended_variation", 0.5, "[0,1]", normalize="constant", norm_constant=1.0,
                         variation_eps=0.0)
    (g0,) = torch.autograd.grad(th0.sum(), flat)
    assert not torch.isfinite(g0).all()
    d = torch.tensor(_rand((1, 7, 2), 8), requires_grad=True)
    assert not FO.build_clock(torch.arange(7, dtype=DT), d, "blended_variation", 0.5, "[0,1]",
                              stop_gradient=True).requires_grad


def test_learned_alpha_derivative_at_the_bounds():
    """jnp.clip = minimum(maximum(x, 0), 1) gives derivative 1/2 at a bound (a tie of max or min): the learned
    alpha of ews/clocks.py:502-506 initialised at 0 or 1 gets half the gradient. Checked on torch's own tie rule
    of maximum/minimum, which also splits evenly."""
    for x0, want in ((0.5, 1.0), (1.0, 0.5), (0.0, 0.5), (1.3, 0.0)):
        x = torch.tensor(x0, dtype=DT, requires_grad=True)
        torch.minimum(torch.maximum(x, torch.tensor(0.0, dtype=DT)), torch.tensor(1.0, dtype=DT)).backward()
        assert float(x.grad) == want, (x0, float(x.grad))


def test_increment_path_lift_and_fill():
    """tests/test_paths.py:72-85 (the increment path freezes past the mask), B (ews/params.py:1181-1191) against
    an explicit per-row product, and the forward fill + basepoint row of ews/block.py:295-301."""
    p = torch.tensor(_rand((1, 5, 2), 0))
    mask = torch.tensor([[True, True, True, False, False]])
    inc = FO.increment_path(p, mask)
    assert torch.equal(inc[0, 3], inc[0, 2]) and torch.equal(inc[0, 4], inc[0, 2])
    np.testing.assert_allclose(FO.increment_path(p, None)[0].numpy(), np.cumsum(p[0].numpy(), 0), rtol=1e-12)
    M = torch.tensor(_rand((4, 2), 1))
    u = torch.tensor(_rand((1, 5, 3), 2))
    lifted = FO.lift(u, M, True)
    for r in range(5):
        want = [float(u[0, r, 0])] + [float(sum(M[o, i] * u[0, r, 1 + i] for i in range(2))) for o in range(4)]
        np.testing.assert_allclose(lifted[0, r].numpy(), want, rtol=1e-12)
    full = FO.lift(u, torch.tensor(_rand((4, 3), 3)), False)
    assert full.shape == (1, 5, 4)
    filled = FO.forward_fill(lifted, mask)
    assert torch.equal(filled[0, 3], lifted[0, 2]) and torch.equal(filled[0, 4], lifted[0, 2])
    assert torch.equal(FO.forward_fill(lifted, torch.zeros_like(mask))[0, 0], lifted[0, 4])  # no real row
    theta = torch.tensor(_rand((1, 5), 4))
    pin, tin = FO.block_front(u[..., 1:], theta, u[..., 0], mask, M, True, False, True)
    assert pin.shape == (1, 6, 5) and float(pin[0, 0].abs().sum()) == 0.0
    assert float(tin[0, 0]) == float(tin[0, 1]) == float(theta[0, 0])
    assert torch.equal(pin[0, 1:], filled[0])
