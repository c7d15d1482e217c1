"""Pins the float64 mixer-epilogue oracle (oracle/mixer_oracle.py) to the reference's own tests of the
GradedRMSNorm and the block prescale (tests/test_block.py:301-415, ews/block.py:336-357), and checks the product's
GradedRMSNorm module (its plain-torch forward, used on flat graded tensors) against it. CPU only."""

import math

import numpy as np
import pytest
import torch

import ews_mi355x as E
from oracle import mixer_oracle as MO

DT = torch.float64


def _rand(shape, seed):
    return torch.tensor(np.random.default_rng(seed).normal(size=shape), dtype=DT)


def test_level_slices_level0_free():  # tests/test_block.py:301-303
    assert MO.level_slices(3, 2) == [(0, 3), (3, 12)]
    assert MO.level_slices(2, 3) == [(0, 2), (2, 6), (6, 14)]


def test_live_rms_unit_rms_per_level():  # tests/test_block.py:323-333
    d, n, L = 3, 3, 7
    D = sum(d**k for k in range(1, n + 1))
    x = _rand((L, D), 22)
    for k, (s, e) in enumerate(MO.level_slices(d, n)):
        x[:, s:e] *= 10.0 ** (-2 * k)
    y = MO.graded_rms_norm(x, d, n, "live_rms", (0.0,) * n, gains=torch.ones(n, dtype=DT))
    np.testing.assert_allclose(MO.per_level_rms(y, d, n).numpy(), np.ones((L, n)), rtol=1e-10)


def test_dilation_exact():  # tests/test_block.py:361-372
    d, n = 2, 3
    x = _rand((4, 14), 24)
    y = MO.graded_rms_norm(x, d, n, "dilation", (1e-3,) * n, lam=torch.tensor(1.7, dtype=DT))
    for k, (s, e) in enumerate(MO.level_slices(d, n)):
        np.testing.assert_allclose(y[:, s:e].numpy(), 1.7 ** (k + 1) * x[:, s:e].numpy(), rtol=1e-12)


def test_zero_input_safe_and_eps_floor():  # tests/test_block.py:375-397
    d, n = 3, 2
    zeros = torch.zeros((4, 12), dtype=DT, requires_grad=True)
    g = torch.ones(n, dtype=DT)
    y = MO.graded_rms_norm(zeros, d, n, "live_rms", (1e-3,) * n, gains=g)
    assert torch.equal(y, torch.zeros_like(y))
    (y**2).sum().backward()
    assert torch.isfinite(zeros.grad).all()
    base = _rand((5, 6), 25)
    norms = [float(MO.graded_rms_norm(s * base, 2, 2, "live_rms", (1e-3,) * 2, gains=torch.ones(2, dtype=DT)).norm())
             for s in (1.0, 1e-2, 1e-4, 0.0)]
    assert norms[0] > norms[1] > norms[2] > norms[3] == 0.0


def test_gains_and_lam_receive_gradient():  # tests/test_block.py:336-358
    x = _rand((6, 14), 23)
    g = torch.ones(3, dtype=DT, requires_grad=True)
    (MO.graded_rms_norm(x, 2, 3, "live_rms", (1e-3,) * 3, gains=g) ** 2).sum().backward()
    assert (g.grad != 0).all() and torch.isfinite(g.grad).all()
    lam = torch.tensor(1.0, dtype=DT, requires_grad=True)
    (MO.graded_rms_norm(x, 2, 3, "dilation", (1e-3,) * 3, lam=lam) ** 2).sum().backward()
    assert lam.grad != 0 and torch.isfinite(lam.grad)


def test_binomial_prescale_is_inverse_binomial():  # ews/block.py:336-357 against exact binomials
    d, n, L = 2, 3, 9
    ones = torch.ones((L, 14), dtype=DT)
    got = MO.binomial_prescale(ones, d, n)
    for k, (s, e) in enumerate(MO.level_slices(d, n), start=1):
        for t in range(L):
            want = 1.0 / math.comb(max(t + 1, k), k)
            np.testing.assert_allclose(got[t, s:e].numpy(), want, rtol=1e-12)


def test_levels_from_flat_drops_level0_and_prepends_zero_row():  # ews/block.py:302-305
    flat = _rand((2, 4, 1 + 6), 3)
    lv = MO.levels_from_flat(flat, basepoint=False)
    assert lv.shape == (2, 5, 6) and torch.equal(lv[:, 0], torch.zeros(2, 6)) and torch.equal(lv[:, 1:], flat[..., 1:])
    assert torch.equal(MO.levels_from_flat(flat, basepoint=True), flat[..., 1:])


@pytest.mark.parametrize("variant", ["live_rms", "static_gain", "dilation"])
def test_product_graded_module_matches_oracle(variant):
    d, n = 3, 2
    m = E.GradedRMSNorm(d, n, variant=variant, eps=(1e-3, 2e-3), dtype=DT)
    with torch.no_grad():
        if variant == "dilation":
            m.lam.fill_(1.3)
        else:
            m.gains.copy_(torch.tensor([0.7, 1.9], dtype=DT))
    x = _rand((5, 12), 8)
    x[2, :3] = 0.0  # an all-zero level
    want = MO.graded_rms_norm(x, d, n, variant, (1e-3, 2e-3), gains=m.gains, lam=m.lam)
    assert torch.equal(m(x), want)
    np.testing.assert_allclose(m.per_level_rms(x).numpy(), MO.per_level_rms(x, d, n).numpy(), rtol=1e-15)
