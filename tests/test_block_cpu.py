"""CPU checks of the block and stack modules (ews_mi355x.block, no kernel calls) and of their float64 checker
(oracle/block_oracle.py).

- Constructor checks and errors as the reference's (ews/block.py:134-145, 523-528, 571-574), the reference's field
  names (a checkpoint converted key by key lands in the same places), the lift width rule (m, plus a preserved
  clock channel when a clock is appended: ews/block.py:176-195).
- AParamDefinitePlusSkew (ews/params.py:152-163, 372-391) against a brute-force fill of the triangles and its
  invariants (symmetric part L L^T + eps I, antisymmetric part U - U^T).
- The checker's pieces against independent implementations (torch's tanh-approximate GELU and LayerNorm) and its
  composition against what the block's algebra fixes: with c_down and the channel stage zeroed, a "pre" block is
  the identity and a "slice_post" block is the LayerNorm of its input; a block with the mixer zeroed adds exactly
  its channel stage of the normed input.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ews_mi355x as E
from oracle import block_oracle as BO

DT = torch.float64


def test_constructor_errors():
    with pytest.raises(ValueError, match="norm_placement"):
        E.EWSBlock(8, norm_placement="post")
    with pytest.raises(ValueError, match="channel_stage"):
        E.EWSBlock(8, channel_stage="swiglu")
    with pytest.raises(ValueError, match="graded_prescale"):
        E.EWSBlock(8, graded_prescale="poisson")
    with pytest.raises(ValueError, match="path_mode"):
        E.EWSBlock(8, path_mode="delta")
    with pytest.raises(ValueError, match="ff_mult"):
        E.EWSBlock(8, ff_mult=0)
    with pytest.raises(ValueError, match="num_blocks"):
        E.StackedEWS(0, 4, 8, 2)
    with pytest.raises(ValueError, match="head_mode"):
        E.StackedEWS(1, 4, 8, 2, head_mode="last")
    with pytest.raises(ValueError, match="per_block_kwargs"):
        E.StackedEWS(2, 4, 8, 2, per_block_kwargs=[{}])
    with pytest.raises(TypeError, match="label_dim"):
        E.StackedEWS(1, 4, 8, [2])
    with pytest.raises(ValueError, match="width"):
        E.EWSBlock(8, m=4, a_param=E.AParamEFM(torch.zeros(5)))


def test_fields_and_widths():
    blk = E.EWSBlock(10, m=6, n=2, channel_stage="mlp", output_gate=True, key=1)
    names = {n for n, _ in blk.named_parameters()}
    for want in ("norm1.weight", "norm2.weight", "ff1.weight", "ff2.weight", "gate.weight", "b_layer.matrix",
                 "mixer.c_down.weight", "mixer.graded.gains", "ewms.A_param.lower", "ewms.A_param.upper"):
        assert want in names, want
    assert blk.c_down is blk.mixer.c_down and blk.graded is blk.mixer.graded
    assert blk.w_eff == 6 and blk.D == 6 + 36
    assert tuple(blk.c_down.weight.shape) == (10, 42)
    # an appended clock adds a preserved channel: lift (m, H) on the branch, w = m + 1
    blk2 = E.EWSBlock(10, m=6, n=1, append_clock=dict(mode="time"), key=2)
    assert blk2.w_eff == 7 and tuple(blk2.b_layer.matrix.shape) == (6, 10) and blk2.b_layer.preserve_first_channel
    blk3 = E.EWSBlock(10, m=6, n=1, lift=False, key=3)
    assert blk3.b_layer is None and blk3.w_eff == 10
    assert E.EWSBlock(10, norm_placement="slice_post").norm1 is None
    stk = E.StackedEWS(2, 5, 8, (3, 2), tokens=False, key=4)
    assert isinstance(stk.head, torch.nn.ModuleList) and len(stk.head) == 2


def test_definite_plus_skew_layout_and_invariants():
    n, eps = 5, 0.3
    rng = np.random.default_rng(0)
    lower = torch.tensor(rng.normal(size=n * (n + 1) // 2))
    upper = torch.tensor(rng.normal(size=n * (n - 1) // 2))
    A = E.AParamDefinitePlusSkew(lower, upper, n, eps)().detach()
    Lm = np.zeros((n, n))
    Um = np.zeros((n, n))
    k = 0
    for i in range(n):          # jnp.tril_indices: row-major over the lower triangle
        for j in range(i + 1):
            Lm[i, j] = lower[k]
            k += 1
    k = 0
    for i in range(n):          # jnp.triu_indices(k=1): row-major over the strict upper triangle
        for j in range(i + 1, n):
            Um[i, j] = upper[k]
            k += 1
    want = Lm @ Lm.T + eps * np.eye(n) + Um - Um.T
    assert np.allclose(A.numpy(), want, atol=1e-12)
    sym = 0.5 * (A + A.t())
    assert float(torch.linalg.eigvalsh(sym).min()) >= eps - 1e-12
    assert torch.allclose(0.5 * (A - A.t()), torch.tensor(Um - Um.T), atol=1e-12)
    with pytest.raises(ValueError):
        E.AParamDefinitePlusSkew(lower[:-1], upper, n)


def test_oracle_pieces_match_independent_implementations():
    x = torch.linspace(-6, 6, 301, dtype=DT)
    assert torch.allclose(BO.gelu(x), F.gelu(x, approximate="tanh"), atol=1e-14)
    y = torch.randn(4, 7, dtype=DT)
    w, b = torch.randn(7, dtype=DT), torch.randn(7, dtype=DT)
    assert torch.allclose(BO.layer_norm(y, w, b, 1e-6), F.layer_norm(y, (7,), w, b, 1e-6), atol=1e-12)
    r = BO.rms_norm(y, torch.ones(7, dtype=DT), 0.0)
    assert torch.allclose((r * r).mean(-1), torch.ones(4, dtype=DT), atol=1e-12)


def _params(H, m, N, stage, rng, zero_mix=False, zero_channel=False, slice_post=False):
    D = sum(m**k for k in range(1, N + 1))
    P = {"blocks.0.b_layer.matrix": torch.tensor(rng.normal(size=(m, H)) / math.sqrt(H)),
         "blocks.0.mixer.graded.gains": torch.ones(N, dtype=DT),
         "blocks.0.mixer.c_down.weight": torch.zeros(H, D, dtype=DT) if zero_mix else
         torch.tensor(rng.normal(size=(H, D)) * 0.1),
         "blocks.0.mixer.c_down.bias": torch.zeros(H, dtype=DT) if zero_mix else torch.tensor(rng.normal(size=H)),
         "blocks.0.norm1.weight": torch.tensor(rng.uniform(0.5, 1.5, size=H)),
         "blocks.0.norm2.weight": torch.tensor(rng.uniform(0.5, 1.5, size=H))}
    if slice_post:
        P["blocks.0.norm2.bias"] = torch.tensor(rng.normal(size=H))
    widths = {"mlp": [(4 * H, H), (H, 4 * H)], "glu": [(2 * H, H)], "tanh": [(H, H)], "gelu_glu": [(H, H), (H, H)]}
    for k, (o, i) in enumerate(widths[stage]):
        P[f"blocks.0.ff{k + 1}.weight"] = torch.zeros(o, i, dtype=DT) if zero_channel else torch.tensor(
            rng.normal(size=(o, i)) / math.sqrt(i))
        P[f"blocks.0.ff{k + 1}.bias"] = torch.zeros(o, dtype=DT) if zero_channel else torch.tensor(
            rng.normal(size=o) * 0.1)
    return P


def test_oracle_block_algebra():
    rng = np.random.default_rng(3)
    H, m, N, Bn, L = 6, 3, 2, 2, 9
    x = torch.tensor(rng.normal(size=(Bn, L, H)))
    t = torch.arange(L, dtype=DT)
    lam = torch.tensor(rng.uniform(0.2, 1.5, size=m))
    A_fn = lambda P: torch.diag(lam)  # noqa: E731
    layer = dict(leaf="series", series_q=12)
    # mixer and channel zeroed: a pre block is the identity
    for stage in ("mlp", "glu", "tanh"):
        P = _params(H, m, N, stage, rng, zero_mix=True, zero_channel=True)
        y = BO.block(x, P, "blocks.0.", dict(n=N, channel_stage=stage, layer=layer), A_fn, t)
        assert torch.allclose(y, x, atol=1e-14)
    # slice_post with the mixer and the channel zeroed: LayerNorm of the input
    P = _params(H, m, N, "tanh", rng, zero_mix=True, zero_channel=True, slice_post=True)
    y = BO.block(x, P, "blocks.0.", dict(n=N, channel_stage="tanh", norm_placement="slice_post", layer=layer),
                 A_fn, t)
    assert torch.allclose(y, F.layer_norm(x, (H,), P["blocks.0.norm2.weight"], P["blocks.0.norm2.bias"], 1e-6),
                          atol=1e-12)
    # mixer zeroed, channel live: x + channel(RMSNorm2(x))
    P = _params(H, m, N, "glu", rng, zero_mix=True)
    y = BO.block(x, P, "blocks.0.", dict(n=N, channel_stage="glu", layer=layer), A_fn, t)
    xh = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * P["blocks.0.norm2.weight"]
    h = xh @ P["blocks.0.ff1.weight"].t() + P["blocks.0.ff1.bias"]
    assert torch.allclose(y, x + h[..., :H] * torch.sigmoid(h[..., H:]), atol=1e-12)
    # channel zeroed, mixer live: the residual adds exactly the epilogue of the scan rows, whose first row is the
    # c_down bias (the zero state before the first interval)
    P = _params(H, m, N, "tanh", rng, zero_channel=True)
    y = BO.block(x, P, "blocks.0.", dict(n=N, channel_stage="tanh", layer=layer), A_fn, t)
    assert torch.allclose(y[:, 0] - x[:, 0], P["blocks.0.mixer.c_down.bias"].expand(Bn, H), atol=1e-12)
