"""CPU checks of the Jordan-chain parametrisation and the layer's Jordan options, after the reference's
tests/test_jordan_repeated.py (block structure, chains, multiplicities, guards) and the option checks of
ews/layer.py:134-152. The leaf's numbers are checked on the GPU (tests/test_gpu_jordan.py)."""

import numpy as np
import pytest
import torch

import ews_mi355x as E


def _A(sizes, kinds, seed=0):
    rng = np.random.default_rng(seed)
    params = [torch.tensor([rng.normal(-1.5, 0.7)] if k == "real" else [rng.normal(-1.5, 0.7), rng.uniform(0.3, 1.5)],
                           dtype=torch.float64) for k in kinds]
    return E.AParamJordanRepeated(sizes, kinds, params)


def test_real_block_repeats_one_eigenvalue_with_ones_above():
    p = _A([3], ["real"])
    A = p().detach().numpy()
    lam = float(torch.nn.functional.softplus(p.block_params[0][0]))
    np.testing.assert_allclose(np.diag(A), lam)
    np.testing.assert_array_equal(np.diag(A, 1), 1.0)
    assert np.count_nonzero(np.triu(A, 2)) == 0 and np.count_nonzero(np.tril(A, -1)) == 0
    assert lam >= 0.0  # softplus: the eigenvalue is non-negative by construction


def test_complex_block_repeats_one_rotation():
    p = _A([6], ["complex"], seed=1)
    A = p().detach().numpy()
    R = A[:2, :2]
    for i in range(3):
        np.testing.assert_array_equal(A[2 * i: 2 * i + 2, 2 * i: 2 * i + 2], R)
        if i < 2:
            np.testing.assert_array_equal(A[2 * i: 2 * i + 2, 2 * i + 2: 2 * i + 4], np.eye(2))
    assert R[0, 0] == R[1, 1] and R[0, 1] == -R[1, 0]


def test_nilpotent_part_certifies_the_chain_and_multiplicity():
    for n in (2, 3, 4):
        A = _A([n], ["real"], seed=n)().detach().numpy()
        Nil = A - A[0, 0] * np.eye(n)
        assert np.abs(np.linalg.matrix_power(Nil, n - 1)).max() > 0
        assert np.abs(np.linalg.matrix_power(Nil, n)).max() == 0
        assert np.linalg.matrix_rank(Nil) == n - 1  # geometric multiplicity 1


def test_blocks_parameters_and_chains():
    p = _A([2, 2, 4], ["real", "real", "complex"])
    assert p.dim == 8 and sum(q.numel() for q in p.parameters()) == 1 + 1 + 2
    assert E.jordan_chains_of(p) is None  # mixed kinds
    assert E.jordan_chains_of(_A([3, 3], ["real", "real"])) == ("real", 3)
    assert E.jordan_chains_of(_A([8, 8], ["complex", "complex"])) == ("complex", 8)
    assert E.jordan_chains_of(_A([5, 5], ["real", "real"])) is None  # unsupported chain size
    eig = np.linalg.eigvals(_A([2, 2], ["real", "real"], seed=3)().detach().numpy())
    assert len(set(np.round(eig.real, 9))) == 2  # different eigenvalues come from different blocks


@pytest.mark.parametrize("sizes,kinds", [([1], ["real"]), ([2], ["complex"]), ([5], ["complex"]), ([3], ["bogus"])])
def test_degenerate_blocks_are_rejected(sizes, kinds):
    with pytest.raises(ValueError):
        E.AParamJordanRepeated(sizes, kinds, [torch.tensor([0.0, 0.0])])


def test_layer_jordan_options():
    A = _A([2, 2], ["real", "real"])
    layer = E.EWS(A, N=2, leaf="jordan_closed", combine="block_kernel", jordan_flows=True)
    assert layer.jordan_flows and layer._engine_check() == "dense"
    with pytest.raises(ValueError, match="jordan_flows needs combine='block_kernel'"):
        E.EWS(A, N=2, jordan_flows=True)
    with pytest.raises(ValueError, match="jordan_repeated A"):
        E.EWS(E.AParamConstant(torch.eye(4)), N=2, leaf="jordan_closed_tables")
    with pytest.raises(NotImplementedError, match="depths 1 and 2"):
        E.EWS(A, N=3, leaf="jordan_closed")._engine_check()
    # block_series on general blocks: the same route (tests/test_engines.py:267-273: depth 3 fails fast)
    blk = E.AParamBlockDiag([torch.eye(3), torch.eye(2)], [3, 2])
    assert E.EWS(blk, N=2, leaf="block_series", series_q=12)._engine_check() == "dense"
    with pytest.raises(NotImplementedError, match="depths 1 and 2"):
        E.EWS(blk, N=3, leaf="block_series", series_q=12)._engine_check()
