"""The float64 oracle against the reference's own golden files.

* ``tests/golden/reference_model_init.npz`` (copied from the reference's ``tests/``): the PRNG restatement must
  reproduce the fixture model's init draws (A, B at d_in=4, the float64 MLP head).
* ``tests/golden/reference_kernel_outputs.npz``: the 13 pinned logits of the reference classifier
  (``tests/test_kernel_outputs_pinned.py``): Van Loan leaf (M=4, exact expm) in all three reweighting modes,
  terminal by tree and by associative scan, mean and max readouts, and the depth-2 log-signature feature.
  The reference computed them in float32; the oracle is float64, so the bar is 1e-5 relative.
"""

import numpy as np
import pytest
import torch

from oracle import ews_oracle as O
from oracle import fixture_model as FM
from oracle import jax_prng as P

GOLD = "tests/golden/"


def _path(name):
    import os

    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)


def test_prng_restatement_reproduces_init_fixture():
    z = np.load(_path("reference_model_init.npz"))
    A, Bm, head = FM.fixture_params(d_in=4)
    # float32 normals: XLA's float32 erf_inv vs float64-then-round differ by at most ~1 ulp
    np.testing.assert_allclose(A, z["arr_1"], rtol=0, atol=3e-7)
    np.testing.assert_allclose(Bm, z["arr_0"], rtol=0, atol=3e-7)
    # float64 uniforms are exact bit manipulations
    np.testing.assert_allclose(head[0][0], z["arr_2"], rtol=0, atol=1e-16)
    np.testing.assert_allclose(head[0][1], z["arr_3"], rtol=0, atol=1e-16)
    np.testing.assert_array_equal(head[1][0], z["arr_4"])
    np.testing.assert_array_equal(head[1][1], z["arr_5"])
    np.testing.assert_array_equal(z["arr_6"], np.ones(2, np.float32))  # learned gains start at 1


def test_threefry_known_answer():
    # Salmon et al. SC'11 known-answer vectors for Threefry-2x32, 20 rounds
    x = P.threefry2x32(0, 0, np.array([0], np.uint32), np.array([0], np.uint32))
    assert (int(x[0][0]), int(x[1][0])) == (0x6B200159, 0x99BA4EFE)
    x = P.threefry2x32(0xFFFFFFFF, 0xFFFFFFFF, np.array([0xFFFFFFFF], np.uint32), np.array([0xFFFFFFFF], np.uint32))
    assert (int(x[0][0]), int(x[1][0])) == (0x1CB996FC, 0xBB002BE7)
    x = P.threefry2x32(0x13198A2E, 0x03707344, np.array([0x243F6A88], np.uint32), np.array([0x85A308D3], np.uint32))
    assert (int(x[0][0]), int(x[1][0])) == (0xC4923A9C, 0x483DF7A0)


@pytest.mark.parametrize("name", list(FM.combinations().keys()))
def test_oracle_reproduces_pinned_logits(name, rel):
    ref = np.load(_path("reference_kernel_outputs.npz"))
    mode, readout, reduce, feature = FM.combinations()[name]
    paths, clocks = FM.fixture_inputs()
    A, Bm, head = FM.fixture_params(feature=feature)
    x = torch.tensor(FM.lift(paths, Bm), dtype=torch.float64)
    c = torch.tensor(clocks, dtype=torch.float64)
    At = torch.tensor(A, dtype=torch.float64)
    kw = dict(leaf="van_loan", M=4, van_loan_expm="exact", chen_expm="exact", reweighting_mode=mode,
              terminal_reduce=reduce)
    if feature == "signature":
        feats = O.ews(x, c, At, 2, readout, **kw).numpy()
    else:
        feats = torch.stack([O.log_ews_single(x[b], c[b], At, 2, readout, **kw) for b in range(4)]).numpy()
    got = FM.head_apply(feats, head)
    assert got.shape == ref[name].shape
    assert rel(got, ref[name]) < 1e-5
