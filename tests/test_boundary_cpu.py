"""CPU checks of the boundary: the built library loads and exports every C-ABI symbol include/ews_hip.h
declares (no compute call: there is no GPU here), the host layer mirrors the reference's constructor
validation and call-shape errors (ews/layer.py:82-152, 290-302; tests/test_engines.py:170-192), and the
C ABI rejects bad descriptors with its error codes."""

import ctypes
import os
import re

import pytest
import torch

import ews_mi355x as E
from ews_mi355x import _native as nat
from ews_mi355x import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    src = open(os.path.join(ROOT, "include", "ews_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:size_t|int|const char\*)\s+(ews_\w+)\s*\(", src, re.M)))


def test_library_exports_every_declared_symbol():
    lib = nat.load()
    declared = _declared_functions()
    assert len(declared) >= 6
    for name in declared:
        assert hasattr(lib, name), name
    assert set(nat.EXPORTED) <= set(declared)
    assert lib.ews_version().decode().count(".") == 2


def _desc(**kw):
    base = dict(batch=2, length=10, dim=8, depth=2, structure=1, flow_mode=0, readout=0, level0=1, path_dtype=0,
                chunk=0)
    base.update(kw)
    return nat.DiagDesc(**base)


def test_c_abi_error_codes():
    lib = nat.load()
    good = _desc()
    assert lib.ews_diag_workspace_bytes(ctypes.byref(good)) > 0
    assert lib.ews_diag_residual_bytes(ctypes.byref(good)) > 0
    null = ctypes.c_void_p(0)
    # NULL pointers are rejected before any launch
    assert lib.ews_diag_forward(ctypes.byref(good), null, null, null, null, null, null, null) == -1
    bad = {
        "depth": (_desc(depth=3), -3),
        "odd planes": (_desc(dim=7), -2),
        "length": (_desc(length=1), -2),
        "structure": (_desc(structure=9), -4),
        "readout": (_desc(readout=7), -4),
        "dtype": (_desc(path_dtype=5), -4),
        "real too wide": (_desc(structure=2, dim=40), -2),
    }
    for name, (dsc, code) in bad.items():
        assert lib.ews_diag_forward(ctypes.byref(dsc), null, null, null, null, null, null, null) == code, name
        assert lib.ews_diag_workspace_bytes(ctypes.byref(dsc)) == 0, name
    assert lib.ews_error_string(-2).decode().startswith("batch/length/dim")


def test_sequential_plan_selection_and_log_readout():
    """The per-sample sequential kernels: asked for by chunk = EWS_CHUNK_SEQUENTIAL, chosen by chunk 0 for the
    log-prefix readout or B >= 128 and L <= 1025 (real diagonal, depth 2, d <= 32, per-interval flows). Their
    residual is one state checkpoint per 16 steps (lanes = 32 d rounded to 64, plus the d level-1 states), their
    workspace the per-sample parameter partials."""
    lib = nat.load()
    null = ctypes.c_void_p(0)

    def sizes(**kw):
        dsc = _desc(**{"structure": 2, "dim": 32, **kw})
        return lib.ews_diag_residual_bytes(ctypes.byref(dsc)), lib.ews_diag_workspace_bytes(ctypes.byref(dsc))

    def al(x):
        return (x + 255) // 256 * 256

    # c4's block: B = 256, L = 512 -> 32 blocks of (1024 + 32) floats per sample
    assert sizes(batch=256, length=512) == (al(256 * 32 * 1056 * 4), al(256 * 32 * 4))
    assert sizes(batch=256, length=512, readout=4) == sizes(batch=256, length=512)
    assert sizes(batch=2, length=100, chunk=-1) == (al(2 * 7 * 1056 * 4), al(2 * 32 * 4))
    assert sizes(batch=2, length=100, chunk=-1, dim=5) == (al(2 * 7 * (192 + 5) * 4), al(2 * 5 * 4))
    # not chosen: few samples, long sequences, or an explicit chunk length (the chunk kernels' larger residual)
    assert sizes(batch=2, length=100)[0] != sizes(batch=2, length=100, chunk=-1)[0]
    assert sizes(batch=256, length=2000)[0] != sizes(batch=256, length=2000, chunk=-1)[0]
    assert sizes(batch=256, length=512, chunk=16)[0] != sizes(batch=256, length=512)[0]
    # the log readout off the sequential kernels (planes, cached flows, an explicit chunk length): the chunk
    # kernels, whose residual adds level 1 of every step and whose workspace adds one flat-row cotangent per step
    for kw in (dict(structure=1, dim=8), dict(structure=2, dim=8, flow_mode=1), dict(structure=2, dim=8, chunk=16)):
        B, L, d = 3, 50, 8
        r0 = lib.ews_diag_residual_bytes(ctypes.byref(_desc(batch=B, length=L, level0=0, **kw)))
        w0 = lib.ews_diag_workspace_bytes(ctypes.byref(_desc(batch=B, length=L, level0=0, **kw)))
        r1 = lib.ews_diag_residual_bytes(ctypes.byref(_desc(batch=B, length=L, readout=4, **kw)))
        w1 = lib.ews_diag_workspace_bytes(ctypes.byref(_desc(batch=B, length=L, readout=4, **kw)))
        assert (r1, w1) == (r0 + al(B * (L - 1) * d * 4), w0 + al(B * (L - 1) * (d + d * d) * 4)), kw
    bad = {
        "log readout, depth 1": _desc(structure=2, depth=1, readout=4),
        "sequential planes": _desc(chunk=-1),
        "sequential terminal": _desc(structure=2, readout=1, chunk=-1),
        "chunk -2": _desc(structure=2, chunk=-2),
    }
    for name, dsc in bad.items():
        assert lib.ews_diag_workspace_bytes(ctypes.byref(dsc)) == 0, name
        assert lib.ews_diag_forward(ctypes.byref(dsc), null, null, null, null, null, null, null) in (-2, -3, -4), name


def _planes(K=2):
    return E.AParamDampedRotation(torch.zeros(K), torch.zeros(K), 2 * K)


def test_layer_option_validation_mirrors_reference():
    with pytest.raises(ValueError):
        E.EWS(E.AParamGeneral(torch.zeros(4, 4)), N=1, combine="block_kernel")
    with pytest.raises(ValueError):
        E.EWS(E.AParamGeneral(torch.zeros(4, 4)), N=1, leaf="plane_closed")
    with pytest.raises(ValueError):
        E.EWS(E.AParamBlockDiag([torch.zeros(2, 2), torch.zeros(2, 2)], [2, 2]), N=1, leaf="plane_closed")
    with pytest.raises(ValueError):
        E.EWS(E.AParamGeneral(torch.zeros(4, 4)), N=1, combine="nonsense")
    with pytest.raises(ValueError):
        E.EWS(E.AParamBlockDiag([torch.zeros(2, 2), torch.zeros(2, 2)], [2, 2]), N=2, leaf="block_series")
    with pytest.raises(ValueError):
        E.EWS(_planes(), N=2, leaf="series")  # series needs series_q
    with pytest.raises(ValueError):
        E.EWS(_planes(), N=2, terminal_reduce="sideways")
    with pytest.raises(ValueError):
        E.EWS(_planes(), N=2, van_loan_expm="taylor")
    layer = E.EWS(_planes(3), N=2, leaf="plane_closed", combine="block_kernel")
    assert layer.block_sizes == (2, 2, 2) and layer.signature_dim == 6 + 36
    assert E.block_sizes_of(E.AParamGeneral(torch.zeros(3, 3))) is None


def test_layer_call_shape_errors_and_no_cpu_path():
    layer = E.EWS(_planes(2), N=2, leaf="plane_closed")
    with pytest.raises(ValueError):
        layer(torch.zeros(5, 4), torch.zeros(4))  # misaligned clock
    with pytest.raises(ValueError):
        layer(torch.zeros(2, 5, 4), torch.zeros(5))  # batched path needs a 2-D clock
    with pytest.raises(ValueError):
        layer(torch.zeros(5), torch.zeros(5))
    with pytest.raises(ValueError):
        layer(torch.zeros(5, 4), torch.zeros(5), readout="median")
    with pytest.raises(ValueError):
        layer(torch.zeros(5, 4), torch.zeros(5), readout="mean", output_format="list")
    with pytest.raises(NotImplementedError):
        E.EWS(_planes(2), N=3, leaf="plane_closed")(torch.zeros(5, 4), torch.zeros(5))
    with pytest.raises(RuntimeError, match="HIP device"):
        layer(torch.zeros(5, 4), torch.linspace(0, 1, 5))  # CPU tensors never fall back


def test_log_dims_mirror_reference():
    for d, N, expect in [(3, 3, 14), (4, 2, 10), (2, 4, 8)]:
        assert E.log_signature_dim(d, N) == expect
    assert E.log_level_slices(4, 2) == ((0, 4), (4, 10))
    lib = nat.load()
    for d, N in [(3, 3), (4, 2), (16, 3), (32, 2), (1, 3)]:  # the library's Witt numbers (host Duval)
        assert lib.ews_log_dim(d, N) == E.log_signature_dim(d, N)
    assert lib.ews_log_dim(4, 4) == 0


def test_log_c_abi_error_codes():
    lib = nat.load()
    null = ctypes.c_void_p(0)
    good = nat.LogDesc(2, 5, 16, 3, 1, 0)
    assert lib.ews_log_workspace_bytes(ctypes.byref(good)) > 0
    assert lib.ews_log_forward(ctypes.byref(good), null, null, null, null) == -1
    bad = {"depth": (nat.LogDesc(2, 5, 4, 4, 1, 0), -3), "wide depth 3": (nat.LogDesc(2, 5, 17, 3, 1, 0), -2),
           "terminal rows": (nat.LogDesc(2, 5, 4, 2, 1, 1), -2), "readout": (nat.LogDesc(2, 5, 4, 2, 1, 7), -4),
           "rows": (nat.LogDesc(2, 0, 4, 2, 1, 0), -2)}
    for name, (dsc, code) in bad.items():
        assert lib.ews_log_forward(ctypes.byref(dsc), null, null, null, null) == code, name
        assert lib.ews_log_workspace_bytes(ctypes.byref(dsc)) == 0, name


def _ddesc(**kw):
    base = dict(batch=2, length=10, dim=16, depth=3, series_q=20, flow_mode=0, readout=0, level0=1, chunk=0,
                leaf=0, vl_steps=0, vl_expm=0, vl_mode=0, chen_expm=0)
    base.update(kw)
    return nat.DenseDesc(**base)


def test_dense_c_abi_error_codes():
    lib = nat.load()
    good = _ddesc()
    ws = lib.ews_dense_workspace_bytes(ctypes.byref(good))
    # powers table + padded levels/flows of 2 x 9 intervals + summaries + carries
    assert ws >= 2 * 9 * (16 + 256 + 4096 + 256) * 4
    assert lib.ews_dense_num_passes() == 4
    null = ctypes.c_void_p(0)
    assert lib.ews_dense_forward(ctypes.byref(good), null, null, null, null, null, null) == -1
    bad = {
        "depth": (_ddesc(depth=4), -3),
        "too wide": (_ddesc(dim=33), -2),
        "wide at depth 3": (_ddesc(dim=17, depth=3), -2),
        "wide block series": (_ddesc(dim=17, leaf=2, depth=2), -2),
        "length": (_ddesc(length=1), -2),
        "series order": (_ddesc(series_q=41), -4),
        "readout": (_ddesc(readout=9), -4),
        "flow mode": (_ddesc(flow_mode=3), -4),
        "basepoint length": (_ddesc(flow_mode=2, length=2), -2),
        "leaf": (_ddesc(leaf=3), -4),
        "block series at depth 3": (_ddesc(leaf=2, depth=3), -3),
        "van loan knots 0": (_ddesc(leaf=1, vl_steps=0), -4),
        "van loan knots 65": (_ddesc(leaf=1, vl_steps=65), -4),
        "van loan scheme": (_ddesc(leaf=1, vl_steps=20, vl_expm=4), -4),
        "van loan mode": (_ddesc(leaf=1, vl_steps=20, vl_mode=3), -4),
        "van loan basepoint length": (_ddesc(leaf=1, vl_steps=20, vl_mode=2, length=2), -2),
        "flow scheme": (_ddesc(chen_expm=4), -4),
    }
    for name, (dsc, code) in bad.items():
        assert lib.ews_dense_forward(ctypes.byref(dsc), null, null, null, null, null, null) == code, name
        assert lib.ews_dense_workspace_bytes(ctypes.byref(dsc)) == 0, name
    # 16 < d <= 32 at depths 1-2 (series and Van Loan leaves): padded 32 x 32 step matrices and states
    for leaf, kw in ((0, {}), (1, {"vl_steps": 4})):
        wd = _ddesc(dim=24, depth=2, leaf=leaf, **kw)
        wsz = lib.ews_dense_workspace_bytes(ctypes.byref(wd))
        assert wsz >= 2 * 9 * (32 + 1024) * 4, leaf
        assert lib.ews_dense_backward_workspace_bytes(ctypes.byref(wd)) > wsz
        assert lib.ews_dense_forward(ctypes.byref(wd), null, null, null, null, null, null) == -1
    # the block-series leaf (depths 1 and 2): the series leaf's buffers plus its level-1 adjoint's
    bsd = _ddesc(leaf=2, depth=2)
    assert lib.ews_dense_workspace_bytes(ctypes.byref(bsd)) == lib.ews_dense_workspace_bytes(
        ctypes.byref(_ddesc(depth=2)))
    assert lib.ews_dense_backward_workspace_bytes(ctypes.byref(bsd)) > lib.ews_dense_backward_workspace_bytes(
        ctypes.byref(_ddesc(depth=2)))
    # the Van Loan leaf ignores the series order; its options are checked instead
    vl = _ddesc(leaf=1, vl_steps=64, vl_expm=3, vl_mode=2, series_q=99, chen_expm=2)
    assert lib.ews_dense_workspace_bytes(ctypes.byref(vl)) > 0
    assert lib.ews_dense_forward(ctypes.byref(vl), null, null, null, null, null, null) == -1


def test_dense_layer_routing_and_errors():
    A = E.AParamGeneral(torch.zeros(4, 4))
    assert E.EWS(A, N=3, leaf="series", series_q=8)._engine_check() == "dense"
    assert E.EWS(_planes(2), N=3, leaf="series", series_q=8)._engine_check() == "dense"
    assert E.EWS(_planes(2), N=2, leaf="series", series_q=8)._engine_check() == "diag"
    # the Van Loan leaf (the reference default) runs on the dense kernels for every generator structure
    assert E.EWS(A, N=2)._engine_check() == "dense"
    assert E.EWS(_planes(2), N=2)._engine_check() == "dense"
    assert E.EWS(A, N=3, M=64, van_loan_expm="pade_lite")._engine_check() == "dense"
    # flows of another scheme: the dense kernels evaluate it; the closed-form kernels take exact flows only
    assert E.EWS(A, N=3, leaf="series", series_q=8, chen_expm="cayley")._engine_check() == "dense"
    assert E.EWS(_planes(2), N=2, leaf="series", series_q=8, chen_expm="pade")._engine_check() == "dense"
    # closed-form leaf with approximate flows: the exact integrals on the dense kernels (d <= 16)
    assert E.EWS(_planes(2), N=2, leaf="plane_closed", chen_expm="cayley")._engine_check() == "dense"
    with pytest.raises(NotImplementedError):
        E.EWS(_planes(9), N=2, leaf="plane_closed", chen_expm="cayley")._engine_check()
    with pytest.raises(NotImplementedError):
        E.EWS(A, N=4)._engine_check()
    # 16 < d <= 32: the wide dense kernels at depths 1-2 (series and Van Loan leaves)
    assert E.EWS(E.AParamGeneral(torch.zeros(17, 17)), N=2)._engine_check() == "dense"
    assert E.EWS(E.AParamGeneral(torch.zeros(32, 32)), N=1, leaf="series", series_q=8)._engine_check() == "dense"
    assert E.EWS(_planes(12), N=2, van_loan_expm="cayley")._engine_check() == "dense"
    with pytest.raises(NotImplementedError):
        E.EWS(E.AParamGeneral(torch.zeros(17, 17)), N=3)._engine_check()
    with pytest.raises(NotImplementedError):
        E.EWS(E.AParamGeneral(torch.zeros(33, 33)), N=2, leaf="series", series_q=8)._engine_check()
    with pytest.raises(NotImplementedError):
        ops.DenseLeaf("van_loan", M=65)
    with pytest.raises(ValueError):
        ops.DenseLeaf("van_loan", reweighting_mode="uniform")
    with pytest.raises(RuntimeError, match="HIP device"):
        E.EWS(A, N=3, leaf="series", series_q=8)(torch.zeros(5, 4), torch.linspace(0, 1, 5))


def _mdesc(**kw):
    base = dict(batch=2, rows=5, dim=4, depth=2, level0=1, hidden=7, variant=0, prepend=1, prescale=0)
    base.update(kw)
    eps = kw.pop("eps", (1e-3, 1e-3, 1e-3))
    base.pop("eps", None)
    return nat.MixerDesc(**base, eps=(ctypes.c_float * 3)(*eps))


def test_mixer_c_abi_error_codes():
    lib = nat.load()
    null = ctypes.c_void_p(0)
    good = _mdesc()
    # level products (10 rows x 2 levels x 7) then factors (10 x 2 x 3), each 256-byte aligned
    assert lib.ews_mixer_residual_bytes(ctypes.byref(good)) == 768 + 256
    assert lib.ews_mixer_forward(ctypes.byref(good), null, null, null, null, null, null, null) == -1
    assert lib.ews_mixer_backward(ctypes.byref(good), null, null, null, null, null, null, null) == -1
    bad = {"depth": (_mdesc(depth=4), -3), "wide depth 3": (_mdesc(dim=17, depth=3), -2),
           "dim": (_mdesc(dim=65), -2), "hidden": (_mdesc(hidden=0), -2), "rows": (_mdesc(rows=0), -2),
           "variant": (_mdesc(variant=3), -4)}
    for name, (dsc, code) in bad.items():
        assert lib.ews_mixer_forward(ctypes.byref(dsc), null, null, null, null, null, null, null) == code, name
        assert lib.ews_mixer_backward(ctypes.byref(dsc), null, null, null, null, null, null, null) == code, name
        assert lib.ews_mixer_residual_bytes(ctypes.byref(dsc)) == 0, name


def test_mixer_module_mirrors_reference_fields_and_errors():
    m = E.MixerEpilogue(3, 2, 5, graded_variant="dilation", graded_prescale="binomial")
    assert m.graded.level_slices == ((0, 3), (3, 12)) and m.graded.gains is None and m.graded.lam.shape == ()
    assert tuple(m.c_down.weight.shape) == (5, 12) and tuple(m.c_down.bias.shape) == (5,)
    assert E.graded_level_slices(2, 3) == ((0, 2), (2, 6), (6, 14))
    with pytest.raises(ValueError, match="variant must be one of"):
        E.GradedRMSNorm(2, 2, variant="flat")
    with pytest.raises(ValueError, match="eps must be a scalar"):
        E.GradedRMSNorm(2, 2, eps=[1e-3])
    with pytest.raises(ValueError, match="last axis must be D"):
        E.GradedRMSNorm(2, 2)(torch.zeros(5, 7))
    with pytest.raises(ValueError, match="graded_prescale must be None or 'binomial'"):
        E.MixerEpilogue(2, 2, 3, graded_prescale="poisson")
    with pytest.raises(TypeError, match="HIP device"):  # no CPU path for the fused epilogue
        m(torch.zeros(4, 13))


def _cdesc(**kw):
    base = dict(batch=2, length=300, channels=3, mode=1, scaling=1, normalize=0, gates=0, has_mask=0,
                increment_driver=0, has_time_denominator=0, basepoint=0, learned_alpha=0, alpha=0.5,
                norm_constant=1.0, time_denominator=1.0, variation_eps=1e-8, in_scale=1.0)
    base.update(kw)
    return nat.ClockDesc(**base)


def test_clock_c_abi_error_codes():
    lib = nat.load()
    null = ctypes.c_void_p(0)
    good = _cdesc()
    # residual: 2 last-row ints, then 2 samples x 2 chunks of 256 rows of float64 sums (256-byte aligned)
    assert lib.ews_clock_residual_bytes(ctypes.byref(good)) == 256 + 256
    assert lib.ews_clock_num_params(ctypes.byref(good)) == 0
    assert lib.ews_clock_num_params(ctypes.byref(_cdesc(mode=4, gates=3, scaling=0, normalize=1))) == 3 * 3 + 3
    assert lib.ews_clock_num_params(ctypes.byref(_cdesc(learned_alpha=1))) == 1
    assert lib.ews_clock_forward(ctypes.byref(good), null, null, null, null, null, null, null) == -1
    bad = {"mode": (_cdesc(mode=5), -4), "scaling": (_cdesc(scaling=4), -4), "channels": (_cdesc(channels=65), -2),
           "length": (_cdesc(length=0), -2), "steps blended": (_cdesc(scaling=3), -4),
           "gate scaling": (_cdesc(mode=3, gates=1, scaling=1, normalize=1), -4),
           "gate per-sample": (_cdesc(mode=3, gates=1, scaling=0, normalize=0), -4),
           "token gates": (_cdesc(mode=3, gates=2, scaling=0, normalize=1), -2),
           "clamped gates": (_cdesc(mode=4, gates=9, scaling=0, normalize=1), -2),
           "learned time": (_cdesc(mode=0, learned_alpha=1), -4)}
    for name, (dsc, code) in bad.items():
        assert lib.ews_clock_forward(ctypes.byref(dsc), null, null, null, null, null, null, null) == code, name
        assert lib.ews_clock_residual_bytes(ctypes.byref(dsc)) == 0, name
        assert lib.ews_clock_num_params(ctypes.byref(dsc)) == -1, name


def _ldesc(**kw):
    base = dict(batch=2, length=300, branch_dim=6, append=0, out_dim=16, lift=1, increment=0, has_mask=0,
                basepoint=0)
    base.update(kw)
    return nat.LiftDesc(**base)


def test_lift_c_abi_error_codes():
    lib = nat.load()
    null = ctypes.c_void_p(0)
    good = _ldesc(increment=1)
    # residual: 2 last-row ints, then 2 samples x 3 chunks of 128 rows x 6 float64 channel sums
    assert lib.ews_lift_residual_bytes(ctypes.byref(good)) == 256 + 512
    assert lib.ews_lift_forward(ctypes.byref(good), null, null, null, null, null, null, null) == -1
    bad = {"branch": (_ldesc(branch_dim=65), -2), "out": (_ldesc(out_dim=65), -2), "lift": (_ldesc(lift=3), -4),
           "no lift width": (_ldesc(lift=0, out_dim=5), -2), "preserve": (_ldesc(lift=2, branch_dim=1), -2),
           "length": (_ldesc(length=0), -2)}
    for name, (dsc, code) in bad.items():
        assert lib.ews_lift_forward(ctypes.byref(dsc), null, null, null, null, null, null, null) == code, name
        assert lib.ews_lift_backward(ctypes.byref(dsc), null, null, null, null, null, null, null, null, null,
                                     null, null) == code, name
        assert lib.ews_lift_residual_bytes(ctypes.byref(dsc)) == 0, name


def test_front_modules_mirror_reference_fields_and_errors():
    """ClockSpec / make_clock / B checks and messages of ews/clocks.py:51-124, 528-537 and ews/params.py:1165-1191
    (the cases of tests/test_clocks.py:99-124)."""
    with pytest.raises(ValueError):
        E.ClockSpec(mode="token_gated").validate()  # needs constant normalisation
    with pytest.raises(ValueError):
        E.ClockSpec(mode="nope").validate()
    with pytest.raises(ValueError, match="needs a key"):
        E.make_clock(E.ClockSpec(mode="token_gated", scaling="none", normalize="constant", norm_constant=1.0), 2)
    with pytest.raises(ValueError, match="alpha = 0"):
        E.make_clock(E.ClockSpec(mode="blended_variation", alpha=0.5, scaling="none", normalize="constant",
                                 norm_constant=1.0), 2).per_token_increment(torch.ones(2, 2))
    with pytest.raises(ValueError, match="unknown clock keys"):
        E.ClockSpec.from_config({"mode": "time", "bogus": 1})
    with pytest.raises(ValueError, match="'steps'"):
        E.ClockSpec(mode="blended_variation", alpha=0.5, scaling="steps").validate()
    clk = E.make_clock(E.ClockSpec(mode="clamped_gate", scaling="none", normalize="constant", norm_constant=2.0,
                                   gate_init_bias=(-1.0, 0.0, 1.0)), dim=3, key=2)
    assert isinstance(clk, E.GatedClock) and not clk.is_static
    assert tuple(clk.w.shape) == (3, 3) and tuple(clk.b.tolist()) == (-1.0, 0.0, 1.0)
    tok = E.make_clock(E.ClockSpec(mode="token_gated", scaling="none", normalize="constant", norm_constant=4.0,
                                   gate_init_bias=-0.5), dim=5, key=1)
    assert tuple(tok.w.shape) == (5,) and float(tok.b.detach()) == -0.5
    lrn = E.make_clock(E.ClockSpec(mode="blended_learn", alpha=0.3, alpha_parametrisation="sigmoid"), dim=3)
    assert isinstance(lrn, E.LearnableBlendedClock) and abs(float(lrn.alpha.detach()) - 0.3) < 1e-6
    assert isinstance(E.make_clock(E.ClockSpec(), 3), E.FixedClock)
    with pytest.raises(NotImplementedError):
        lrn.per_token_increment(torch.ones(2, 3))
    with pytest.raises(ValueError, match="at least 2 channels"):
        E.B(torch.zeros(2, 0))(torch.zeros(4, 1))
    with pytest.raises(TypeError, match="HIP device"):  # no CPU path for the front kernels
        E.make_clock(E.ClockSpec(mode="blended_variation", alpha=0.5), 3)(torch.arange(6.0), torch.zeros(6, 3))
    with pytest.raises(ValueError, match="path_mode"):
        E.BlockFront(E.make_clock(E.ClockSpec(), 3), path_mode="delta")


def test_token_scan_c_abi_error_codes():
    lib = nat.load()
    null = ctypes.c_void_p(0)
    good = ops.make_dense_desc(2, 51, 4, 2, 0, "per_interval", "prefix", False)
    assert lib.ews_token_scan_workspace_bytes(ctypes.byref(good), 5) > 0
    assert lib.ews_token_scan_workspace_bytes(ctypes.byref(good), 0) == 0
    assert lib.ews_token_scan(ctypes.byref(good), null, null, null, null, 5, null, null, null) == -1
    assert lib.ews_token_scan(ctypes.byref(good), null, null, null, null, 0, null, null, null) == -2
    assert lib.ews_token_scan_backward(ctypes.byref(good), null, null, null, null, 5, null, null, null, null,
                                       null) == -1
    wide = ops.make_dense_desc(2, 51, 17, 2, 0, "per_interval", "prefix", False)
    assert lib.ews_token_scan(ctypes.byref(wide), null, null, null, null, 5, null, null, null) == -2
    assert lib.ews_dense_local_terms_backward(ctypes.byref(good), null, null, null, null, null, null, null, null,
                                              null, null) == -1
    with pytest.raises(TypeError, match="HIP device"):
        E.token_cached_prefix_scan(torch.zeros(5, dtype=torch.int64), None, torch.zeros(3, 20), torch.zeros(3, 4, 4),
                                   4, 2)
