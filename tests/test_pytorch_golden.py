"""The oracle against the reference's own PyTorch model (CPU).

Fixtures: tests/golden/make_pytorch_golden.py ran the reference's
model_pytorch.Model forward and wrote each net with the reference's exporter
(export_model_pytorch.py). These pin, with outputs the reference computed
itself, what KataGo's C++ test records (model versions 5-11) leave open:
the two- and four-channel policy outputs and their policyOptimism mix, the
version-15 pass MLP, fixed and learnable 2-D RoPE with grouped-query
attention, the transformer RMSNorm, SwiGLU, transformer blocks nested in
bottleneck blocks, and the per-position and spatial RMSNorm trunk tips.

Tolerance: 2e-5 absolute on every output (the fp32 oracle against a float64
trunk; measured at most 3.2e-6). A dropped term, a transposed operand or a
wrong RoPE pairing moves these outputs by 1e-2 or more.
"""
import numpy as np
import pytest

import pytorch_golden as pg
from katago_amd import nn
from oracle import oracle

TOL = 2e-5
OPTIMISM = [0.0, 0.5, 1.0]

# model version and policy channels each fixture net must declare
DECLARED = {
    "b4c32-fson-mish": (15, 2),
    "b3c48h3tfrs-silu-rnh-q": (17, 4),
    "b2c96h6kv3qk32v16tflrs-silu-rsnh": (17, 2),
    "b3c64h2nbttfrs-mish-rsnh": (17, 2),
}


def test_fixture_nets_are_the_declared_versions():
    assert sorted(pg.names()) == sorted(DECLARED)
    for name, (version, channels) in DECLARED.items():
        info = nn.LoadedModel(pg.model_path(name)).info
        assert (info.model_version, info.num_policy_channels) == (version, channels), name
        assert pg.expected(name, np.zeros(16))["channels"] == channels


@pytest.mark.parametrize("opt", OPTIMISM)
@pytest.mark.parametrize("name", sorted(DECLARED))
def test_oracle_matches_reference_pytorch_forward(name, opt):
    sp, gl = pg.inputs()
    n = sp.shape[0]
    om = oracle.OracleModel(pg.model_path(name))
    out = om.forward(sp, gl, None, np.full(n, opt, np.float32))
    exp = pg.expected(name, np.full(n, opt))
    errs = pg.max_errors(out, exp)
    assert max(errs.values()) <= TOL, (name, opt, errs)


def test_oracle_mixes_policy_per_row():
    """Each row takes its own policyOptimism (a batch with 0, 1/2 and 1)."""
    name = "b3c48h3tfrs-silu-rnh-q"
    sp, gl = pg.inputs()
    opt = np.array([OPTIMISM[i % 3] for i in range(sp.shape[0])], np.float32)
    out = oracle.OracleModel(pg.model_path(name)).forward(sp, gl, None, opt)
    assert pg.max_errors(out, pg.expected(name, opt))["policy"] <= TOL


def test_rmsnorm_tip_activation_follows_the_eigen_backend():
    """After an RMSNorm trunk tip KataGo's Eigen backend applies the tip
    activation only when it is SiLU (eigenbackend.cpp:982-984,1012-1014);
    the PyTorch model applies its configured one (here mish). The oracle
    follows the Eigen backend: it matches the reference forward with the tip
    activation removed, and differs materially from the unmodified one."""
    name = "b3c64h2nbttfrs-mish-rsnh"
    sp, gl = pg.inputs()
    n = sp.shape[0]
    out = oracle.OracleModel(pg.model_path(name)).forward(sp, gl, None, np.zeros(n, np.float32))
    assert max(pg.max_errors(out, pg.expected(name, np.zeros(n))).values()) <= TOL
    model_act = pg.expected(name, np.zeros(n), prefix="model_act/")
    assert pg.max_errors(out, model_act)["value"] > 0.1


@pytest.mark.parametrize("name", sorted(DECLARED))
def test_oracle_layer_dump_matches_reference_trunk(name):
    """The oracle's per-block trunk dump (the lines of the reference's
    DEBUG_INTERMEDIATE_VALUES build) against the trunk the reference's
    PyTorch forward reports through ExtraOutputs: after the embedding, after
    each block, after the tip. Loaded without transformToReduceActivations,
    which rescales trunk channels, so both hold the same trunk. Element
    counts exact; min, max and rms within 1e-5 relative, mean within 1e-5 of
    the rms."""
    from helpers import parse_layer_dump
    sp, gl = pg.inputs()
    n = sp.shape[0]
    om = oracle.OracleModel(pg.model_path(name), load_time_transforms=False)
    om.set_layer_dump(True)
    om.forward(sp, gl, None, np.zeros(n, np.float32))
    got = parse_layer_dump(om.layer_dump())
    exp = pg.data()[f"{name}/trunkstats"]
    names = [g[0] for g in got]
    assert names == [f"Blockstack block {i}" for i in range(len(exp) - 2)] + ["Trunk after blocks", "Trunk tip"]
    for g, e in zip(got, exp):
        assert g[1] == int(e[0]), (g[0], g[1], e[0])
        for k, (a, b) in enumerate(zip(g[2:6], e[1:5])):
            tol = 1e-5 * (e[4] if k == 2 else max(abs(b), 1e-3))
            assert abs(a - b) <= tol + 2e-6 * abs(b), (name, g[0], ["min", "max", "mean", "rms"][k], a, b)
