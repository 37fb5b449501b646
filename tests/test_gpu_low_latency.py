"""Low-latency mode (hipLowLatency / kgh_handle_set_low_latency): split-K 3x3
convolutions for handles of at most 16 rows. Checked against the CPU oracle at
the fp16 whole-net tolerances (the summation order differs from the default
kernels, so these rows are not bitwise equal to a default handle's), and for
batch-size independence within the mode."""
import numpy as np
import pytest

from katago_amd import modelgen, nn
from oracle import oracle
from test_gpu_parity import _compare

pytestmark = pytest.mark.gpu


def _handle(lm, n, low_latency=True):
    ctx = nn.ComputeContext(lm, 19, 19, use_fp16=True, low_latency=low_latency)
    return ctx, nn.ComputeHandle(ctx, max_batch=n)


@pytest.mark.parametrize("n,board_sizes,cfg_idx", [
    (1, (19,), 2),
    (4, (19,), 2),
    (8, (9, 13, 19), 3),
    (16, (19, 9), 3),
], ids=["c2-b1", "c2-b4", "c3-b8-mixed", "c3-b16-mixed"])
def test_low_latency_matches_oracle(model_dir, n, board_sizes, cfg_idx):
    cfg = modelgen.configs()[cfg_idx]
    path = modelgen.ensure_model(model_dir, cfg)
    om = oracle.OracleModel(path, 19, 19)
    lm = nn.LoadedModel(path)
    ctx, h = _handle(lm, n)
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed + n, n, board_sizes=board_sizes)
    sym = np.arange(n) % 8
    opt = (np.arange(n) % 3) / 2.0
    gpu = h.get_output(sp, gl, sym, opt)
    ora = om.forward(sp, gl, sym, opt)
    _compare(gpu, ora, True, lm.info.output_scale_multiplier, board_sizes, n, f"low-latency C{cfg_idx} n={n}")
    for k in gpu:
        assert np.isfinite(gpu[k]).all(), k


def test_low_latency_rows_do_not_depend_on_batch(model_dir):
    """Within the mode every call runs the same split-K kernels, so a row's
    outputs are bitwise the same at batch 1 and inside a batch of 12; the mode
    is deterministic (a repeat gives the same bits)."""
    cfg = modelgen.configs()[3]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    ctx, h = _handle(lm, 12)
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, 12, board_sizes=(9, 13, 19))
    full = h.get_output(sp, gl)
    again = h.get_output(sp, gl)
    for k in full:
        assert np.array_equal(full[k], again[k]), k
    for r in (0, 5, 11):
        one = h.get_output(sp[r:r + 1], gl[r:r + 1])
        for k in full:
            assert np.array_equal(full[k][r], one[k][0]), (r, k)


def test_low_latency_close_to_default_kernels(model_dir):
    """The split-K sums differ from the default kernels only by fp32 rounding
    order: the outputs agree far inside the fp16 tolerances."""
    cfg = modelgen.configs()[2]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, 4)
    _, fast = _handle(lm, 4, True)
    _, dflt = _handle(lm, 4, False)
    a = fast.get_output(sp, gl)
    b = dflt.get_output(sp, gl)
    for k in a:
        d = np.abs(a[k] - b[k]).max()
        assert d <= 5e-3, (k, d)


def test_low_latency_device_handle_limits(model_dir):
    """kgh_handle_set_low_latency on a device handle: accepted up to 16 rows,
    refused above with a message, and it can be switched off again."""
    cfg = modelgen.configs()[2]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    dm = nn.DeviceModel(lm, use_fp16=True)
    big = nn.DeviceHandle(dm, max_batch=17)
    with pytest.raises(nn.StringError, match="low-latency"):
        big.set_low_latency(True)
    big.close()
    h = nn.DeviceHandle(dm, max_batch=2)
    h.set_low_latency(True)
    h.set_low_latency(False)
    h.close()
    dm.close()
