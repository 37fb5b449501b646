"""The per-block trunk dump on the GPU (kgh_handle_set_layer_dump, the
runtime counterpart of the reference's DEBUG_INTERMEDIATE_VALUES prints,
debugprint.h:14-49, eigenbackend.cpp:1773-1785) against the oracle's dump of
the same forward.

The device dump's values are multiplied by outputScaleMultiplier, which
undoes the load-time scale-by-8, so both dumps describe the same trunk: the
oracle applies transformToReduceActivations as the device does (the oracle's
dump itself is pinned against the reference's PyTorch forward in
tests/test_pytorch_golden.py). Same lines in the same order, the same element
counts; min, max and rms within 1e-4 relative in fp32 and 2e-2 in fp16, mean
within that fraction of the rms. Dumping does not change the outputs."""
import numpy as np
import pytest

import pytorch_golden as pg
from helpers import parse_layer_dump
from katago_amd import modelgen, nn
from oracle import oracle

pytestmark = pytest.mark.gpu

NETS = ["C1", "C4"] + pg.names()


def _net(model_dir, key):
    if key.startswith("C"):
        cfg = modelgen.configs()[int(key[1])]
        return modelgen.ensure_model(model_dir, cfg), cfg.board_sizes
    return pg.model_path(key), None


def _inputs(key, board_sizes, n):
    if board_sizes is None:
        sp, gl = pg.inputs()
        return sp[:n], gl[:n]
    return modelgen.synthetic_inputs(7, n, board_sizes=(19, 9, 13))


@pytest.mark.parametrize("fp16", [False, True], ids=["fp32", "fp16"])
@pytest.mark.parametrize("key", NETS)
def test_device_layer_dump_matches_oracle(model_dir, key, fp16):
    path, board_sizes = _net(model_dir, key)
    n = 6
    sp, gl = _inputs(key, board_sizes, n)
    lm = nn.LoadedModel(path)
    dm = nn.DeviceModel(lm, use_fp16=fp16)
    h = nn.DeviceHandle(dm, n)
    bufs = [nn.DeviceBuffer.from_array(a) for a in (sp, gl, np.zeros(n, np.int32), np.zeros(n, np.float32))]
    out = nn.DeviceBuffer(n * h.row_floats * 4)
    run = lambda: (h.forward_device(n, *(b.ptr for b in bufs), out.ptr), h.synchronize(),
                   out.to_array(np.float32, (n, h.row_floats)))[2]
    plain = run()
    h.set_layer_dump(True, lm.info.output_scale_multiplier)
    dumped = run()
    assert np.array_equal(plain, dumped)
    got = parse_layer_dump(h.layer_dump())
    h.set_layer_dump(False)

    om = oracle.OracleModel(path)
    om.set_layer_dump(True)
    om.forward(sp, gl, None, np.zeros(n, np.float32))
    exp = parse_layer_dump(om.layer_dump())
    print(f"\n{key} {'fp16' if fp16 else 'fp32'}: {len(got)} dump lines; last: {got[-1][:6]} vs {exp[-1][:6]}")
    assert [g[0] for g in got] == [e[0] for e in exp]
    rel = 2e-2 if fp16 else 1e-4
    for g, e in zip(got, exp):
        assert g[1] == e[1], (g[0], g[1], e[1])
        rms = e[5]
        for k, (a, b) in enumerate(zip(g[2:6], e[2:6])):
            tol = rel * (rms if k == 2 else max(abs(b), 1e-3 * rms)) + 1e-6
            assert abs(a - b) <= tol, (key, g[0], ["min", "max", "mean", "rms"][k], a, b)
