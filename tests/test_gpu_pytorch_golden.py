"""getOutput on the GPU against the reference's own PyTorch model.

The nets and outputs are the fixtures of tests/test_pytorch_golden.py
(written by tests/golden/make_pytorch_golden.py from the reference's
model_pytorch.py and export_model_pytorch.py): model versions 15 and 17,
16 KataGo-featurized positions on 19x19, 19x11, 17x19, 7x15 and 9x9 boards in
19x19 tensors, each row with its own policyOptimism (0, 1/2, 1).

Tolerances (the north star's): policy max-abs <= 1e-3 (fp32) / 2e-2 (fp16)
over legal entries with an identical top move (unless the reference's own top
two lie within that tolerance), value and score <= 1e-3 / 1e-2, ownership as
policy.
"""
import numpy as np
import pytest

import pytorch_golden as pg
from katago_amd import nn

pytestmark = pytest.mark.gpu

TOL = {False: dict(policy=1e-3, value=1e-3, score=1e-3, ownership=1e-3),
       True: dict(policy=2e-2, value=1e-2, score=1e-2, ownership=2e-2)}


@pytest.mark.parametrize("fp16", [False, True], ids=["fp32", "fp16"])
@pytest.mark.parametrize("name", pg.names())
def test_get_output_matches_reference_pytorch_forward(name, fp16):
    sp, gl = pg.inputs()
    n = sp.shape[0]
    opt = np.array([(0.0, 0.5, 1.0)[i % 3] for i in range(n)], np.float32)
    lm = nn.LoadedModel(pg.model_path(name))
    h = nn.ComputeHandle(nn.ComputeContext(lm, 19, 19, use_fp16=fp16), max_batch=n)
    assert h.using_fp16 == fp16
    out = h.get_output(sp, gl, np.zeros(n, np.int32), opt)
    exp = pg.expected(name, opt)
    s = lm.info.output_scale_multiplier
    errs = pg.max_errors(out, exp, s)
    print(f"{name} {'fp16' if fp16 else 'fp32'} max-abs errors: {errs}")
    for k, tol in TOL[fp16].items():
        assert errs[k] <= tol, (name, k, errs)
    assert not pg.argmax_disagreements(out, exp, TOL[fp16]["policy"], s), name
