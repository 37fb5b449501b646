"""transformToReduceActivations (desc.cpp:352-1111 in the reference, always
applied at load, desc.cpp:2631) moves batch-norm scales below 1 into the
preceding convolution or matmul. It must not change what a net computes: the
oracle's outputs with and without it agree to within fp32 rounding
(2e-5 of each output's magnitude), on trained nets of model versions 5, 8, 9,
11 and 17 and on the synthetic benchmark nets. On the conv nets the two
forwards must also differ somewhere, so that the transform was exercised."""
import numpy as np
import pytest

from helpers import G170_MODEL, GOLDEN, TRANSFORMER_MODELS
from katago_amd import modelgen, nn
from oracle import oracle

TRAINED = [G170_MODEL, f"{GOLDEN}/g103-b6c96-s103408384-d26419149.txt.gz", f"{GOLDEN}/tinymodel_relu.bin.gz",
           f"{GOLDEN}/tinymodel_mish.bin.gz"] + TRANSFORMER_MODELS


def _check(path, n, exercised):
    info = nn.LoadedModel(path).info
    sp, gl = modelgen.synthetic_inputs(7, n, board_sizes=(19, 13, 9), num_global=info.num_input_global_channels)
    sym = (np.arange(n) * 3 % 8).astype(np.int32)
    with_t = oracle.OracleModel(path).forward(sp, gl, sym)
    without = oracle.OracleModel(path, load_time_transforms=False).forward(sp, gl, sym)
    total = 0.0
    for k in with_t:
        d = np.abs(with_t[k] - without[k]).max()
        total += d
        assert d <= 2e-5 * max(1.0, np.abs(without[k]).max()), (path, k, d)
    if exercised:
        assert total > 0.0, f"{path}: the transform changed nothing"


@pytest.mark.parametrize("path", TRAINED, ids=lambda p: p.split("/")[-1].split("-s")[0].split(".")[0])
def test_transform_keeps_trained_net_outputs(path):
    _check(path, 3, exercised=path not in TRANSFORMER_MODELS)


@pytest.mark.parametrize("cfg_index,n", [(0, 3), (1, 3), (2, 2), (4, 1)], ids=["C0", "C1", "C2", "C4"])
def test_transform_keeps_synthetic_net_outputs(model_dir, cfg_index, n):
    _check(modelgen.ensure_model(model_dir, modelgen.configs()[cfg_index]), n, exercised=True)
