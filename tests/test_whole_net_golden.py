"""The oracle against whole-network outputs recorded by KataGo's own tests.

These are the only pins the reference itself wrote for a whole net end to
end: the model parser and load-time transforms, every block kind of these
nets, the heads, the symmetry handling of getOutput, the score-channel
routing per model version and the evaluator's post-processing. Inputs are the
rows KataGo's own featurizer builds for each position (fixture written by
tests/golden/make_whole_net_golden.py from oracle/_ref, KataGo's nninputs
and game sources compiled as they are):

* runNNOnTinyBoardTest.txt (g170-b6c96, model version 8, 5x5 board in a 6x6
  tensor, symmetry 3) and runNNSymmetriesTest.txt (g103-b6c96, model version
  5, 9x13 board in a 13x13 tensor, symmetries 0-7): printed to 0.01% for
  values, 0.01 for scores, permille for policy and ownership by
  NNOutput::debugPrint; compared at one printed step;
* tinymodel.cpp:135-490 (tiny ReLU and Mish nets, model versions 9 and 11,
  19x19 and 13x6 boards in 19x19 tensors, symmetries 6, 7, 1): with that
  test's own tolerances.

The reference produced these numbers with its CUDA backend in fp32
(runsearchtests.sh:40,44) and on GPUs in general (tinymodel.cpp).
"""
import numpy as np
import pytest

from helpers import GOLDEN
from oracle import oracle
from oracle.postprocess import PostProcessParams, postprocess_row
from katago_amd import nn
from whole_net_golden import check_printed, check_tinymodel, inputs_of, load_cases

CASES = load_cases()


def oracle_post(case):
    path = f"{GOLDEN}/{case['model']}"
    info = nn.LoadedModel(path).info
    om = oracle.OracleModel(path, case["nnx"], case["nny"])
    sp, gl = inputs_of(case)
    raw = om.forward(sp, gl, np.array([case["symmetry"]], np.int32))
    # The oracle's outputs are the net's logits with the output multiplier
    # already applied (no scale8 transform on the CPU path).
    return postprocess_row(raw["policy"][0], raw["value"][0], raw["score"][0], raw["ownership"][0], case["legal"],
                           nn_x=case["nnx"], nn_y=case["nny"], board_x=case["x"], board_y=case["y"],
                           white_to_move=case["pla"] == "w", no_result_disabled=case["no_result_disabled"],
                           passing_hacks=False, temperature=1.0, model_version=info.model_version,
                           params=PostProcessParams(output_scale_multiplier=1.0))


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_reference_whole_net_outputs(case):
    policy, values, own = oracle_post(case)
    if case["check"] == "printed":
        errs = check_printed(case, policy, values, own)
    else:
        errs = check_tinymodel(case, policy, values, own)
    assert not errs, "\n".join(errs[:20])
