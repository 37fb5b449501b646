"""getOutput on the GPU against the whole-network outputs KataGo's own tests
recorded (see tests/test_whole_net_golden.py for the records and inputs):
the raw rows of getOutput post-processed by the CPU restatement, and the rows
post-processed on the device (HipBackend::getOutputPostProcessed), each in
fp32 and fp16.

Tolerances: fp32 as for the oracle (one printed step, three for the g103
record's value fields; one permille for policy and ownership;
tinymodel.cpp's own tolerances). fp16: twice the spread between the
reference's own fp16 and fp32 records of runNNSymmetriesTest (per value
field, at least one printed step; policy and ownership in permille), and
tinymodel.cpp's own tolerances, which the reference applies to every GPU
backend in any precision.
"""
import numpy as np
import pytest

from helpers import GOLDEN
from katago_amd import nn
from oracle.postprocess import PostProcessParams, postprocess_row
from whole_net_golden import (VALUE_STEPS, check_printed, check_tinymodel, inputs_of, load_cases,
                              reference_fp16_spread)

pytestmark = pytest.mark.gpu

CASES = load_cases()
# One getOutput batch per model and tensor size: the g103 record's eight
# symmetries run as eight rows of one batch.
GROUPS = {}
for c in CASES:
    GROUPS.setdefault((c["model"], c["nnx"], c["nny"]), []).append(c)


def _check(case, policy, values, own, fp16):
    if case["check"] == "tinymodel":
        return check_tinymodel(case, policy, values, own)
    if not fp16:
        return check_printed(case, policy, values, own)
    spread = reference_fp16_spread()
    steps = VALUE_STEPS.get(case["model"], 1.0)
    return check_printed(case, policy, values, own,
                         value_tol=lambda name, step: max(2.0 * spread[name], steps * step),
                         policy_slack=lambda e: 2 * spread["policy_permille"] + 1,
                         own_slack=lambda e: 2 * spread["ownership_permille"] + 1)


@pytest.mark.parametrize("fp16", [False, True], ids=["fp32", "fp16"])
@pytest.mark.parametrize("key", list(GROUPS), ids=[f"{m.split('-')[0].split('.')[0]}-{x}x{y}" for m, x, y in GROUPS])
def test_get_output_matches_reference_whole_net_outputs(key, fp16):
    model, nnx, nny = key
    cases = GROUPS[key]
    lm = nn.LoadedModel(f"{GOLDEN}/{model}")
    h = nn.ComputeHandle(nn.ComputeContext(lm, nnx, nny, use_fp16=fp16, auto_tune=False), max_batch=len(cases))
    rows = [inputs_of(c) for c in cases]
    sp = np.concatenate([r[0] for r in rows])
    gl = np.concatenate([r[1] for r in rows])
    sym = np.array([c["symmetry"] for c in cases], np.int32)
    legal = np.array([c["legal"] for c in cases], np.uint8)
    info = np.array([nn.post_info(True, c["pla"] == "w", c["no_result_disabled"], False, c["x"], c["y"]) for c in cases],
                    np.int32)
    raw = h.get_output(sp, gl, sym)
    post = h.get_output_post(sp, gl, legal, info, symmetry=sym)
    errs = []
    for i, c in enumerate(cases):
        # Raw rows, post-processed by the CPU restatement with the model's
        # output multiplier (the device net carries the scale8 transform).
        p, v, o = postprocess_row(raw["policy"][i], raw["value"][i], raw["score"][i], raw["ownership"][i], c["legal"],
                                  nn_x=nnx, nn_y=nny, board_x=c["x"], board_y=c["y"], white_to_move=c["pla"] == "w",
                                  no_result_disabled=c["no_result_disabled"], passing_hacks=False, temperature=1.0,
                                  model_version=lm.info.model_version,
                                  params=PostProcessParams(output_scale_multiplier=lm.info.output_scale_multiplier))
        errs += [f"{c['name']} (getOutput): {e}" for e in _check(c, p, v, o, fp16)]
        errs += [f"{c['name']} (device post-processing): {e}" for e in
                 _check(c, post["policy"][i], post["values"][i].astype(np.float64), post["ownership"][i], fp16)]
    assert not errs, "\n".join(errs[:30])
