"""KataGo's canary tests (Tests::runCanaryTests, testnnevalcanary.cpp:14-245):
a trained net on six named positions must put most of its policy on the known
move and give plausible values (winrate, lead, score mean), under every
symmetry. The positions are KataGo's own fillRowV7 rows
(tests/golden/canary_golden.json.gz, written by make_canary_golden.py).

The nets are the reference's three trained version-17 test nets (transformer
and nested-bottleneck trunks, all of trunk spatial conv depth <= 21, so the
reference's lenience for small nets applies, testnnevalcanary.cpp:27-32),
which pass every assertion, and g170-b6c96 (version 8), whose policy passes
but whose lead and score estimates at these positions are outside the
canaries' ranges on the reference's own arithmetic (the oracle gives the same
numbers, e.g. a lead of -103 points at komi -7 where -21 to -7 are allowed),
so only its policy assertions are checked.

On the CPU the checks run on the oracle with the post-processing
restatement; on the GPU on getOutput with the device post-processing
(HipBackend::getOutputPostProcessed), in fp32 and fp16.
"""
import gzip
import json
import os

import numpy as np
import pytest

from katago_amd import nn
from helpers import G170_MODEL
from oracle import oracle
from oracle.postprocess import PostProcessParams, postprocess_row

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with gzip.open(os.path.join(GOLDEN, "canary_golden.json.gz"), "rt") as _f:
    FIXTURE = json.load(_f)
NNX, NNY = FIXTURE["nnx"], FIXTURE["nny"]
CANARIES = FIXTURE["canaries"]
LENIENCE = FIXTURE["lenience_small_net"]
GTP_COLUMNS = "ABCDEFGHJKLMNOPQRST"  # Location::ofString: no I
VALUE_INDEX = {"white_win": 0, "white_no_result": 2, "white_score_mean": 3, "white_lead": 5}


def policy_index(point, x_size, y_size):
    """NNPos::locToPos of a GTP coordinate (or pass) on an x_size x y_size
    board in the NNX x NNY tensor."""
    if point == "pass":
        return NNX * NNY
    x = GTP_COLUMNS.index(point[0])
    y = y_size - int(point[1:])
    assert 0 <= x < x_size and 0 <= y < y_size, point
    return y * NNX + x


NETS = {"b7c96h3tfrs": "b7c96h3tfrs-test5-cnorm.bin.gz", "b7c96h6kv3qk32v16tflrs": "b7c96h6kv3qk32v16tflrs-fson-bnh.bin.gz",
        "b4c256h4nbttflrs": "b4c256h4nbttflrs-fson-silu-rsnh.bin.gz", "g170-b6c96": os.path.basename(G170_MODEL)}
POLICY_ONLY = {"g170-b6c96"}


def failed_checks(canary, policy, values, policy_only=False):
    """The canary's assertions that policy probabilities [NNX*NNY+1] and
    values [9] (white's perspective) do not meet, as text."""
    fails = []
    for quantity, op, bound, kind in canary["checks"]:
        if policy_only and not quantity.startswith("policy:"):
            continue
        if kind is not None:
            bound = bound + LENIENCE[kind] if op in ("<", "<=") else bound - LENIENCE[kind]
        if quantity.startswith("policy:"):
            v = float(policy[policy_index(quantity.split(":")[1], canary["x_size"], canary["y_size"])])
        else:
            v = float(values[VALUE_INDEX[quantity]])
        ok = {"<": v < bound, "<=": v <= bound, ">": v > bound, ">=": v >= bound}[op]
        if not ok:
            fails.append(f"{canary['name']}: {quantity} = {v:.4f}, expected {op} {bound:.4f}")
    return fails


def rows():
    sp = np.array([c["spatial_nhwc"] for c in CANARIES], np.float32)
    gl = np.array([c["global"] for c in CANARIES], np.float32)
    return sp, gl


def post_inputs():
    legal = np.array([c["legal"] for c in CANARIES], np.uint8)
    info = np.array([nn.post_info(True, c["pla"] == "w", c["no_result_disabled"], False, c["x_size"], c["y_size"])
                     for c in CANARIES], np.int32)
    return legal, info


def test_fixture_positions_and_checks():
    """The fixture holds the six canaries with the reference's board shapes,
    legal-move counts (empty points + pass) and check lists."""
    assert [c["name"] for c in CANARIES] == ["opening-E16", "opening-P15", "corner-Q2", "corner-komi-7", "corner-komi21",
                                             "rect16x11-N3"]
    for c in CANARIES:
        area = c["x_size"] * c["y_size"]
        assert len(c["spatial_nhwc"]) == 22 * NNX * NNY and len(c["global"]) == 19
        stones = sum(1 for p in range(NNX * NNY) if any(c["spatial_nhwc"][p * 22 + k] for k in (1, 2)))
        assert stones <= c["turns"] and sum(c["legal"]) <= area - stones + 1
    assert CANARIES[5]["x_size"] == 16 and CANARIES[5]["y_size"] == 11
    assert policy_index("E16", 19, 19) == 3 * 19 + 4 and policy_index("N3", 16, 11) == 8 * 19 + 12


@pytest.mark.parametrize("net", list(NETS))
def test_oracle_passes_canaries(net):
    """The oracle (KataGo's Eigen backend restated) with the post-processing
    restatement, symmetries 0 and 5: every canary assertion holds."""
    path = os.path.join(GOLDEN, NETS[net])
    om = oracle.OracleModel(path)
    lm = nn.LoadedModel(path)
    sp, gl = rows()
    fails = []
    for symmetry in (0, 5):
        out = om.forward(sp, gl, np.full(len(CANARIES), symmetry))
        for i, c in enumerate(CANARIES):
            policy, values, _ = postprocess_row(out["policy"][i], out["value"][i], out["score"][i], out["ownership"][i],
                                                c["legal"], nn_x=NNX, nn_y=NNY, board_x=c["x_size"], board_y=c["y_size"],
                                                white_to_move=c["pla"] == "w", no_result_disabled=c["no_result_disabled"],
                                                passing_hacks=False, temperature=1.0, model_version=lm.info.model_version,
                                                params=PostProcessParams(
                                                    output_scale_multiplier=lm.info.output_scale_multiplier))
            fails += [f"symmetry {symmetry}: {f}" for f in failed_checks(c, policy, values, net in POLICY_ONLY)]
    assert not fails, "\n".join(fails)


@pytest.mark.gpu
@pytest.mark.parametrize("fp16", [False, True], ids=["fp32", "fp16"])
@pytest.mark.parametrize("net", list(NETS))
def test_device_passes_canaries(net, fp16):
    """getOutput with the device post-processing, all eight symmetries of the
    six canaries in one batch: every canary assertion holds."""
    lm = nn.LoadedModel(os.path.join(GOLDEN, NETS[net]))
    n = 8 * len(CANARIES)
    h = nn.ComputeHandle(nn.ComputeContext(lm, NNX, NNY, use_fp16=fp16, auto_tune=False), max_batch=n)
    sp, gl = rows()
    legal, info = post_inputs()
    reps = np.repeat(np.arange(len(CANARIES)), 8)
    sym = np.tile(np.arange(8), len(CANARIES)).astype(np.int32)
    out = h.get_output_post(sp[reps], gl[reps], legal[reps], info[reps], symmetry=sym)
    fails = []
    for r, i in enumerate(reps):
        fails += [f"symmetry {sym[r]}: {f}"
                  for f in failed_checks(CANARIES[i], out["policy"][r], out["values"][r], net in POLICY_ONLY)]
    assert not fails, "\n".join(fails)


@pytest.mark.gpu
@pytest.mark.parametrize("net", ["b4c256h4nbttflrs", "g170-b6c96"])
def test_low_latency_mode_passes_canaries(net):
    """The handle's low-latency mode (split-K 3x3 convs, handles of at most 16
    rows), one position per call as a single-threaded search evaluates:
    every canary assertion holds under every symmetry."""
    lm = nn.LoadedModel(os.path.join(GOLDEN, NETS[net]))
    h = nn.ComputeHandle(nn.ComputeContext(lm, NNX, NNY, use_fp16=True, auto_tune=False, low_latency=True), max_batch=1)
    sp, gl = rows()
    legal, info = post_inputs()
    fails = []
    for i, c in enumerate(CANARIES):
        for s in range(8):
            out = h.get_output_post(sp[i:i + 1], gl[i:i + 1], legal[i:i + 1], info[i:i + 1], symmetry=np.array([s], np.int32))
            fails += [f"symmetry {s}: {f}" for f in failed_checks(c, out["policy"][0], out["values"][0], net in POLICY_ONLY)]
    assert not fails, "\n".join(fails)
