"""KataGo's GPU acceptance statistics (GpuErrorStats,
testnnevalcanary.cpp:249-434), restated over post-processed outputs, and the
inputs its test runs them on here: the 300 positions of the featurizer
fixture (tests/golden/featurize_golden.json.gz, rows built by KataGo's own
fillRowV7 from seeded random games under every ruleset, 19x19 to 5x5
tensors).

An output is a dict of one position's post-processed NNOutput: "policy"
(probabilities, nn_x*nn_y+1, -1 where illegal), "values" (whiteWinProb,
whiteLossProb, whiteNoResultProb, whiteScoreMean, whiteScoreMeanSq,
whiteLead, varTimeLeft, shorttermWinlossError, shorttermScoreError) and
"ownership" (nn_x*nn_y)."""
from __future__ import annotations

import functools
import gzip
import json
import math
import os

import numpy as np

from helpers import GOLDEN
from oracle import postprocess as pp

# Reference thresholds (testnnevalcanary.cpp:727-749):
# (winrate %, score, top policy delta %, policy KL) for the 99th percentile
# and the maximum.
FP32_99 = (0.45, 0.225, 0.45, 0.0006)
FP32_MAX = (1.35, 0.900, 1.35, 0.0012)
FP16_99 = (2.0, 1.00, 2.50, 0.0020)
FP16_MAX = (5.0, 3.00, 6.00, 0.0040)

FIELDS = ["winrateError", "leadError", "scoreMeanError", "scoreStdevError", "topPolicyDiff", "policyKLDiv",
          "shorttermWinlossErrorError", "shorttermScoreErrorError", "ownershipError"]


class GpuErrorStats:
    """Errors of candidate outputs against base (reference) outputs."""

    def __init__(self):
        self.v = {k: [] for k in FIELDS}

    def append(self, base, other):
        """appendStats (testnnevalcanary.cpp:259-307)."""
        b, o = base["values"], other["values"]
        self.v["winrateError"].append(abs(0.5 * (b[0] - b[1]) - 0.5 * (o[0] - o[1])) + abs(b[2] - o[2]))
        self.v["leadError"].append(abs(b[5] - o[5]))
        self.v["scoreMeanError"].append(abs(b[3] - o[3]))
        sd = lambda v: math.sqrt(max(0.0, v[4] - v[3] * v[3]))
        self.v["scoreStdevError"].append(abs(sd(b) - sd(o)))
        # First index of the largest base probability (illegal entries are -1).
        top = int(np.argmax(base["policy"]))
        self.v["topPolicyDiff"].append(abs(float(base["policy"][top]) - float(other["policy"][top])))
        bp = base["policy"].astype(np.float64)
        op = other["policy"].astype(np.float64)
        on = bp > 1e-30
        self.v["policyKLDiv"].append(float((bp[on] * (np.log(bp[on]) - np.log(op[on]))).sum()))
        self.v["shorttermWinlossErrorError"].append(abs(b[7] - o[7]))
        self.v["shorttermScoreErrorError"].append(abs(b[8] - o[8]))
        self.v["ownershipError"].extend(np.abs(base["ownership"].astype(np.float64) - other["ownership"]).tolist())

    def _sorted(self, k):
        return sorted(self.v[k])

    def average(self, k):
        return sum(self.v[k]) / len(self.v[k])

    def p90(self, k):
        s = self._sorted(k)
        return s[(len(s) - 1) * 9 // 10]

    def p99(self, k):
        s = self._sorted(k)
        return s[(len(s) - 1) * 99 // 100]

    def max(self, k):
        return self._sorted(k)[-1]

    def failures(self, thresholds, which):
        """checkStats99 / checkStatsMax (testnnevalcanary.cpp:333-359): the
        list of (field, value, bound) that exceed their bound."""
        wr, score, tpd, pkld = thresholds
        get = self.p99 if which == "99" else self.max
        own = wr * (1.75 if which == "99" else 4.0)
        checks = [("winrateError", 100 * get("winrateError"), wr), ("leadError", get("leadError"), score),
                  ("scoreMeanError", get("scoreMeanError"), score), ("scoreStdevError", get("scoreStdevError"), score * 0.6),
                  ("topPolicyDiff", 100 * get("topPolicyDiff"), tpd), ("policyKLDiv", get("policyKLDiv"), pkld),
                  ("shorttermWinlossErrorError", 100 * get("shorttermWinlossErrorError"), wr * 1.8),
                  ("shorttermScoreErrorError", get("shorttermScoreErrorError"), score * 0.75),
                  ("ownershipError", 100 * get("ownershipError"), own)]
        return [c for c in checks if not c[1] <= c[2]]

    def report(self, name):
        """reportStats (testnnevalcanary.cpp:362-432): average, 90%, 99% and
        max of each field, percent fields scaled by 100 as there."""
        pct = {"winrateError", "topPolicyDiff", "shorttermWinlossErrorError", "ownershipError"}
        lines = []
        for k in FIELDS:
            s = 100.0 if k in pct else 1.0
            lines.append(f"{name} {k:27s} " + "  ".join(f"{s * f(k):9.5f}" for f in (self.average, self.p90, self.p99, self.max)))
        return "\n".join(lines)


@functools.lru_cache(maxsize=1)
def positions():
    with gzip.open(os.path.join(GOLDEN, "featurize_golden.json.gz"), "rt") as f:
        return json.load(f)["positions"]


def rows(fx):
    """The fixture's input row (NHWC) and global features."""
    c, hw = 22, fx["nnx"] * fx["nny"]
    digits = fx["spatial_nhwc_bits"]
    bits = np.unpackbits(np.frombuffer(bytes.fromhex(digits + ("0" if len(digits) % 2 else "")), np.uint8))
    return bits[: hw * c].astype(np.float32), np.asarray(fx["global"], np.float32)


def legal_moves(fx):
    """Empty on-board points other than the ko point, and pass: the
    positions carry no legality record, so suicide is not excluded (it
    changes which entries the softmax covers, for base and candidate
    alike)."""
    nx, ny, xs, ys = fx["nnx"], fx["nny"], fx["x_size"], fx["y_size"]
    legal = np.zeros(nx * ny + 1, bool)
    colors = fx["colors"][0]
    for y in range(ys):
        for x in range(xs):
            legal[y * nx + x] = colors[y * xs + x] == 0 and y * xs + x != fx["ko_point"][0]
    legal[nx * ny] = True
    return legal


def post_params(path):
    """ModelPostProcessParams from the model file's header (desc.cpp: the
    multipliers follow name, version and the input counts from version 13
    on; defaults before), with the output scale the caller passes."""
    with gzip.open(path, "rb") as f:
        head = f.read(4096).split(b"\n")
    version = int(head[1])
    if version < 13:
        return version, pp.PostProcessParams()
    m = [float(x) for x in head[5:11]]  # after tdScoreMultiplier
    return version, pp.PostProcessParams(score_mean_multiplier=m[0], score_stdev_multiplier=m[1], lead_multiplier=m[2],
                                         variance_time_multiplier=m[3], shortterm_value_error_multiplier=m[4],
                                         shortterm_score_error_multiplier=m[5])


def post(raw, i, fx, version, params, scale=1.0):
    """Row i of raw getOutput outputs, post-processed as NNEvaluator does."""
    pol, values, own = pp.postprocess_row(
        raw["policy"][i] * scale, raw["value"][i] * scale, raw["score"][i] * scale, raw["ownership"][i] * scale,
        legal_moves(fx), nn_x=fx["nnx"], nn_y=fx["nny"], board_x=fx["x_size"], board_y=fx["y_size"],
        white_to_move=fx["next_player"] == 2, no_result_disabled=False, passing_hacks=False, temperature=1.0,
        model_version=version, params=params)
    return {"policy": pol, "values": values, "ownership": own}
