"""TEST INFRASTRUCTURE ONLY: CPU restatement of NNEvaluator's post-processing
of raw network outputs (/root/reference/cpp/neuralnet/nneval.cpp:946-1240),
the checker for the device post-processing kernel.

Imported only by tests/. Follows the reference's arithmetic types: the policy
in float32 with a sequential sum, value and score in float64.

Parity pins (tests/test_postprocess.py): closed forms (uniform policy, the
95% pass cap, temperature as a power of the probabilities, softmax sums,
perspective flips, the softplus-based score stdev, the short-term error
formulas of each model-version branch), hand-computed known answers, and the
reference's own invariants (illegal moves -1, off-board ownership 0), and
its two errors for non-finite results (a NaN logit of a legal move, a NaN
value or score field).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass
class PostProcessParams:
    """ModelPostProcessParams (desc.h:468-481) with the defaults of
    desc.cpp:2252-2261."""
    output_scale_multiplier: float = 1.0
    score_mean_multiplier: float = 20.0
    score_stdev_multiplier: float = 20.0
    lead_multiplier: float = 20.0
    variance_time_multiplier: float = 40.0
    shortterm_value_error_multiplier: float = 0.25
    shortterm_score_error_multiplier: float = 30.0


def soft_plus(x: float) -> float:
    """nneval.cpp:753-759."""
    return x if x > 40.0 else math.log(1.0 + math.exp(x))


def raw_score_fields(score, model_version: int):
    """The six NNOutput score fields as a backend fills them from the score
    channels (eigenbackend.cpp:2571-2615): (scoreMean, scoreMeanSq, lead,
    varTimeLeft, shorttermWinlossError, shorttermScoreError)."""
    s = [float(x) for x in score]
    if model_version >= 9:
        return s[0], s[1], s[2], s[3], s[4], s[5]
    if model_version >= 8:
        return s[0], s[1], s[2], s[3], 0.0, 0.0
    if model_version >= 4:
        return s[0], s[1], s[0], 0.0, 0.0, 0.0
    # Version 3 has one score channel; its square stands in for the second
    # moment (eigenbackend.cpp:2596-2604).
    return s[0], s[0] * s[0], s[0], 0.0, 0.0, 0.0


def postprocess_row(policy, value, score, ownership, legal, *, nn_x: int, nn_y: int, board_x: int, board_y: int,
                    white_to_move: bool, no_result_disabled: bool, passing_hacks: bool, temperature: float,
                    model_version: int, params: PostProcessParams):
    """One row: raw policy[nn_x*nn_y+1], value[3], score channels, ownership
    [nn_x*nn_y], legal[nn_x*nn_y+1] -> (policy probs, values[9], ownership).
    values = whiteWinProb, whiteLossProb, whiteNoResultProb, whiteScoreMean,
    whiteScoreMeanSq, whiteLead, varTimeLeft, shorttermWinlossError,
    shorttermScoreError."""
    hw = nn_x * nn_y
    policy_size = hw + 1
    f32 = np.float32
    # Policy, nneval.cpp:946-1024 (float arithmetic).
    scaling = f32(params.output_scale_multiplier) / f32(temperature)
    pol = np.zeros(policy_size, np.float32)
    max_policy = f32(-1e25)
    legal_count = 0
    for i in range(policy_size):
        if legal[i]:
            legal_count += 1
            v = f32(policy[i]) * scaling
        else:
            v = f32(-1e30)
        pol[i] = v
        if v > max_policy:
            max_policy = v
    if legal_count <= 0:
        raise ValueError("no legal move")
    policy_sum = f32(0.0)
    if passing_hacks:
        for i in range(policy_size - 1):
            pol[i] = np.exp(f32(pol[i] - max_policy))
            policy_sum = f32(policy_sum + pol[i])
        i = policy_size - 1
        pol[i] = max(f32(1e-20), min(np.exp(f32(pol[i] - max_policy)), f32(policy_sum * f32(19.0))))
        policy_sum = f32(policy_sum + pol[i])
    else:
        for i in range(policy_size):
            pol[i] = np.exp(f32(pol[i] - max_policy))
            policy_sum = f32(policy_sum + pol[i])
    if not np.isfinite(policy_sum):
        raise ValueError("Got nonfinite for policy sum")
    out_pol = np.empty(policy_size, np.float32)
    for i in range(policy_size):
        if policy_sum <= 0.0:
            out_pol[i] = f32(1.0) / f32(legal_count) if legal[i] else f32(-1.0)
        else:
            out_pol[i] = pol[i] / policy_sum if legal[i] else f32(-1.0)

    # Value and score, nneval.cpp:1097-1216 (double arithmetic), version >= 4.
    if model_version < 4:
        raise ValueError("post-processing needs model version >= 4")
    osm = float(params.output_scale_multiplier)
    sm, smsq, lead, vtl, stw, sts = raw_score_fields(score, model_version)
    win_logits = float(value[0]) * osm
    loss_logits = float(value[1]) * osm
    no_result_logits = float(value[2]) * osm
    if no_result_disabled:
        no_result_logits -= 100000.0
    max_logits = max(win_logits, loss_logits, no_result_logits)
    win = math.exp(win_logits - max_logits)
    loss = math.exp(loss_logits - max_logits)
    no_result = math.exp(no_result_logits - max_logits)
    if no_result_disabled:
        no_result = 0.0
    prob_sum = win + loss + no_result
    win /= prob_sum
    loss /= prob_sum
    no_result /= prob_sum
    score_mean = sm * osm * params.score_mean_multiplier
    score_stdev = soft_plus(smsq * osm) * params.score_stdev_multiplier
    score_mean_sq = score_mean * score_mean + score_stdev * score_stdev
    lead_v = lead * osm * params.lead_multiplier
    var_time_left = soft_plus(vtl * osm) * params.variance_time_multiplier
    score_mean *= 1.0 - no_result
    score_mean_sq *= 1.0 - no_result
    lead_v *= 1.0 - no_result
    if model_version >= 14:
        s = soft_plus(stw * osm * 0.5)
        st_wl = math.sqrt(s * s * params.shortterm_value_error_multiplier)
        s = soft_plus(sts * osm * 0.5)
        st_sc = math.sqrt(s * s * params.shortterm_score_error_multiplier)
    elif model_version >= 10:
        st_wl = math.sqrt(soft_plus(stw * osm) * params.shortterm_value_error_multiplier)
        st_sc = math.sqrt(soft_plus(sts * osm) * params.shortterm_score_error_multiplier)
    else:
        st_wl = soft_plus(stw * osm)
        st_sc = soft_plus(sts * osm) * 10.0
    # nneval.cpp:1167-1184.
    if not all(math.isfinite(v) for v in (prob_sum, score_mean, score_mean_sq, lead_v, var_time_left, st_wl, st_sc)):
        raise ValueError("Got nonfinite for nneval value")
    if white_to_move:
        vals = [win, loss, no_result, score_mean, score_mean_sq, lead_v]
    else:
        vals = [loss, win, no_result, -score_mean, score_mean_sq, -lead_v]
    if model_version >= 9:
        vals += [var_time_left, st_wl, st_sc]
    else:
        vals += [-1.0, -1.0, -1.0]

    # Ownership, nneval.cpp:1222-1241.
    own = np.zeros(hw, np.float32)
    for pos in range(hw):
        y, x = divmod(pos, nn_x)
        if y >= board_y or x >= board_x:
            own[pos] = 0.0
        else:
            t = math.tanh(float(ownership[pos]) * osm)
            own[pos] = t if white_to_move else -t
    return out_pol, np.array(vals, np.float64), own
