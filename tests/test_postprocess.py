"""Post-processing of raw outputs into NNEvaluator's results
(nneval.cpp:946-1240): the CPU restatement (oracle/postprocess.py) pinned by
closed forms and known answers, then the device kernel and the getOutput
path checked against it on the GPU.

Tolerances (device vs restatement): policy probabilities rtol 1e-5 (float32
sums over up to 362 terms in another order), values rtol 1e-6 (double
arithmetic on both sides, rounded to float32), ownership atol 1e-6 (tanhf vs
double tanh).
"""
import math

import numpy as np
import pytest

from katago_amd import modelgen, nn
from helpers import G170_MODEL
from oracle import postprocess as pp

HW = 361
P = pp.PostProcessParams()


def _row(policy, value=(0.0, 0.0, 0.0), score=(0.0,) * 6, own=None, legal=None, **kw):
    args = dict(nn_x=19, nn_y=19, board_x=19, board_y=19, white_to_move=True, no_result_disabled=False,
                passing_hacks=False, temperature=1.0, model_version=15, params=P)
    args.update(kw)
    own = np.zeros(HW, np.float32) if own is None else own
    legal = np.ones(HW + 1, bool) if legal is None else legal
    return pp.postprocess_row(np.asarray(policy, np.float32), value, score, own, legal, **args)


def test_uniform_logits_give_uniform_legal_moves():
    legal = np.zeros(HW + 1, bool)
    legal[[0, 5, 100, 360, HW]] = True
    pol, _, _ = _row(np.full(HW + 1, 3.0), legal=legal)
    assert np.allclose(pol[legal], 0.2, rtol=1e-6)
    assert (pol[~legal] == -1.0).all()


def test_pass_cap_is_nineteen_twentieths():
    # Pass logit 10 above 361 moves at 0: exp(10)=22026 > 19 * 361 * 1, so the
    # pass prior is capped at 19x the other moves' total: exactly 95%.
    logits = np.zeros(HW + 1)
    logits[HW] = 10.0
    pol, _, _ = _row(logits, passing_hacks=True)
    assert pol[HW] == pytest.approx(0.95, rel=1e-6)
    assert pol[:HW].sum() == pytest.approx(0.05, rel=1e-5)
    pol2, _, _ = _row(logits, passing_hacks=False)
    assert pol2[HW] == pytest.approx(math.exp(10) / (math.exp(10) + HW), rel=1e-5)


def test_temperature_raises_probabilities_to_a_power():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal(HW + 1)
    p1, _, _ = _row(logits)
    p_half, _, _ = _row(logits, temperature=0.5)
    q = p1.astype(np.float64) ** 2
    assert np.allclose(p_half, q / q.sum(), rtol=1e-4)
    assert p1.sum() == pytest.approx(1.0, rel=1e-5)


def test_output_scale_multiplier_scales_logits():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal(HW + 1)
    p2, _, _ = _row(logits, params=pp.PostProcessParams(output_scale_multiplier=2.0))
    q = np.exp(2.0 * logits - (2.0 * logits).max())
    assert np.allclose(p2, q / q.sum(), rtol=1e-4)


def test_value_known_answers_and_perspective():
    # Equal logits: 1/3 each; score fields at raw 0 give softplus(0) = ln 2.
    _, v, _ = _row(np.zeros(HW + 1), value=(0.0, 0.0, 0.0), score=(0.5, 0.0, 0.25, 0.0, 0.0, 0.0))
    assert v[:3] == pytest.approx([1 / 3, 1 / 3, 1 / 3], rel=1e-12)
    mean = 0.5 * 20.0 * (2 / 3)
    assert v[3] == pytest.approx(mean, rel=1e-12)
    assert v[4] == pytest.approx(((0.5 * 20.0) ** 2 + (20.0 * math.log(2)) ** 2) * (2 / 3), rel=1e-12)
    assert v[5] == pytest.approx(0.25 * 20.0 * (2 / 3), rel=1e-12)
    assert v[6] == pytest.approx(40.0 * math.log(2), rel=1e-12)  # unscaled by noResult
    assert v[7] == pytest.approx(0.5 * math.log(2), rel=1e-12)  # sqrt(ln2^2 * 0.25), version >= 14
    assert v[8] == pytest.approx(math.log(2) * math.sqrt(30.0), rel=1e-12)
    _, b, _ = _row(np.zeros(HW + 1), value=(1.0, 0.0, -1.0), score=(0.5, 0.0, 0.25, 0.0, 0.0, 0.0), white_to_move=False)
    _, w, _ = _row(np.zeros(HW + 1), value=(1.0, 0.0, -1.0), score=(0.5, 0.0, 0.25, 0.0, 0.0, 0.0), white_to_move=True)
    e = math.e
    assert w[0] == pytest.approx(e / (e + 1 + 1 / e), rel=1e-12)
    assert (b[0], b[1], b[2]) == pytest.approx((w[1], w[0], w[2]), rel=1e-12)
    assert (b[3], b[4], b[5]) == pytest.approx((-w[3], w[4], -w[5]), rel=1e-12)


def test_no_result_disabled_rules():
    _, v, _ = _row(np.zeros(HW + 1), value=(0.0, 0.0, 5.0), score=(0.5, 0.0, 0.0, 0.0, 0.0, 0.0), no_result_disabled=True)
    assert v[2] == 0.0 and v[0] + v[1] == pytest.approx(1.0)
    assert v[3] == pytest.approx(10.0, rel=1e-12)  # no (1 - noResult) shrink


def test_shortterm_error_version_branches():
    s = (0.0,) * 6
    ln2 = math.log(2)
    _, v13, _ = _row(np.zeros(HW + 1), score=s, model_version=13)
    assert (v13[7], v13[8]) == pytest.approx((math.sqrt(ln2 * 0.25), math.sqrt(ln2 * 30.0)), rel=1e-12)
    _, v9, _ = _row(np.zeros(HW + 1), score=s, model_version=9)
    assert (v9[7], v9[8]) == pytest.approx((ln2, 10 * ln2), rel=1e-12)
    _, v8, _ = _row(np.zeros(HW + 1), score=(0.0,) * 4, model_version=8)
    assert (v8[6], v8[7], v8[8]) == (-1.0, -1.0, -1.0)


@pytest.mark.parametrize("version", [14, 15, 17])
def test_shortterm_error_squared_softplus_branch(version):
    """Model versions 14+ (nneval.cpp:1148-1157): the two shortterm outputs
    are variances the training model produces as softplus(x / 2)^2
    (SoftPlusWithGradientFloorFunction with square=True,
    model_pytorch.py:111-131), so the error is sqrt(multiplier) *
    softplus(x / 2). Known answers away from 0, where the v10-13 branch
    sqrt(softplus(x) * multiplier) gives other values."""
    for xw, xs in [(2.0, -3.0), (-1.5, 4.0), (6.0, 0.7)]:
        _, v, _ = _row(np.zeros(HW + 1), score=(0.0, 0.0, 0.0, 0.0, xw, xs), model_version=version)
        sp = lambda x: math.log1p(math.exp(x))
        assert v[7] == pytest.approx(math.sqrt(0.25) * sp(xw / 2), rel=1e-12)
        assert v[8] == pytest.approx(math.sqrt(30.0) * sp(xs / 2), rel=1e-12)
        _, v13, _ = _row(np.zeros(HW + 1), score=(0.0, 0.0, 0.0, 0.0, xw, xs), model_version=13)
        assert abs(v13[7] - v[7]) > 1e-3 and abs(v13[8] - v[8]) > 1e-3
    # x = 2 ln(e - 1): softplus(x / 2) = 1 exactly, so the errors are the
    # square roots of the multipliers.
    x = 2 * math.log(math.e - 1)
    _, v, _ = _row(np.zeros(HW + 1), score=(0.0, 0.0, 0.0, 0.0, x, x), model_version=version)
    assert (v[7], v[8]) == pytest.approx((0.5, math.sqrt(30.0)), rel=1e-12)


def test_ownership_tanh_sign_and_off_board_zero():
    own = np.full(HW, 0.5, np.float32)
    _, _, ow = _row(np.zeros(HW + 1), own=own, board_x=9, board_y=13, white_to_move=False)
    grid = ow.reshape(19, 19)
    assert np.allclose(grid[:13, :9], -math.tanh(0.5), rtol=1e-6)
    assert (grid[13:, :] == 0).all() and (grid[:, 9:] == 0).all()


def test_no_legal_move_is_an_error():
    with pytest.raises(ValueError):
        _row(np.zeros(HW + 1), legal=np.zeros(HW + 1, bool))


def test_nonfinite_results_are_errors():
    """nneval.cpp:1012-1016 and 1167-1184: a NaN or infinite logit of a
    legal move makes the policy sum non-finite; a NaN value or score field
    makes the value results non-finite. Both are errors. A NaN on an illegal
    move is never read."""
    with np.errstate(invalid="ignore"):
        for bad in (np.nan, np.inf):
            pol = np.zeros(HW + 1, np.float32)
            pol[40] = bad
            with pytest.raises(ValueError, match="nonfinite for policy sum"):
                _row(pol)
        legal = np.ones(HW + 1, bool)
        legal[40] = False
        pol = np.zeros(HW + 1, np.float32)
        pol[40] = np.nan
        probs, _, _ = _row(pol, legal=legal)
        assert probs[40] == -1.0 and np.isclose(probs[legal].sum(), 1.0)
        with pytest.raises(ValueError, match="nonfinite for nneval value"):
            _row(np.zeros(HW + 1), value=(np.nan, 0.0, 0.0))
        for field in range(6):
            score = [0.0] * 6
            score[field] = np.nan
            with pytest.raises(ValueError, match="nonfinite for nneval value"):
                _row(np.zeros(HW + 1), score=tuple(score))


# ---------------------------------------------------------------------------
# GPU


def _random_rows(rng, n, score_c):
    rows_floats = 2 * HW + 1 + 3 + score_c
    raw = rng.standard_normal((n, rows_floats)).astype(np.float32) * 2.0
    legal = rng.random((n, HW + 1)) < 0.6
    legal[:, HW] = True
    legal[1] = False
    legal[1, HW] = True  # only pass legal
    info, temp, flags = [], [], []
    for i in range(n):
        f = dict(white_to_move=bool(i % 2), no_result_disabled=bool(i % 3 == 0), passing_hacks=bool(i % 4 == 1),
                 board_x=(9, 13, 19)[i % 3], board_y=(9, 13, 19)[(i // 3) % 3])
        flags.append(f)
        info.append(nn.post_info(**f))
        temp.append((1.0, 0.5, 1.7)[i % 3])
    raw[2, HW] = 12.0  # a capped pass
    return raw, legal, np.array(info, np.int32), np.array(temp, np.float32), flags


def _check_rows(post, raw, legal, temp, flags, score_c, version, params):
    for i in range(raw.shape[0]):
        r = raw[i]
        pol, vals, own = pp.postprocess_row(r[:HW + 1], r[HW + 1:HW + 4], r[HW + 4:HW + 4 + score_c], r[HW + 4 + score_c:],
                                            legal[i], nn_x=19, nn_y=19, temperature=float(temp[i]), model_version=version,
                                            params=params, **flags[i])
        d = post[i]
        np.testing.assert_allclose(d[:HW + 1], pol, rtol=1e-5, atol=1e-9, err_msg=f"row {i} policy")
        np.testing.assert_allclose(d[HW + 1:HW + 10], vals.astype(np.float32), rtol=1e-6, atol=1e-9, err_msg=f"row {i} values")
        np.testing.assert_allclose(d[HW + 10:], own, rtol=0, atol=1e-6, err_msg=f"row {i} ownership")


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["c1", "g170"])
def test_device_postprocess_matches_restatement(which, model_dir):
    path = modelgen.ensure_model(model_dir, modelgen.configs()[1]) if which == "c1" else G170_MODEL
    lm = nn.LoadedModel(path)
    dm = nn.DeviceModel(lm, use_fp16=False)
    n = 12
    h = nn.DeviceHandle(dm, n)
    score_c = lm.info.num_score_value_channels
    version = lm.info.model_version
    rng = np.random.default_rng(7)
    raw, legal, info, temp, flags = _random_rows(rng, n, score_c)
    params = pp.PostProcessParams(output_scale_multiplier=0.9, lead_multiplier=18.0)
    cp = nn.PostParams(params.output_scale_multiplier, params.score_mean_multiplier, params.score_stdev_multiplier,
                       params.lead_multiplier, params.variance_time_multiplier, params.shortterm_value_error_multiplier,
                       params.shortterm_score_error_multiplier)
    d_raw = nn.DeviceBuffer.from_array(raw)
    d_legal = nn.DeviceBuffer.from_array(legal.astype(np.uint8))
    d_info = nn.DeviceBuffer.from_array(info)
    d_temp = nn.DeviceBuffer.from_array(temp)
    d_post = nn.DeviceBuffer(n * (2 * HW + 10) * 4)
    h.postprocess_device(n, d_raw.ptr, d_legal.ptr, d_info.ptr, d_temp.ptr, cp, d_post.ptr)
    post = d_post.to_array(np.float32, (n, 2 * HW + 10))
    _check_rows(post, raw, legal, temp, flags, score_c, version, params)
    # A row without a legal move is an error, as in the reference.
    bad = legal.astype(np.uint8).copy()
    bad[3] = 0
    d_bad = nn.DeviceBuffer.from_array(bad)
    with pytest.raises(nn.StringError, match="no legal move"):
        h.postprocess_device(n, d_raw.ptr, d_bad.ptr, d_info.ptr, d_temp.ptr, cp, d_post.ptr)


@pytest.mark.gpu
def test_device_postprocess_nonfinite_results_are_errors():
    """The device kernel raises the reference's two errors for non-finite
    results (nneval.cpp:1012-1016, 1167-1184) where the restatement does: a
    NaN logit of a legal move, a NaN value logit. The same handle then
    post-processes clean rows as before."""
    lm = nn.LoadedModel(G170_MODEL)
    dm = nn.DeviceModel(lm, use_fp16=False)
    n = 4
    h = nn.DeviceHandle(dm, n)
    score_c = lm.info.num_score_value_channels
    raw, legal, info, temp, flags = _random_rows(np.random.default_rng(11), n, score_c)
    params = pp.PostProcessParams()
    cp = nn.PostParams(params.output_scale_multiplier, params.score_mean_multiplier, params.score_stdev_multiplier,
                       params.lead_multiplier, params.variance_time_multiplier, params.shortterm_value_error_multiplier,
                       params.shortterm_score_error_multiplier)
    d_legal = nn.DeviceBuffer.from_array(legal.astype(np.uint8))
    d_info = nn.DeviceBuffer.from_array(info)
    d_temp = nn.DeviceBuffer.from_array(temp)
    d_post = nn.DeviceBuffer(n * (2 * HW + 10) * 4)

    def run(rows):
        d_raw = nn.DeviceBuffer.from_array(rows)
        h.postprocess_device(n, d_raw.ptr, d_legal.ptr, d_info.ptr, d_temp.ptr, cp, d_post.ptr)
        return d_post.to_array(np.float32, (n, 2 * HW + 10))

    bad = raw.copy()
    bad[2, np.flatnonzero(legal[2])[0]] = np.nan
    with pytest.raises(nn.StringError, match="nonfinite for policy sum"):
        run(bad)
    bad = raw.copy()
    bad[1, HW + 1] = np.nan
    with pytest.raises(nn.StringError, match="nonfinite for nneval value"):
        run(bad)
    _check_rows(run(raw), raw, legal, temp, flags, score_c, lm.info.model_version, params)


@pytest.mark.gpu
def test_get_output_post_processes_on_device(model_dir):
    """getOutput rows flagged for post-processing equal the restatement applied
    to the raw getOutput of the same rows; unflagged rows stay raw."""
    cfg = modelgen.configs()[1]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    n = 6
    h = nn.ComputeHandle(nn.ComputeContext(lm, 19, 19, use_fp16=True), max_batch=n)
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, n, board_sizes=(19, 13, 9))
    sym = np.arange(n) % 8
    raw = h.get_output(sp, gl, symmetry=sym)
    rng = np.random.default_rng(3)
    legal = rng.random((n, HW + 1)) < 0.7
    legal[:, HW] = True
    flags = [dict(white_to_move=bool(i % 2), no_result_disabled=bool(i == 2), passing_hacks=bool(i == 4),
                  board_x=(19, 13, 9)[i % 3], board_y=(19, 13, 9)[i % 3]) for i in range(n)]
    info = np.array([nn.post_info(enabled=(i != 5), **flags[i]) for i in range(n)], np.int32)
    temp = np.array([1.0, 0.8, 1.0, 1.2, 1.0, 1.0], np.float32)
    out = h.get_output_post(sp, gl, legal, info, temperature=temp, symmetry=sym)
    desc_params = pp.PostProcessParams(output_scale_multiplier=lm.info.output_scale_multiplier)
    for i in range(5):
        pol, vals, own = pp.postprocess_row(raw["policy"][i], raw["value"][i], raw["score"][i], raw["ownership"][i], legal[i],
                                            nn_x=19, nn_y=19, temperature=float(temp[i]),
                                            model_version=lm.info.model_version, params=desc_params, **flags[i])
        np.testing.assert_allclose(out["policy"][i], pol, rtol=1e-5, atol=1e-9)
        np.testing.assert_allclose(out["values"][i], vals.astype(np.float32), rtol=1e-6, atol=1e-9)
        np.testing.assert_allclose(out["ownership"][i], own, atol=1e-6)
    assert np.array_equal(out["policy"][5], raw["policy"][5])
