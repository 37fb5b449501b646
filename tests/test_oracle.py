"""Pins the CPU oracle (oracle/eigen_oracle.cpp) before it is trusted.

Checks, in order of strength: the reference's own known-answer tests
(testnn.cpp layer KATs, symmetry golden vectors), definitions (Winograd vs
direct convolution in double; activation closed forms), an independent
float64 torch re-derivation of whole networks, and invariants (batch
independence, a small board padded into a 19x19 tensor equals the same board
evaluated unpadded).
"""
import math
import os

import numpy as np
import pytest

from helpers import G170_MODEL, TRANSFORMER_MODELS, approx_equal_kat, load_kats, load_symmetry_cases, nchw_to_nhwc
from katago_amd import modelgen, nn
from oracle import oracle

KIND = {"conv": 0, "bn": 1, "residual": 2, "gpool": 3}


@pytest.mark.parametrize("kat", load_kats(), ids=lambda k: k["label"])
def test_oracle_layer_kats(kat):
    n, X, Y = kat["batch"], kat["nnXLen"], kat["nnYLen"]
    inp = nchw_to_nhwc(kat["input_nchw"], n, kat["inChannels"], Y, X)
    exp = nchw_to_nhwc(kat["expected_nchw"], n, kat["outChannels"], Y, X)
    out = oracle.test_evaluate(KIND[kat["kind"]], kat["desc_text"], n, X, Y, inp, kat["mask"], kat["outChannels"])
    assert approx_equal_kat(out, exp, fp16=False).all(), (out, exp)


def _conv_desc_text(w_oiyx, ky, kx, cin, cout):
    fo = np.asarray(w_oiyx, np.float32).reshape(cout, cin, ky, kx).transpose(2, 3, 1, 0).reshape(-1)
    return f"c {ky} {kx} {cin} {cout} 1 1\n" + " ".join(repr(float(v)) for v in fo)


@pytest.mark.parametrize("ksize,cin,cout,nx,ny,batch", [
    (3, 8, 12, 19, 19, 2), (3, 5, 3, 9, 9, 3), (3, 4, 4, 7, 5, 1), (5, 3, 6, 19, 19, 1), (5, 2, 2, 6, 7, 2),
    (3, 16, 16, 1, 1, 2), (1, 7, 9, 19, 19, 2), (7, 2, 3, 8, 8, 1),
])
def test_oracle_winograd_matches_direct_convolution(ksize, cin, cout, nx, ny, batch):
    rng = np.random.default_rng(ksize * 1000 + cin * 10 + nx)
    w = rng.standard_normal((cout, cin, ksize, ksize)).astype(np.float32)
    x = rng.standard_normal((batch, ny, nx, cin)).astype(np.float32)
    got = oracle.test_evaluate(0, _conv_desc_text(w, ksize, ksize, cin, cout), batch, nx, ny, x, None, cout)
    ref = oracle.direct_conv_f64(w, x, ksize, ksize, cin, cout, batch, nx, ny)
    scale = np.abs(ref).max() + 1.0
    assert np.abs(got - ref).max() < 2e-5 * scale * math.sqrt(cin * ksize * ksize)


def _bn_act_text(c, act, scale=None, bias=None):
    scale = np.ones(c) if scale is None else scale
    bias = np.zeros(c) if bias is None else bias
    arr = lambda a: " ".join(repr(float(v)) for v in a)
    return f"bn {c} 1e-20 1 1\n{arr(np.zeros(c))}\n{arr(np.full(c, 1 - 1e-20))}\n{arr(scale)}\n{arr(bias)}\nact {act}\n"


@pytest.mark.parametrize("act", ["ACTIVATION_IDENTITY", "ACTIVATION_RELU", "ACTIVATION_MISH", "ACTIVATION_SILU"])
def test_oracle_activation_closed_forms(act):
    c = 4
    x = np.linspace(-30, 30, 2 * 3 * 5 * c).astype(np.float32)
    mask = np.ones(2 * 3 * 5, np.float32)
    mask[3] = 0.0
    got = oracle.test_evaluate(5, _bn_act_text(c, act), 2, 5, 3, x, mask, c).reshape(-1, c)
    xd = x.astype(np.float64).reshape(-1, c)
    ref = {
        "ACTIVATION_IDENTITY": xd,
        "ACTIVATION_RELU": np.maximum(xd, 0),
        "ACTIVATION_MISH": xd * np.tanh(np.logaddexp(0.0, xd)),
        "ACTIVATION_SILU": xd / (1 + np.exp(-xd)),
    }[act]
    ref = ref * (mask[:, None] == 1.0)
    assert np.allclose(got, ref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("case", load_symmetry_cases(), ids=lambda c: f"{c['label']}-{c['kind']}-nhwc{c['nhwc']}-s{c['symmetry']}")
def test_oracle_symmetry_golden(case):
    out = oracle.copy_with_symmetry(case["src"], case["nSize"], case["hSize"], case["wSize"], case["cSize"], case["nhwc"],
                                    case["symmetry"], case["kind"] == "output")
    assert np.array_equal(out, np.asarray(case["expected"], np.float32))


def _tiny_nbt(activation="ACTIVATION_MISH"):
    return modelgen.Arch("tiny-nbt", 15, 32, 32, 16, ["bottlenest2", "bottlenest2gpool", "regular", "regulargpool"],
                         16, 16, 32, 24, activation, residual_gain=0.5)


def _torch_check(path, rows=3, board_sizes=(19,), nn_x=19, nn_y=19, seed=7):
    import torch_reference as tr
    om = oracle.OracleModel(path, nn_x, nn_y)
    lm = nn.LoadedModel(path)
    layers, weights = tr.flatten(lm)
    sp, gl = modelgen.synthetic_inputs(seed, rows, nn_x, nn_y, board_sizes)
    opt = np.linspace(0, 1, rows).astype(np.float32)
    ora = om.forward(sp, gl, policy_optimism=opt)
    ref = tr.forward(layers, weights, sp, gl, nn_x, nn_y, policy_optimism=opt, output_scale=lm.info.output_scale_multiplier)
    for key in ("policy", "value", "ownership"):
        a, b = ora[key], ref[key]
        assert np.abs(a - b).max() <= 1e-3 * max(1.0, np.abs(b).max()), (key, np.abs(a - b).max())
    nscore = lm.info.num_score_value_channels
    assert np.abs(ora["score"][:, :nscore] - ref["score"]).max() <= 1e-3 * max(1.0, np.abs(ref["score"]).max())


def test_oracle_whole_net_b6c96_matches_torch_f64(model_dir):
    cfg = modelgen.configs()[0]
    _torch_check(modelgen.ensure_model(model_dir, cfg))


def test_oracle_whole_net_nbt_mish_mixed_boards_matches_torch_f64(model_dir):
    path = modelgen.write_model(_tiny_nbt(), 11, f"{model_dir}/tiny-nbt.bin.gz")
    _torch_check(path, rows=4, board_sizes=(9, 13, 19, 7))


def test_oracle_whole_net_trained_g170_matches_torch_f64():
    _torch_check(G170_MODEL, rows=2)


def _tiny_transformer(learnable_rope=True, kv_heads=2, q_dim=16, v_dim=16, rmsnorm_tip=True):
    kinds = ["attention", "ffn", "regular", "attention", "ffn"]
    return modelgen.Arch("tiny-tf", 17, 64, 64, 32, kinds, 16, 16, 32, 24, "ACTIVATION_SILU", heads=4, kv_heads=kv_heads,
                         q_head_dim=q_dim, v_head_dim=v_dim, ffn_c=96, learnable_rope=learnable_rope, trunk_rmsnorm=rmsnorm_tip,
                         transformer_std=0.08, residual_gain=0.5)


@pytest.mark.parametrize("learnable,kv,tip", [(True, 2, True), (False, 4, True), (True, 1, False)],
                         ids=["gqa-learnable-rms", "mha-fixed-rms", "mqa-learnable-bn"])
def test_oracle_whole_net_tiny_transformer_matches_torch_f64(model_dir, learnable, kv, tip):
    """Attention (torch scaled_dot_product_attention), RMSNorm, SwiGLU and both
    RoPE forms, mixed with a residual conv block, on mixed board sizes."""
    arch = _tiny_transformer(learnable_rope=learnable, kv_heads=kv, rmsnorm_tip=tip)
    path = modelgen.write_model(arch, 21 + kv, f"{model_dir}/tiny-tf-{learnable}-{kv}-{tip}.bin.gz")
    _torch_check(path, rows=3, board_sizes=(19, 9, 13))


@pytest.mark.parametrize("path", TRANSFORMER_MODELS, ids=lambda p: os.path.basename(p).split("-")[0])
def test_oracle_reference_transformer_nets_match_torch_f64(path):
    _torch_check(path, rows=2, board_sizes=(19, 11))


def test_oracle_batch_independence(model_dir):
    path = modelgen.write_model(_tiny_nbt(), 12, f"{model_dir}/tiny-nbt-12.bin.gz")
    om = oracle.OracleModel(path)
    sp, gl = modelgen.synthetic_inputs(5, 5, board_sizes=(19, 9))
    full = om.forward(sp, gl)
    one = om.forward(sp[2:3], gl[2:3])
    for k in full:
        assert np.allclose(full[k][2:3], one[k], atol=1e-5)


def test_oracle_small_board_padding_equals_unpadded(model_dir):
    """A 9x9 board inside a 19x19 tensor must give the same on-board outputs as
    the same board evaluated with a 9x9 tensor: every op is masked."""
    path = modelgen.write_model(_tiny_nbt(), 13, f"{model_dir}/tiny-nbt-13.bin.gz")
    big = oracle.OracleModel(path, 19, 19)
    small = oracle.OracleModel(path, 9, 9)
    sp19, gl = modelgen.synthetic_inputs(9, 2, 19, 19, (9,))
    sp9 = sp19.reshape(2, 19, 19, 22)[:, :9, :9, :].reshape(2, -1)
    a = big.forward(sp19, gl)
    b = small.forward(sp9, gl)
    pol19 = a["policy"][:, :361].reshape(2, 19, 19)[:, :9, :9].reshape(2, 81)
    assert np.allclose(pol19, b["policy"][:, :81], atol=2e-4)
    assert np.allclose(a["policy"][:, 361], b["policy"][:, 81], atol=2e-4)
    assert np.allclose(a["value"], b["value"], atol=2e-4)
    assert np.allclose(a["score"], b["score"], atol=2e-4)
    own19 = a["ownership"].reshape(2, 19, 19)[:, :9, :9].reshape(2, 81)
    assert np.allclose(own19, b["ownership"], atol=2e-4)


def test_oracle_symmetry_bookkeeping(model_dir):
    """getOutput with row symmetry s equals symmetry 0 applied to inputs the
    host pre-transformed by s, with outputs mapped back by the inverse."""
    path = modelgen.ensure_model(model_dir, modelgen.configs()[0])
    om = oracle.OracleModel(path)
    sp, gl = modelgen.synthetic_inputs(3, 1)
    for s in range(8):
        direct = om.forward(sp, gl, symmetry=[s])
        pre = oracle.copy_with_symmetry(sp, 1, 19, 19, 22, 1, s, False)
        base = om.forward(pre, gl)
        pol = oracle.copy_with_symmetry(base["policy"][:, :361], 1, 19, 19, 1, 0, s, True)
        assert np.allclose(direct["policy"][:, :361], pol, atol=1e-6)
        assert np.allclose(direct["value"], base["value"], atol=1e-6)
