"""The algorithmic FLOP counts bench.py divides by measured time (the
roofline's `achieved`, `conv_frac`, `mfma_frac_end_to_end`), checked against
closed forms of the benchmark nets' architectures on the CPU: a dropped
conv, a padded channel count or a wrong attention term changes them."""
import importlib.util
import os

import pytest

from katago_amd import modelgen, nn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HW = 361


def _bench():
    spec = importlib.util.spec_from_file_location("bench_module", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _flops(model_dir, index):
    layers, _ = nn.flatten_model(nn.LoadedModel(modelgen.ensure_model(model_dir, modelgen.configs()[index])))
    return _bench().conv_flops(layers, HW)


def test_c2_nested_bottleneck_conv_flops(model_dir):
    """b18c384nbt: the 22->384 stem; 18 blocks of a 384->192 and a 192->384
    1x1 conv around two inner residual blocks of two 192->192 3x3 convs,
    where the five gpool blocks' second conv reads the 128 regular channels;
    the heads' 1x1 convs (p1, g1, v1 from 384 channels; p2 from p1's 48)."""
    f3, f1, _ = _flops(model_dir, 2)
    assert f3 == 2 * 9 * HW * (22 * 384 + 67 * 192 * 192 + 5 * 128 * 192)
    trunk_1x1 = 18 * 2 * (384 * 192 + 192 * 384) * HW
    heads_1x1 = 2 * HW * 384 * (48 + 48 + 96)
    assert trunk_1x1 + heads_1x1 <= f1 <= trunk_1x1 + heads_1x1 + 2 * HW * 48 * 4
    assert f3 / 1e9 == pytest.approx(16.902, abs=1e-3)


def test_c4_transformer_flops(model_dir):
    """t12d384h6: a 3x3 stem and, per block, the [Q|K|V] (384 -> 3 x 384),
    output (384 -> 384), [linear1|gate] (384 -> 2 x 1024) and linear2
    (1024 -> 384) projections per position, and attention's two products
    (2 * HW^2 * (dq + dv) per head)."""
    f3, f1, other = _flops(model_dir, 4)
    assert f3 == 2 * 9 * HW * 22 * 384
    projections = 12 * 2 * HW * (384 * 3 * 384 + 384 * 384 + 384 * 2 * 1024 + 1024 * 384)
    attention = 12 * 6 * 2 * HW * HW * (64 + 64)
    assert projections + attention <= f1 + other <= (projections + attention) * 1.01


def test_roofline_traffic_comes_from_the_committed_counter_profile():
    """bench.py's roofline.traffic is the FETCH_SIZE + WRITE_SIZE mean per 3x3
    launch from profiles/: within 1.0-1.3x of the ~106 MB of algorithmic
    bytes a C2 trunk conv moves on average (input, residual where there is
    one, one or two outputs)."""
    traffic = _bench().measured_traffic()
    algorithmic = (36 * (4 * 35.5e6) + 36 * (2 * 35.5e6)) / 72
    assert traffic is not None and 1.0 * algorithmic <= traffic <= 1.3 * algorithmic
