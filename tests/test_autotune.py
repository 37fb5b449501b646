"""On-device autotuner (kgh_handle_autotune) and its persisted tables, per
(gpu, board size, batch, dtype, architecture), in the manner of the OpenCL
backend's tuner (opencltuner.cpp:779, 4948-4980).

Every kernel variant sums in the same order, so a tuned handle's outputs must
equal, bitwise, those of a handle using the built-in choices.
"""
import glob
import os

import numpy as np
import pytest

from katago_amd import modelgen, nn

def _variant_count():
    """CONV_VARIANT_COUNT: the entries of ConvVariant in kgh_common.h."""
    import re
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "katago_amd", "csrc", "kgh_common.h")
    body = re.search(r"enum ConvVariant \{(.*?)CONV_VARIANT_COUNT", open(path).read(), re.S).group(1)
    return len(re.findall(r"^\s*(CONV_\w+)", body, re.M))


# Kernel variant ids 0..VARIANTS-1 (ConvVariant in kgh_common.h).
VARIANTS = _variant_count()

pytestmark = pytest.mark.gpu


def _forward(handle, sp, gl):
    return handle.get_output(sp, gl, symmetry=np.arange(len(gl)) % 8)


def test_tune_save_load_and_identical_results(model_dir, tmp_path):
    cfg = modelgen.configs()[1]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    n = 48
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, n, board_sizes=(19, 13))
    home = str(tmp_path)

    tuned = nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=True, auto_tune=True, home_data_dir=home), max_batch=n)
    src, table = tuned.tuning()
    assert src == 2
    lines = [l for l in table.splitlines() if l.strip()]
    assert len(lines) >= 3  # the 3x3 trunk conv, the head 1x1s, ...
    for l in lines:
        f = l.split()
        assert int(f[4]) == n * 361 and 0 <= int(f[8]) < VARIANTS  # M, variant id (0: built-in choice kept)
    files = glob.glob(os.path.join(home, "hiptuning", f"tune1_*_x19_y19_b{n}_fp16_arch*.txt"))
    assert len(files) == 1
    assert open(files[0]).read().startswith("VERSION=2")

    loaded = nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=True, auto_tune=True, home_data_dir=home), max_batch=n)
    src2, table2 = loaded.tuning()
    assert src2 == 1
    assert [l.split()[:9] for l in table2.splitlines() if l.strip()] == [l.split()[:9] for l in lines]

    builtin = nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=True, auto_tune=False), max_batch=n)
    assert builtin.tuning() == (0, "")

    a, b, c = _forward(tuned, sp, gl), _forward(loaded, sp, gl), _forward(builtin, sp, gl)
    for k in a:
        assert np.array_equal(a[k], c[k]), k
        assert np.array_equal(b[k], c[k]), k


def test_explicit_tuner_file_and_small_batches(model_dir, tmp_path):
    cfg = modelgen.configs()[0]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    path = str(tmp_path / "my_tuning.txt")
    h = nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=False, auto_tune=True, tuner_file=path), max_batch=16)
    assert h.tuning()[0] == 2 and os.path.exists(path)
    # Batches of 8 or fewer keep the built-in choices.
    small = nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=False, auto_tune=True, tuner_file=path), max_batch=8)
    assert small.tuning()[0] == 0
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, 8)
    x, y = _forward(h, sp, gl), _forward(small, sp, gl)
    for k in x:
        assert np.array_equal(x[k], y[k]), k


@pytest.mark.parametrize("fp16", [True, False], ids=["fp16", "fp32"])
def test_every_kernel_variant_gives_identical_bits(model_dir, fp16):
    """Pin every shape to each variant in turn (a variant that does not apply
    to a shape falls back to the built-in choice): outputs stay bitwise equal
    to the built-in choices, since all variants sum in the same order."""
    cfg = modelgen.configs()[1]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    n = 40
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, n, board_sizes=(19, 9))
    tuned = nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=fp16, auto_tune=True, tuner_file=str(model_dir) + f"/t{fp16}.txt"),
                             max_batch=n)
    shapes = [l.split()[:8] for l in tuned.tuning()[1].splitlines() if l.strip()]
    assert shapes
    ref = _forward(nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=fp16, auto_tune=False), max_batch=n), sp, gl)
    for v in range(1, VARIANTS):
        tuned.set_tuning("".join(" ".join(k) + f" {v}\n" for k in shapes))
        out = _forward(tuned, sp, gl)
        for k in out:
            assert np.array_equal(out[k], ref[k]), (v, k)


@pytest.mark.parametrize("variant", [16, 17, 18, 20, 21, 13, 15, 19, 23, 24],
                         ids=["dma1x1h_192", "dma1x1h_128", "dma1x1h_64", "allk1x1_64", "allk1x1_32", "board192", "board64",
                              "boardhalf64", "boardhalf64t32", "boardhalf192"])
def test_variants_give_identical_bits_on_nbt(model_dir, variant):
    """On C2's nested-bottleneck shapes (192-channel 3x3 convs, which the
    b10c128 test above cannot pin to the 192-column board kernels): the
    192-row and whole-K 1x1 kernels, including the post 1x1 conv whose
    residual is loaded into the accumulators (through the stage that shares
    the A buffers in the 192-row kernel), and the one-board 3x3 kernels on
    whole and half boards: bitwise the built-in outputs."""
    cfg = modelgen.configs()[2]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    n = 12  # batches of 8 boards or fewer are not tuned
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, n, board_sizes=(19, 13))
    tuned = nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=True, auto_tune=True, tuner_file=str(model_dir) + "/t_nbt.txt"),
                             max_batch=n)
    shapes = [l.split()[:8] for l in tuned.tuning()[1].splitlines() if l.strip()]
    assert any(k[0] == "1" and k[6] == "1" for k in shapes)  # a 1x1 shape with a residual
    ref = _forward(nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=True, auto_tune=False), max_batch=n), sp, gl)
    tuned.set_tuning("".join(" ".join(k) + f" {variant}\n" for k in shapes))
    out = _forward(tuned, sp, gl)
    for k in out:
        assert np.array_equal(out[k], ref[k]), k


def test_every_kernel_variant_gives_identical_bits_on_transformer(model_dir):
    """C4's transformer net with every shape pinned to each variant in turn:
    the 1x1 DMA kernels (384- and 192-row tiles) against the built-in tile
    kernel at 12 boards, on the [Q|K|V] and SwiGLU GEMMs that scale their
    rows by the folded RMSNorm, and on the output projection and linear2 with
    their masked residual that record the next norm's sums of squares."""
    cfg = modelgen.configs()[4]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    n = 12
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, n, board_sizes=(19, 13))
    tuned = nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=True, auto_tune=True, tuner_file=str(model_dir) + "/t_c4.txt"),
                             max_batch=n)
    shapes = [l.split()[:8] for l in tuned.tuning()[1].splitlines() if l.strip()]
    assert any(k[0] == "1" and k[5] == "1" for k in shapes)  # the SwiGLU GEMM
    assert any(k[0] == "1" and k[7] == "1" for k in shapes)  # a masked residual
    ref = _forward(nn.ComputeHandle(nn.ComputeContext(lm, use_fp16=True, auto_tune=False), max_batch=n), sp, gl)
    for v in range(1, VARIANTS):
        tuned.set_tuning("".join(" ".join(k) + f" {v}\n" for k in shapes))
        out = _forward(tuned, sp, gl)
        for k in out:
            assert np.array_equal(out[k], ref[k]), (v, k)
