"""CPU tests of the host side: model-file parsing and validation, the
load-time transforms, the C ABI exports, and the synthetic model/input
generator. No device calls."""
import gzip
import os
import re

import numpy as np
import pytest

from helpers import G170_MODEL
from katago_amd import modelgen, nn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kg[hn]_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("katago_hip.h", "hip"), ("katago_nn.h", "host")])
def test_c_abi_library_exports_every_declared_symbol(header, lib):
    so = nn.hip_library() if lib == "hip" else nn.host_library()
    names = _declared_functions(header)
    assert len(names) >= 8
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing


def test_splitmix64_published_vector():
    # Test vector published with SplitMix64 (seed 1234567).
    got = modelgen.SplitMix64(1234567).next_u64(5).tolist()
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                   16408922859458223821]


def test_synthetic_inputs_properties():
    sp, gl = modelgen.synthetic_inputs(2002, 6, board_sizes=(9, 13, 19))
    sp = sp.reshape(6, 19, 19, 22)
    for i, bs in enumerate((9, 13, 19, 9, 13, 19)):
        on = np.zeros((19, 19), bool)
        on[:bs, :bs] = True
        assert np.array_equal(sp[i, :, :, 0] == 1, on)
        assert not (sp[i][~on]).any()
        assert not ((sp[i, :, :, 1] == 1) & (sp[i, :, :, 2] == 1)).any()
    assert set(np.unique(sp)) <= {0.0, 1.0}
    assert (np.abs(gl) <= 1).all()
    sp2, gl2 = modelgen.synthetic_inputs(2002, 6, board_sizes=(9, 13, 19))
    assert np.array_equal(sp.reshape(6, -1), sp2) and np.array_equal(gl, gl2)


def test_model_info_of_generated_configs(model_dir):
    for cfg in modelgen.configs()[:3]:
        m = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
        assert m.info.model_version == 15
        assert m.info.num_input_channels == 22 and m.info.num_input_global_channels == 19
        assert m.info.trunk_num_channels == cfg.arch.trunk_c
        assert m.info.num_policy_channels == 2 and m.info.num_score_value_channels == 6
        # scale8 applied at load for these (BatchNorm-tip, no SiLU) models
        assert m.info.output_scale_multiplier == 8.0


def test_text_and_binary_files_parse_identically(model_dir):
    arch = modelgen.b6c96()
    arch.blocks = arch.blocks[:3]
    pb = modelgen.write_model(arch, 77, f"{model_dir}/a.bin", binary=True)
    pt = modelgen.write_model(arch, 77, f"{model_dir}/a.txt.gz", binary=False)
    import torch_reference as tr
    lb, wb = tr.flatten(nn.LoadedModel(pb))
    lt, wt = tr.flatten(nn.LoadedModel(pt))
    assert np.array_equal(lb, lt)
    assert np.allclose(wb, wt, rtol=1e-6, atol=1e-7)


@pytest.mark.skipif(not os.path.exists("/root/reference/cpp/tests/models"), reason="needs the reference tree")
def test_reference_bin_and_txt_model_files_parse_identically():
    base = "/root/reference/cpp/tests/models/g170-b6c96-s175395328-d26788732"
    import torch_reference as tr
    lb, wb = tr.flatten(nn.LoadedModel(base + ".bin.gz"))
    lt, wt = tr.flatten(nn.LoadedModel(base + ".txt.gz"))
    assert np.array_equal(lb["op"], lt["op"]) and np.array_equal(lb["i"], lt["i"])
    assert np.allclose(wb, wt, rtol=2e-5, atol=1e-6)


def test_trained_model_fixture_loads():
    m = nn.LoadedModel(G170_MODEL)
    assert m.info.model_version == 8 and m.info.trunk_num_channels == 96
    assert m.info.num_score_value_channels == 4 and m.info.num_policy_channels == 1


def _write_raw(path, data):
    with open(path, "wb") as f:
        f.write(data)
    return path


def _small_model_bytes(binary=True):
    arch = modelgen.b6c96()
    arch.blocks = ["regular"]
    return modelgen._Builder(arch, 5, binary).model()


def test_parser_rejects_nan_weight(model_dir):
    data = bytearray(_small_model_bytes())
    i = data.index(b"@BIN@") + 5
    data[i:i + 4] = np.float32(np.nan).tobytes()
    with pytest.raises(nn.StringError, match="Nan or infinite"):
        nn.LoadedModel(_write_raw(f"{model_dir}/nan.bin", bytes(data)))


def test_parser_rejects_truncated_file(model_dir):
    data = _small_model_bytes()
    with pytest.raises(nn.StringError):
        nn.LoadedModel(_write_raw(f"{model_dir}/trunc.bin", data[: len(data) // 2]))
    with pytest.raises(nn.StringError):
        nn.LoadedModel(_write_raw(f"{model_dir}/trunc.bin.gz", gzip.compress(data)[:1000]))


def test_parser_rejects_bad_name_version_and_extension(model_dir):
    data = _small_model_bytes()
    bad_name = data.replace(b"b6c96-synthetic", b"bad.name!", 1)
    with pytest.raises(nn.StringError, match="alphanumeric"):
        nn.LoadedModel(_write_raw(f"{model_dir}/badname.bin", bad_name))
    bad_version = data.replace(b"\n15\n", b"\n99\n", 1)
    with pytest.raises(nn.StringError, match="newer KataGo"):
        nn.LoadedModel(_write_raw(f"{model_dir}/badver.bin", bad_version))
    with pytest.raises(nn.StringError, match="should end with"):
        nn.LoadedModel(_write_raw(f"{model_dir}/model.weights", data))
    with pytest.raises(nn.StringError, match="unknown activation"):
        nn.LoadedModel(_write_raw(f"{model_dir}/badact.bin", data.replace(b"ACTIVATION_RELU", b"ACTIVATION_FOO", 1)))


def test_sha256_verification(model_dir):
    import hashlib
    data = gzip.compress(_small_model_bytes())
    path = _write_raw(f"{model_dir}/sha.bin.gz", data)
    good = hashlib.sha256(data).hexdigest()
    nn.LoadedModel(path, good)
    nn.LoadedModel(path, good.upper())
    with pytest.raises(nn.StringError, match="sha256"):
        nn.LoadedModel(path, "0" * 64)


def test_flattened_program_structure(model_dir):
    import torch_reference as tr
    cfg = modelgen.configs()[2]
    layers, weights = tr.flatten(nn.LoadedModel(modelgen.ensure_model(model_dir, cfg)))
    ops = layers["op"]
    assert ops[0] == tr.OP_TRUNK and layers[0]["i"][0] == 18 and layers[0]["i"][1] == 384
    assert (ops == tr.OP_BLOCK_NBT if hasattr(tr, "OP_BLOCK_NBT") else ops == tr.OP_NBT).sum() == 18
    assert (ops == tr.OP_GPOOL).sum() == 5
    convs = layers[ops == tr.OP_CONV]
    three = convs[(convs["i"][:, 0] == 3)]
    # stem + 36 ordinary-pair convs + 5 gpool blocks with regular+gpool+final
    assert len(three) == 1 + 2 * 31 + 3 * 5
    assert np.isfinite(weights).all()
    assert (layers["w"][:, 0] + layers["wn"][:, 0] <= len(weights)).all()


def test_hot_kernels_keep_everything_in_registers():
    """The build records the compiler's per-kernel resource report
    (katago_amd/lib/kernel_resources.json). A matrix-core kernel whose
    accumulators fall out of registers into scratch runs several times
    slower with identical results, so this guards it on the CPU."""
    import json
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "katago_amd", "lib", "kernel_resources.json")
    with open(path) as f:
        usage = json.load(f)
    hot = ("convBoardWindowKernel", "convTapWindowKernel", "conv1x1DmaKernel", "conv1x1AllKKernel", "convMfmaKernel", "flashAttentionKernel",
           "poolVecKernel", "headVectorKernel", "bnActVecKernel", "rmsNormRowKernel", "headSpatialKernel", "gpoolBiasActKernel",
           "splitKEpilogueKernel")
    seen = set()
    for name, u in usage.items():
        for h in hot:
            if h in name:
                seen.add(h)
                assert u["scratch"] == 0 and u["vgpr_spill"] == 0, (name, u)
    assert seen == set(hot), set(hot) - seen


def test_context_config_text_rejects_a_line_without_equals(model_dir):
    """kgn_create_context_cfg reads KataGo config lines ("key = value", '#'
    comments, blank lines); a line with no '=' is an error, reported before
    any device work."""
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, modelgen.configs()[0]))
    lib = nn.host_library()
    err = nn._errbuf()
    ptr = lib.kgn_create_context_cfg(lm._ptr, 19, 19, 1, b"", b"# tuning\n\nhipAutoTune = false\nhipLowLatency\n", err, len(err))
    assert not ptr
    assert "without '='" in err.value.decode() and "hipLowLatency" in err.value.decode()


def test_metadata_encoder_models_parse_and_are_rejected_at_handle_creation(tmp_path):
    """A version-15 net with an SGF metadata encoder (metaEncoderVersion 1,
    the 192 metadata channels; SGFMetadataEncoderDesc, desc.cpp) parses, and
    createComputeHandle rejects it with the documented StringError, on the
    host before any device work (the reference's CUDA backend evaluates such
    nets; none is among the benchmark configs)."""
    import dataclasses
    arch = dataclasses.replace(modelgen.b6c96(), version=15, meta_encoder_version=1, name="b6c96-meta")
    lm = nn.LoadedModel(modelgen.write_model(arch, 3, str(tmp_path / "meta.bin.gz")))
    assert lm.info.num_input_meta_channels == 192 and lm.info.model_version == 15
    ctx = nn.ComputeContext(lm, 19, 19, use_fp16=True)
    with pytest.raises(nn.StringError, match="SGF metadata encoder"):
        nn.ComputeHandle(ctx, max_batch=2)
