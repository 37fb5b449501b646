"""This repository's model parser against KataGo's own (desc.cpp), compiled
from the reference sources into oracle/_ref/ref_modeldesc (oracle/Makefile.ref).

Both load the same file with KataGo's load-time transforms
(transformToReduceActivations, desc.cpp:2631; applyScale8ToReduceActivations
as cudabackend.cpp:3081 applies it) and list every layer in the order the
backend hands the net to its device library. Layer kinds, shapes,
activation codes and every weight (as float bits) must be identical, as must
the model's version, channel counts and output multiplier. Covers model
versions 3, 4, 5, 8 (text and binary files of the same net), 9, 11, 15
(synthetic nets written by this repository) and 17 (transformer nets).

Runs where the reference tree exists (this container); skipped elsewhere.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

from helpers import GOLDEN, TRANSFORMER_MODELS
from katago_amd import modelgen, nn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_CPP = "/root/reference/cpp"
DUMP = os.path.join(ROOT, "oracle", "_ref", "ref_modeldesc")
REF_MODELS = os.path.join(REF_CPP, "tests", "models")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_MODELS), reason="needs the reference source tree")

OP_NAMES = {1: "conv", 2: "bn", 3: "act", 4: "matmul", 5: "matbias", 6: "rmsnorm", 7: "trmsnorm", 10: "ordinary",
            11: "gpool", 12: "nbt", 13: "attention", 14: "ffn", 20: "trunk", 21: "policyhead", 22: "valuehead"}
# Integers of each record that the dump lists (the rest of i[] is unused).
NUM_INTS = {"conv": 6, "bn": 1, "act": 1, "matmul": 2, "matbias": 1, "rmsnorm": 2, "trmsnorm": 1, "ordinary": 0,
            "gpool": 0, "nbt": 1, "attention": 6, "ffn": 3, "trunk": 3, "policyhead": 2, "valuehead": 0}


@pytest.fixture(scope="module")
def dumper():
    if not os.path.exists(DUMP):
        subprocess.run(["make", "-s", "-f", "oracle/Makefile.ref", f"REF={REF_CPP}"], cwd=ROOT, check=True)
    return DUMP


def reference_records(dumper, path):
    out = subprocess.run([dumper, path], capture_output=True, text=True, check=True).stdout
    recs = []
    for line in out.splitlines():
        head, tail = line.split(" | ")
        toks = head.split()
        words = tail.split()
        assert int(words[0]) == len(words) - 1
        recs.append((toks[0], [int(t) for t in toks[1:]], np.array([int(w, 16) for w in words[1:]], np.uint32)))
    return recs


def product_records(path):
    lm = nn.LoadedModel(path)
    layers, weights = nn.flatten_model(lm)
    bits = weights.view(np.uint32)
    info = lm.info
    osm = np.array([info.output_scale_multiplier], np.float32).view(np.uint32)
    recs = [("model", [info.model_version, info.num_input_channels, info.num_input_global_channels,
                       info.num_policy_channels, info.num_value_channels, info.num_score_value_channels,
                       info.num_ownership_channels, info.trunk_num_channels], osm)]
    for rec in layers:
        name = OP_NAMES[int(rec["op"])]
        ints = [int(v) for v in rec["i"][:NUM_INTS[name]]]
        segs = []
        for k in range(2):
            if rec["w"][k] >= 0:
                segs.append(bits[rec["w"][k]:rec["w"][k] + rec["wn"][k]])
        recs.append((name, ints, np.concatenate(segs) if segs else np.zeros(0, np.uint32)))
    return recs


def _compare(dumper, path):
    ref = reference_records(dumper, path)
    mine = product_records(path)
    assert len(ref) == len(mine), (len(ref), len(mine))
    for k, (a, b) in enumerate(zip(ref, mine)):
        assert a[0] == b[0], f"record {k}: reference {a[0]} vs {b[0]}"
        assert a[1] == b[1], f"record {k} ({a[0]}): reference ints {a[1]} vs {b[1]}"
        assert a[2].shape == b[2].shape, f"record {k} ({a[0]}): {a[2].shape} vs {b[2].shape} weights"
        diff = np.nonzero(a[2] != b[2])[0]
        if len(diff):
            i = diff[0]
            fa, fb = (struct.unpack("<f", struct.pack("<I", int(x)))[0] for x in (a[2][i], b[2][i]))
            pytest.fail(f"record {k} ({a[0]}): {len(diff)} weights differ, first at {i}: reference {fa!r} vs {fb!r}")
    return len(ref)


REFERENCE_FILES = [
    "run4-s67105280-d24430742-b6c96.txt.gz",         # version 3
    "grun50-b6c96-s156348160-d118286860.txt.gz",     # version 4
    "grun2-b6c96-s128700160-d49811312.txt.gz",
    "g103-b6c96-s103408384-d26419149.txt.gz",        # version 5
    "g170-b6c96-s175395328-d26788732.bin.gz",        # version 8
    "g170-b6c96-s175395328-d26788732.txt.gz",        # the same net as text
    "g170e-b10c128-s1141046784-d204142634.bin.gz",   # version 8, 10 blocks
]


@pytest.mark.parametrize("name", REFERENCE_FILES, ids=lambda n: n.split("-s")[0])
def test_parser_matches_reference_on_reference_models(dumper, name):
    assert _compare(dumper, os.path.join(REF_MODELS, name)) > 10


@pytest.mark.parametrize("path", [f"{GOLDEN}/tinymodel_relu.bin.gz", f"{GOLDEN}/tinymodel_mish.bin.gz"] + TRANSFORMER_MODELS,
                         ids=lambda p: p.split("/")[-1].split(".")[0])
def test_parser_matches_reference_on_fixture_models(dumper, path):
    assert _compare(dumper, path) > 10


@pytest.mark.parametrize("cfg_index", [0, 1, 2, 4], ids=["C0", "C1", "C2", "C4"])
def test_parser_matches_reference_on_generated_models(dumper, model_dir, cfg_index):
    """The synthetic benchmark nets (version 15 conv nets, version 17
    transformer) as this repository's writer produces them: the reference
    parser reads them to the same weights."""
    assert _compare(dumper, modelgen.ensure_model(model_dir, modelgen.configs()[cfg_index])) > 10


def test_reference_parser_reads_the_generated_metadata_encoder_net(dumper, tmp_path):
    """The writer's SGF metadata encoder (the net the host rejects at handle
    creation, test_host.py) is in the reference's grammar: KataGo's own
    desc.cpp loads the file (its encoder's input width is checked there
    against the 192 metadata channels)."""
    import dataclasses
    arch = dataclasses.replace(modelgen.b6c96(), version=15, meta_encoder_version=1, name="b6c96-meta")
    path = modelgen.write_model(arch, 3, str(tmp_path / "meta.bin.gz"))
    out = subprocess.run([dumper, path], capture_output=True, text=True, check=True).stdout
    assert out.splitlines()[0].startswith("model 15 22 19 ")
