"""Shared helpers for the test suite."""
from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
G170_MODEL = os.path.join(GOLDEN, "g170-b6c96-s175395328-d26788732.bin.gz")
# The reference's in-repo transformer test nets (cpp/tests/models, listed in
# rungpuerrortest.sh:31-33): fixed RoPE + per-position RMSNorm tip; GQA with
# dq=32, dv=16, learnable RoPE, BN tip; transformer blocks nested in
# bottleneck blocks, learnable RoPE, spatial RMSNorm tip with SiLU.
TRANSFORMER_MODELS = [os.path.join(GOLDEN, f + ".bin.gz") for f in (
    "b7c96h3tfrs-test5-cnorm",
    "b7c96h6kv3qk32v16tflrs-fson-bnh",
    "b4c256h4nbttflrs-fson-silu-rsnh",
)]


# Rows whose device argmax differs from the oracle's within the tie allowance
# of the whole-net parity tests, and the number of rows compared; the session
# summary (conftest.py) prints both.
ARGMAX_TIES = []
ARGMAX_ROWS = [0]


def load_kats():
    with open(os.path.join(GOLDEN, "layer_kats.json")) as f:
        return json.load(f)["kats"]


def load_symmetry_cases():
    with open(os.path.join(GOLDEN, "symmetry_golden.json")) as f:
        return json.load(f)["cases"]


def nchw_to_nhwc(a, n, c, h, w):
    return np.asarray(a, np.float32).reshape(n, c, h, w).transpose(0, 2, 3, 1).reshape(-1)


def approx_equal_kat(x, y, fp16: bool):
    """testnn.cpp:8-15: 1e-4*max(|x|,|y|,1) in fp32, 0.03*max(|x|,|y|,3) in fp16."""
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    if fp16:
        tol = 0.03 * np.maximum(np.maximum(np.abs(x), np.abs(y)), 3.0)
    else:
        tol = 1e-4 * np.maximum(np.maximum(np.abs(x), np.abs(y)), 1.0)
    return np.abs(x - y) < tol


def parse_layer_dump(text):
    """Lines of a per-block trunk dump ("DEBUG <name> [NSC NxSxC] valid= min=
    max= mean= rms= first8= ..."): [(name without its backend prefix, valid,
    min, max, mean, rms, first values)]."""
    import re
    out = []
    pat = re.compile(r"^DEBUG (\S+) (.*?) \[NSC (\d+)x(\d+)x(\d+)\] valid=(\d+) min=(\S+) max=(\S+) mean=(\S+) rms=(\S+) first8=(.*)$")
    for line in text.splitlines():
        m = pat.match(line)
        assert m, line
        out.append((m.group(2), int(m.group(6)), float(m.group(7)), float(m.group(8)), float(m.group(9)), float(m.group(10)),
                    [float(v) for v in m.group(11).split()]))
    return out
