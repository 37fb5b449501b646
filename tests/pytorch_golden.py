"""Shared access to the fixtures written from the reference's own PyTorch
model and exporter (tests/golden/make_pytorch_golden.py): four nets of model
versions 15 and 17 in KataGo's format, 16 positions featurized by KataGo's
fillRowV7 in 19x19 tensors, and the reference forward's raw head outputs."""
from __future__ import annotations

import os

import numpy as np

from helpers import GOLDEN

_DATA = None


def data():
    global _DATA
    if _DATA is None:
        with np.load(os.path.join(GOLDEN, "pytorch_golden.npz"), allow_pickle=False) as z:
            _DATA = {k: z[k] for k in z.files}
    return _DATA


def names():
    return [str(s) for s in data()["names"]]


def model_path(name):
    return os.path.join(GOLDEN, f"pytorch_golden_{name}.bin.gz")


def inputs():
    d = data()
    return d["spatial_nhwc"].astype(np.float32), d["global"].astype(np.float32)


def legal_mask():
    """On-board points of each position (plane 0) plus pass: the entries
    getOutput defines; off-board policy entries are not outputs."""
    sp, _ = inputs()
    n = sp.shape[0]
    on = sp.reshape(n, 361, 22)[:, :, 0] > 0
    return np.concatenate([on, np.ones((n, 1), bool)], axis=1), on


def expected(name, optimism, prefix=""):
    """The reference forward's outputs for the rows getOutput produces with
    the given per-row policyOptimism: policy channels 0 and 1 of the file
    mixed as p0 + (p1 - p0) * optimism (eigenbackend.cpp:2539-2549; with four
    channels the last two are the q-value outputs, which getOutput does not
    read), value logits, score channels, ownership."""
    d = data()
    key = f"{name}/{prefix}"
    pol = d[key + "policy"].astype(np.float64)
    opt = np.asarray(optimism, np.float64)[:, None]
    return {
        "policy": pol[:, 0, :] + (pol[:, 1, :] - pol[:, 0, :]) * opt,
        "value": d[key + "value"].astype(np.float64),
        "score": d[key + "score"].astype(np.float64),
        "ownership": d[key + "ownership"].astype(np.float64),
        "channels": pol.shape[1],
    }


def max_errors(out, exp, scale=1.0):
    legal, on = legal_mask()
    return {
        "policy": float(np.abs(out["policy"] * scale - exp["policy"])[legal].max()),
        "value": float(np.abs(out["value"] * scale - exp["value"]).max()),
        "score": float(np.abs(out["score"] * scale - exp["score"]).max()),
        "ownership": float(np.abs(out["ownership"] * scale - exp["ownership"])[on].max()),
    }


def argmax_disagreements(out, exp, tol, scale=1.0):
    """Rows whose top move over legal entries differs from the reference's,
    beyond ties: a different pick is allowed only where the reference's own
    top two lie within the policy tolerance of each other."""
    legal, _ = legal_mask()
    bad = []
    for i in range(legal.shape[0]):
        a = np.where(legal[i], out["policy"][i] * scale, -np.inf).argmax()
        b = np.where(legal[i], exp["policy"][i], -np.inf).argmax()
        if a != b and exp["policy"][i][b] - exp["policy"][i][a] > tol:
            bad.append((i, int(a), int(b)))
    return bad
