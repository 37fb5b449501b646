"""Regenerates the featurizer fixture from KataGo's own fillRowV7.

Run in a container where /root/reference exists (the tests never read it):
    python tests/golden/make_featurize_golden.py

oracle/_ref/ref_featurize (oracle/Makefile.ref) plays seeded random games
with KataGo's own Board and BoardHistory under every named ruleset, on square
and rectangular boards, and for each sampled position prints the
featurizer's input (a kgn_position, include/katago_featurize.h, filled from
KataGo's objects by katago_amd/host/neuralnet/featurizeadapter.cpp) with the
rows KataGo's NNInputs::fillRowV7 builds for it (nninputs.cpp:2273-2720).

Output: featurize_golden.json.gz, positions chosen so that every spatial plane
and global feature fillRowV7 can set is set in some of them (the ko-ban and
encore planes, ladders of the current and previous boards, area, history).
"""
from __future__ import annotations

import gzip
import json
import os
import subprocess

REF = "/root/reference/cpp"
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
DRIVER = os.path.join(ROOT, "oracle", "_ref", "ref_featurize")

RULES = ["tromp-taylor", "chinese", "chinese-ogs", "chinese-kgs", "japanese", "korean", "stone-scoring", "aga", "bga",
         "new-zealand", "aga-button"]
SIZES = [(19, 19, 19, 19), (9, 9, 9, 9), (13, 13, 13, 13), (9, 9, 19, 19), (5, 5, 6, 6), (19, 11, 19, 19), (7, 15, 19, 19),
         (3, 3, 5, 5), (17, 19, 19, 19)]


def games():
    seed = 5000
    lines = []
    for r in RULES:
        for (x, y, nx, ny) in SIZES:
            for k in range(2):
                seed += 1
                lines.append(f"compare {r}-{x}x{y}-{k} {seed} {x} {y} {nx} {ny} {int(x * y * 2.2) + 10} {r} 7")
    return "\n".join(lines) + "\n"


def planes(fx):
    """Spatial planes set anywhere in the fixture, and globals that are nonzero."""
    c = 22
    bits = bin(int(fx["spatial_nhwc_bits"], 16))[2:].zfill(len(fx["spatial_nhwc_bits"]) * 4)
    ps = set()
    for i, b in enumerate(bits):
        if b == "1" and i < fx["nnx"] * fx["nny"] * c:
            ps.add(i % c)
    gs = {i for i, v in enumerate(fx["global"]) if v != 0}
    return ps, gs


def main():
    subprocess.run(["make", "-s", "-f", "oracle/Makefile.ref", f"REF={REF}"], cwd=ROOT, check=True)
    out = subprocess.run([DRIVER], input=games(), capture_output=True, text=True, check=True).stdout
    fixtures, summaries = [], []
    for line in out.splitlines():
        d = json.loads(line)
        (summaries if "summary" in d else fixtures).append(d)
    mismatched = sum(s["mismatched"] for s in summaries)
    print(f"{sum(s['positions'] for s in summaries)} positions compared, {mismatched} mismatched")
    # Greedy cover: first a position for each (ruleset, plane or global)
    # pair not yet covered, then every tenth of the rest up to ~300.
    covered, chosen, rest = set(), [], []
    for fx in fixtures:
        ps, gs = planes(fx)
        ruleset = fx["fixture"].split("-")[0]
        keys = {(ruleset, "p", p) for p in ps} | {(ruleset, "g", g) for g in gs}
        if keys - covered:
            covered |= keys
            chosen.append(fx)
        else:
            rest.append(fx)
    chosen += rest[::10][: max(0, 300 - len(chosen))]
    seen_p, seen_g = set(), set()
    for fx in chosen:
        ps, gs = planes(fx)
        seen_p |= ps
        seen_g |= gs
    print(f"{len(chosen)} fixtures; spatial planes set: {sorted(seen_p)}; nonzero globals: {sorted(seen_g)}")
    with gzip.open(os.path.join(HERE, "featurize_golden.json.gz"), "wt") as f:
        json.dump({"source": "make_featurize_golden.py", "positions": chosen}, f, separators=(",", ":"))


if __name__ == "__main__":
    main()
