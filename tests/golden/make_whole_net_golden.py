"""Regenerates the whole-network golden fixtures from the reference tree.

Run in a container where /root/reference exists (the tests never read it):
    python tests/golden/make_whole_net_golden.py

It builds oracle/_ref/ref_featurize (oracle/Makefile.ref: KataGo's own board,
rules, history and nninputs sources, compiled where they lie, with a driver of
this repository) and writes:

  whole_net_golden.json  for each position the reference's own tests run a
      whole network on: the input rows KataGo's NNEvaluator builds for it
      (NNInputs::fillRowV*, NHWC), the legal moves the evaluator's
      post-processing reads, the symmetry the test used, and the outputs the
      reference recorded for it, which are:
        * cpp/tests/results/runNNOnTinyBoardTest.txt: g170-b6c96 (model
          version 8) on the 5x5 position of testsearchmisc.cpp:18-50 in a 6x6
          tensor, symmetry 3 (runsearchtests.sh:40), printed by
          NNOutput::debugPrint (nninputs.cpp:488-525);
        * cpp/tests/results/runNNSymmetriesTest.txt: g103-b6c96 (model
          version 5) on the 9x13 position of testsearchmisc.cpp:55-101 in a
          13x13 tensor, all eight symmetries (runsearchtests.sh:44);
        * cpp/tests/results/runNNSymmetriesTestFP16.txt: the same test in
          fp16 (runsearchtestsfp16.sh:21), kept only as the spread between
          the reference's own fp16 and fp32 records (reference_fp16_spread);
        * cpp/tests/tinymodel.cpp:135-490: the tiny ReLU and Mish models of
          tinymodeldata.cpp on a 19x19 position (symmetries 6 and 7) and a
          13x6 position (symmetry 1) in 19x19 tensors, with the expected
          values and tolerances written in that test.
  tinymodel_relu.bin.gz, tinymodel_mish.bin.gz  those two models, decoded
      from the base64 text of cpp/tests/tinymodeldata.cpp.
  g103-b6c96-s103408384-d26419149.txt.gz  the model of the symmetries test
      (cpp/tests/models/).
"""
from __future__ import annotations

import base64
import json
import os
import re
import shutil
import subprocess

REF = "/root/reference/cpp"
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
FEATURIZE = os.path.join(ROOT, "oracle", "_ref", "ref_featurize")
G170 = "g170-b6c96-s175395328-d26788732.bin.gz"
G103 = "g103-b6c96-s103408384-d26419149.txt.gz"


def build_featurizer():
    subprocess.run(["make", "-s", "-f", "oracle/Makefile.ref", f"REF={REF}"], cwd=ROOT, check=True)


def featurize(spec: str):
    out = subprocess.run([FEATURIZE], input=spec, capture_output=True, text=True, check=True).stdout
    return [json.loads(l) for l in out.splitlines() if l.strip()]


def case_spec(name, xs, ys, nnx, nny, pla, version, board_text):
    rows = [l for l in board_text.strip("\n").split("\n")]
    assert len(rows) == ys, (name, len(rows))
    return f"case {name} {xs} {ys} {nnx} {nny} {pla} {version} tromp-taylor\n" + "\n".join(rows) + "\n"


# ---------------------------------------------------------------------------
# Outputs printed by NNOutput::debugPrint (nninputs.cpp:488-525).

_SCALARS = [("Win", "whiteWinProb", 0.01, "c"), ("Loss", "whiteLossProb", 0.01, "c"),
            ("NoResult", "whiteNoResultProb", 0.01, "c"), ("ScoreMean", "whiteScoreMean", 1.0, ""),
            ("ScoreMeanSq", "whiteScoreMeanSq", 1.0, ""), ("Lead", "whiteLead", 1.0, ""),
            ("VarTimeLeft", "varTimeLeft", 1.0, ""), ("STWinlossError", "shorttermWinlossError", 0.01, "c"),
            ("STScoreError", "shorttermScoreError", 1.0, "")]


def parse_debug_prints(path, xs, ys):
    """Every debugPrint block of a results file: the nine scalars (in the
    NNOutput units, with the printed step), the policy grid (permille, None
    for an illegal point), pass (permille) and the ownership grid (permille,
    white's perspective)."""
    lines = open(path).read().split("\n")
    blocks = []
    i = 0
    while i < len(lines):
        if not lines[i].startswith("Win "):
            i += 1
            continue
        b = {"scalars": {}, "steps": {}}
        for k, (label, field, mult, suffix) in enumerate(_SCALARS):
            m = re.match(rf"{label} (-?[0-9.]+){suffix}$", lines[i + k])
            assert m, (path, lines[i + k])
            text = m.group(1)
            decimals = len(text.split(".")[1]) if "." in text else 0
            b["scalars"][field] = float(text) * mult
            b["steps"][field] = 10.0 ** -decimals * mult
        i += len(_SCALARS)
        assert lines[i].startswith("OptimismUsed"), lines[i]
        assert lines[i + 1] == "Policy", lines[i + 1]
        b["pass_permille"] = int(lines[i + 2].split()[1])
        i += 3
        pol = []
        for y in range(ys):
            toks = lines[i + y].split()
            assert len(toks) == xs, lines[i + y]
            pol.append([None if t == "-" else int(t) for t in toks])
        i += ys
        own = []
        for y in range(ys):
            toks = lines[i + y].split()
            assert len(toks) == xs, lines[i + y]
            own.append([int(t) for t in toks])
        i += ys
        b["policy_permille"] = pol
        b["ownership_permille"] = own
        blocks.append(b)
    return blocks


# ---------------------------------------------------------------------------
# tinymodel.cpp

def _raw_strings(text):
    return re.findall(r'R"%%\((.*?)\)%%"', text, re.S)


def decode_tiny_models():
    data = open(os.path.join(REF, "tests", "tinymodeldata.cpp")).read()
    parts = {}
    for m in re.finditer(r'const char\* TinyModelTest::(\w+) = R"%%\((.*?)\)%%"', data, re.S):
        parts[m.group(1)] = m.group(2)
    relu = "".join(parts[f"tinyModelBase64Part{k}"] for k in range(7))
    mish = parts["tinyMishModelBase64"]
    out = {}
    for name, text in (("tinymodel_relu.bin.gz", relu), ("tinymodel_mish.bin.gz", mish)):
        # decodeBase64 (tinymodel.cpp:14-45) skips whitespace and stops at the
        # first character outside the alphabet.
        clean = re.sub(r"[\s]", "", text)
        m = re.match(r"[A-Za-z0-9+/]*", clean)
        body = m.group(0)
        body = body[: len(body) - len(body) % 4] if len(body) % 4 == 1 else body
        raw = base64.b64decode(body + "=" * (-len(body) % 4))
        with open(os.path.join(HERE, name), "wb") as f:
            f.write(raw)
        out[name] = len(raw)
    return out


def parse_tinymodel_tests():
    """The three test blocks of tinymodel.cpp: model, board, symmetry, the
    scalar expectations with their scales, the expected policy (x1e4, -1 where
    not checked) and ownership (x1e4) with the tolerance formulas."""
    text = open(os.path.join(REF, "tests", "tinymodel.cpp")).read()
    chunks = text.split("string base64Data;")[1:]
    tests = []
    for ch in chunks:
        model = "tinymodel_relu.bin.gz" if "tinyModelBase64Part0" in ch else "tinymodel_mish.bin.gz"
        sym = int(re.search(r"setDefaultSymmetry\((\d+)\)", ch).group(1))
        bm = re.search(r'Board::parseBoard\((\d+),(\d+),R"%%\((.*?)\)%%"\)', ch, re.S)
        xs, ys, board = int(bm.group(1)), int(bm.group(2)), bm.group(3)
        pla = "b" if "nextPla = P_BLACK" in ch else "w"
        scalars = {f: (float(v), float(s)) for f, v, s in
                   re.findall(r"EQ\(nnOutput\.(\w+),\s*(-?[0-9.]+),\s*([0-9.]+)\)", ch)}
        arrays = {}
        for name, body in re.findall(r"double (expectedPolicy|expectedOwnership)\[\d+\] = \{(.*?)\};", ch, re.S):
            arrays[name] = [float(t) for t in body.replace("\n", " ").split(",") if t.strip()]
        pm = re.search(r"EQ\(prob\*10000, expectedPolicy\[\w+\], std::min\(([0-9.]+), expectedPolicy\[\w+\] \* ([0-9.]+) \+ "
                       r"([0-9.]+)\) \+ std::min\(([0-9.]+), expectedPolicy\[\w+\] \* ([0-9.]+)\)\)", ch)
        om = re.search(r"EQ\(ownership\*10000, expectedOwnership\[\w+\], ([0-9.]+)\)", ch)
        assert len(arrays["expectedPolicy"]) == xs * ys and len(arrays["expectedOwnership"]) == xs * ys
        tests.append({"model": model, "symmetry": sym, "x": xs, "y": ys, "pla": pla, "board": board,
                      "scalars": scalars, "policy_x1e4": arrays["expectedPolicy"],
                      "ownership_x1e4": arrays["expectedOwnership"],
                      "policy_tol": [float(v) for v in pm.groups()], "ownership_tol": float(om.group(1))})
    assert len(tests) == 3, len(tests)
    return tests


def board_text_of(path_txt, start_marker, xs, ys):
    """The parseBoard text of a test function (testsearchmisc.cpp)."""
    text = open(path_txt).read()
    seg = text[text.index(start_marker):]
    bm = re.search(r'Board::parseBoard\(%d,%d,R"%%%%\((.*?)\)%%%%"\)' % (xs, ys), seg, re.S)
    return bm.group(1)


def main():
    build_featurizer()
    shutil.copy(os.path.join(REF, "tests", "models", G103), os.path.join(HERE, G103))
    sizes = decode_tiny_models()
    misc = os.path.join(REF, "tests", "testsearchmisc.cpp")
    cases = []

    # runNNOnTinyBoard: white to move, Tromp-Taylor, 6x6 tensor, symmetry 3.
    tiny_board = board_text_of(misc, "void Tests::runNNOnTinyBoard", 5, 5)
    feat = featurize(case_spec("tinyboard", 5, 5, 6, 6, "w", 7, tiny_board))[0]
    blocks = parse_debug_prints(os.path.join(REF, "tests", "results", "runNNOnTinyBoardTest.txt"), 5, 5)
    assert len(blocks) == 1
    cases.append({**feat, "name": "runNNOnTinyBoard", "model": G170, "symmetry": 3, "check": "printed", **blocks[0]})

    # runNNSymmetries: black to move, 13x13 tensor, symmetries 0..7.
    sym_board = board_text_of(misc, "void Tests::runNNSymmetries", 9, 13)
    feat = featurize(case_spec("symmetries", 9, 13, 13, 13, "b", 4, sym_board))[0]
    blocks = parse_debug_prints(os.path.join(REF, "tests", "results", "runNNSymmetriesTest.txt"), 9, 13)
    assert len(blocks) == 8
    for s, b in enumerate(blocks):
        cases.append({**feat, "name": f"runNNSymmetries-sym{s}", "model": G103, "symmetry": s, "check": "printed", **b})

    # tinymodel.cpp: 19x19 tensors (NNPos::MAX_BOARD_LEN), inputs version 7.
    for k, t in enumerate(parse_tinymodel_tests()):
        feat = featurize(case_spec(f"tinymodel{k}", t["x"], t["y"], 19, 19, t["pla"], 7, t["board"]))[0]
        cases.append({**feat, "name": f"tinymodel-{k}-{t['model'].split('_')[1].split('.')[0]}-sym{t['symmetry']}",
                      "check": "tinymodel", **{kk: v for kk, v in t.items() if kk not in ("board", "x", "y", "pla")}})

    # The spread between the reference's own fp16 and fp32 records of the
    # symmetries test (runsearchtestsfp16.sh:21 vs runsearchtests.sh:44, same
    # GPU): per scalar, and in permille for policy and ownership.
    fp16 = parse_debug_prints(os.path.join(REF, "tests", "results", "runNNSymmetriesTestFP16.txt"), 9, 13)
    assert len(fp16) == 8
    spread = {f: max(abs(a["scalars"][f] - b["scalars"][f]) for a, b in zip(blocks, fp16)) for f in blocks[0]["scalars"]}
    spread["policy_permille"] = max(abs(a["policy_permille"][y][x] - b["policy_permille"][y][x])
                                    for a, b in zip(blocks, fp16) for y in range(13) for x in range(9)
                                    if a["policy_permille"][y][x] is not None)
    spread["ownership_permille"] = max(abs(a["ownership_permille"][y][x] - b["ownership_permille"][y][x])
                                       for a, b in zip(blocks, fp16) for y in range(13) for x in range(9))

    with open(os.path.join(HERE, "whole_net_golden.json"), "w") as f:
        json.dump({"source": "make_whole_net_golden.py", "reference_fp16_spread": spread, "cases": cases}, f,
                  separators=(",", ":"))
    print(f"wrote {len(cases)} cases; tiny models {sizes}")


if __name__ == "__main__":
    main()
