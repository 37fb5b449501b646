"""Regenerates the golden fixtures in this directory from the reference tree.

Run in a container where /root/reference exists:
    python tests/golden/make_golden.py

Outputs (data only; the tests never read /root/reference):
  layer_kats.json     the layer known-answer tests of
                      /root/reference/cpp/tests/testnn.cpp:107-920 (conv 1x1/3x3/5x5,
                      batch norm with and without mask, residual block,
                      global-pooling residual block): geometry, descriptor in the
                      model text format, NCHW input, mask and expected output.
  symmetry_golden.json  the dihedral-symmetry copies printed by
                      Tests::runNNSymmetryTests (testnn.cpp:938-1008), with the
                      outputs recorded in
                      /root/reference/cpp/tests/results/runOutputTests.txt.
  g170-b6c96-s175395328-d26788732.bin.gz   a trained 6-block model the
                      reference's own tests load (cpp/tests/models/).
"""
from __future__ import annotations

import json
import math
import os
import re
import shutil

REF = "/root/reference/cpp"
HERE = os.path.dirname(os.path.abspath(__file__))


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _floats(body: str) -> list[float]:
    vals = [v.strip() for v in body.replace("\n", " ").split(",") if v.strip()]
    return [float(v.rstrip("f")) for v in vals]


def _function_body(text: str, name: str) -> str:
    start = text.index(name)
    i = text.index("{", start)
    depth = 0
    for j in range(i, len(text)):
        if text[j] == "{":
            depth += 1
        elif text[j] == "}":
            depth -= 1
            if depth == 0:
                return text[i:j + 1]
    raise ValueError(name)


def _statements(body: str):
    """Splits on ';' at the top of parentheses (vector literals contain commas only)."""
    out, cur, depth = [], [], 0
    for ch in body:
        if ch == "(":
            depth += 1
        elif ch == ")":
            depth -= 1
        if ch == ";" and depth == 0:
            out.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    return out


def _scalar(v: str, env: dict):
    v = v.strip()
    if v in env:
        return env[v]
    if v in ("true", "false"):
        return v == "true"
    m = re.fullmatch(r'"([^"]*)"', v)
    if m:
        return m.group(1)
    return float(v.rstrip("f")) if any(c in v for c in ".e") else int(v)


def _nchw_to_nhwc(vec, n, c, h, w):
    out = [0.0] * len(vec)
    for b in range(n):
        for ch in range(c):
            for y in range(h):
                for x in range(w):
                    out[((b * h + y) * w + x) * c + ch] = vec[((b * c + ch) * h + y) * w + x]
    return out


# ---------------------------------------------------------------------------
# Descriptor text (model text format, version >= 11 grammar)

def _conv_text(name: str, d: dict) -> str:
    ky, kx, ic, oc = d["convYSize"], d["convXSize"], d["inChannels"], d["outChannels"]
    w = d["weights"]  # (oc, ic, y, x)
    file_order = []
    for y in range(ky):
        for x in range(kx):
            for i in range(ic):
                for o in range(oc):
                    file_order.append(w[((o * ic + i) * ky + y) * kx + x])
    hdr = f"{name} {ky} {kx} {ic} {oc} {d.get('dilationY', 1)} {d.get('dilationX', 1)}"
    return hdr + "\n" + " ".join(repr(v) for v in file_order) + "\n"


def _bn_text(name: str, d: dict) -> str:
    # Both flags set so that scale and bias reach computeMerged exactly as in
    # the test, which sets them even when hasScale/hasBias is false.
    c = d["numChannels"]
    parts = [f"{name} {c} {d['epsilon']!r} 1 1"]
    for key in ("mean", "variance", "scale", "bias"):
        parts.append(" ".join(repr(v) for v in d[key]))
    return "\n".join(parts) + "\n"


def _matmul_text(name: str, d: dict) -> str:
    return f"{name} {d['inChannels']} {d['outChannels']}\n" + " ".join(repr(v) for v in d["weights"]) + "\n"


def _act_text(name: str) -> str:
    return f"{name} ACTIVATION_RELU\n"


def _desc_text(kind: str, desc: dict) -> str:
    if kind == "conv":
        return _conv_text("conv", desc)
    if kind == "bn":
        return _bn_text("bn", desc)
    if kind == "residual":
        return ("block\n" + _bn_text("preBN", desc["preBN"]) + _act_text("preAct") +
                _conv_text("regularConv", desc["regularConv"]) + _bn_text("midBN", desc["midBN"]) +
                _act_text("midAct") + _conv_text("finalConv", desc["finalConv"]))
    if kind == "gpool":
        return ("block\n" + _bn_text("preBN", desc["preBN"]) + _act_text("preAct") +
                _conv_text("regularConv", desc["regularConv"]) + _conv_text("gpoolConv", desc["gpoolConv"]) +
                _bn_text("gpoolBN", desc["gpoolBN"]) + _act_text("gpoolAct") +
                _matmul_text("gpoolToBiasMul", desc["gpoolToBiasMul"]) + _bn_text("midBN", desc["midBN"]) +
                _act_text("midAct") + _conv_text("finalConv", desc["finalConv"]))
    raise ValueError(kind)


def layer_kats() -> list[dict]:
    src = _strip_comments(open(os.path.join(REF, "tests/testnn.cpp")).read())
    kats = []
    for fn, kind in (("testConvLayer(", "conv"), ("testBatchNormLayer(", "bn"), ("testResidualBlock(", "residual"),
                     ("testGlobalPoolingResidualBlock(", "gpool")):
        body = _function_body(src, "static void " + fn)
        # skip the testConfigurations lambda
        lam = body.index("auto testConfigurations")
        lam_end = body.index("};", lam) + 2
        body = body[:lam] + body[lam_end:]
        env: dict = {}
        desc: dict = {}
        for st in _statements(body):
            st = re.sub(r"^[\s{}]+", "", st).strip()
            if not st:
                continue
            m = re.fullmatch(r"int (\w+) = (.+)", st)
            if m:
                env[m.group(1)] = _scalar(m.group(2), env)
                continue
            m = re.fullmatch(r"vector<float> (\w+)\(\{(.*)\}\)", st, re.S)
            if m:
                env[m.group(1)] = _floats(m.group(2))
                continue
            m = re.fullmatch(r'string label\("([^"]*)"\)', st)
            if m:
                env["label"] = m.group(1)
                continue
            m = re.fullmatch(r"(\w+) desc", st)
            if m:
                desc = {}
                continue
            m = re.fullmatch(r"desc\.([\w.]+) = vector<float>\(\{(.*)\}\)", st, re.S)
            if m:
                _set(desc, m.group(1), _floats(m.group(2)))
                continue
            m = re.fullmatch(r"desc\.([\w.]+) = (.+)", st, re.S)
            if m:
                _set(desc, m.group(1), _scalar(m.group(2), env))
                continue
            if re.fullmatch(r"desc\.[\w.]*computeMerged\(\)", st):
                continue
            m = re.fullmatch(r"for\(int i = (\d+); i<(\d+); i\+\+\) \{\s*expected\[i\] \+= \(float\)\((.*)\)", st, re.S)
            if m:
                lo, hi, expr = int(m.group(1)), int(m.group(2)), m.group(3)
                add = eval(" ".join(expr.split()).replace("sqrt", "math.sqrt"), {"math": math})
                env.setdefault("_adds", []).append((lo, hi, add))
                continue
            if re.fullmatch(r"expected\[i\] \*= mask\[i\]", st):
                continue
            if st.startswith("testConfigurations"):
                expected = list(env["expected"])
                for lo, hi, add in env.pop("_adds", []):
                    for i in range(lo, hi):
                        expected[i] = float(
                            __import__("numpy").float32(__import__("numpy").float32(expected[i]) + __import__("numpy").float32(add))
                            * __import__("numpy").float32(env["mask"][i]))
                inc = desc.get("inChannels") or desc.get("numChannels") or desc["preBN"]["numChannels"]
                outc = desc.get("outChannels") or desc.get("numChannels") or desc["preBN"]["numChannels"]
                kats.append({
                    "kind": kind,
                    "label": env["label"],
                    "batch": env["batchSize"],
                    "nnXLen": env["nnXLen"],
                    "nnYLen": env["nnYLen"],
                    "inChannels": inc,
                    "outChannels": outc,
                    "desc_text": _desc_text(kind, desc),
                    "input_nchw": env["input"],
                    "mask": env.get("mask") if kind != "conv" else None,
                    "expected_nchw": expected,
                    "source": "cpp/tests/testnn.cpp " + fn.rstrip("("),
                })
                continue
            if st.startswith(("for(int", "expected[")):
                raise ValueError("unhandled statement: " + st[:80])
        # names declared inside desc paths
    return kats


def _set(d: dict, path: str, value) -> None:
    keys = path.split(".")
    for k in keys[:-1]:
        d = d.setdefault(k, {})
    d[keys[-1]] = value


def symmetry_golden() -> list[dict]:
    src = _strip_comments(open(os.path.join(REF, "tests/testnn.cpp")).read())
    body = _function_body(src, "void Tests::runNNSymmetryTests")
    inputs = [_floats(m) for m in re.findall(r"vector<float> input\(\{(.*?)\}\)", body, re.S)]
    calls = re.findall(r'testConfigurations\("([^"]+)",(\d+),(\d+),(\d+),(\d+),input\)', body)
    lines = open(os.path.join(REF, "tests/results/runOutputTests.txt")).read().splitlines()
    start = next(i for i, l in enumerate(lines) if l.startswith("Symmetry 3-1-3-3 useNHWC 0 0"))
    cases = []
    pos = start
    for ci, (label, batch, chans, nnx, nny) in enumerate(calls):
        batch, chans, nnx, nny = int(batch), int(chans), int(nnx), int(nny)
        inp = inputs[0] if ci < 2 else inputs[1]
        for nhwc in (0, 1):
            for sym in range(8):
                assert lines[pos].strip() == f"{label} useNHWC {nhwc} {sym}", lines[pos]
                exp = [float(v) for v in lines[pos + 1].split()]
                src_arr = _nchw_to_nhwc(inp, batch, chans, nny, nnx) if nhwc else list(inp)
                cases.append({"label": label, "kind": "input", "nhwc": nhwc, "symmetry": sym, "nSize": batch,
                              "hSize": nnx, "wSize": nny, "cSize": chans, "src": src_arr, "expected": exp})
                pos += 2
        for sym in range(8):
            assert lines[pos].strip() == f"{label} OUTPUT", lines[pos]
            exp = [float(v) for v in lines[pos + 1].split()]
            cases.append({"label": label, "kind": "output", "nhwc": 0, "symmetry": sym, "nSize": batch * chans,
                          "hSize": nnx, "wSize": nny, "cSize": 1, "src": list(inp), "expected": exp})
            pos += 2
    return cases


def main() -> None:
    kats = layer_kats()
    with open(os.path.join(HERE, "layer_kats.json"), "w") as f:
        json.dump({"source": "/root/reference/cpp/tests/testnn.cpp:107-920", "kats": kats}, f, indent=1)
    sym = symmetry_golden()
    with open(os.path.join(HERE, "symmetry_golden.json"), "w") as f:
        json.dump({"source": "/root/reference/cpp/tests/testnn.cpp:938-1008 + tests/results/runOutputTests.txt",
                   "cases": sym}, f)
    model = "g170-b6c96-s175395328-d26788732.bin.gz"
    shutil.copyfile(os.path.join(REF, "tests/models", model), os.path.join(HERE, model))
    print(f"{len(kats)} layer KATs, {len(sym)} symmetry cases, model {model}")


if __name__ == "__main__":
    main()
