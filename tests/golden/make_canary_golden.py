"""Writes tests/golden/canary_golden.json.gz: the positions of KataGo's canary
tests (Tests::runCanaryTests, /root/reference/cpp/tests/testnnevalcanary.cpp:14-245)
as the neural-net input rows KataGo's own NNInputs::fillRowV7 builds for them,
with the legal moves the evaluator's post-processing reads, and each canary's
assertions as data.

The game records and thresholds below are the canary test's data
(testnnevalcanary.cpp:44-51, 79-86, 113-120, 148-157, 180-189, 215-222; the
assertions at :67-76, :102-111, :136-145, :165-176, :197-206, :238-245; the
lenience for nets of trunk depth <= 21 at :27-32). The rows come from
oracle/_ref/ref_featurize (KataGo's board, history and fillRowV7 compiled from
the reference sources by oracle/Makefile.ref), which also checks this
repository's featurizer on each position (all values equal).

Run from the repository root in the build container (needs oracle/_ref):
    python tests/golden/make_canary_golden.py
"""
import gzip
import json
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
DRIVER = os.path.join(ROOT, "oracle", "_ref", "ref_featurize")
OUT = os.path.join(ROOT, "tests", "golden", "canary_golden.json.gz")

GAME_A = ("(;GM[1]FF[4]CA[UTF-8]AP[CGoban:3]ST[2]RU[Chinese]SZ[19]KM[7]PW[White]PB[Black];B[pd];W[pp];B[dd];W[dp];B[qn];"
          "W[nq];B[cq];W[dq];B[cp];W[do];B[bn];W[cc];B[cd];W[dc];B[ec];W[eb];B[fb];W[fc];B[ed];W[gb];B[db];W[fa];B[cb];"
          "W[qo];B[pn];W[nc];B[qj];W[qc];B[qd];W[pc];B[od];W[nd];B[ne];W[me];B[mf];W[nf])")
GAME_B = ("(;GM[1]FF[4]CA[UTF-8]AP[CGoban:3]ST[2]RU[Chinese]SZ[19]KM[7]PW[White]PB[Black];B[qd];W[dd];B[pp];W[dp];B[cf];"
          "W[fc];B[nd];W[nq];B[cq];W[dq];B[cp];W[cn];B[co];W[do];B[bn];W[cm];B[bm];W[cl];B[qn];W[pq];B[qq];W[qr];B[oq])")
GAME_C = "(;FF[4]GM[1]CA[UTF-8]RU[Japanese]KM[6]SZ[16:11];B[md];W[nh];B[dh];W[cd];B[lh];W[li];B[ki])"

# (name, game, turns, komi override, checks). A check is
# [quantity, op, bound, lenience kind]: the bound is widened by the
# lenience of that kind (policy, winrate, lead, score) for small nets.
EVEN_VALUE = [["white_win", ">", 0.30, "winrate"], ["white_win", "<", 0.70, "winrate"], ["white_no_result", "<", 0.03, None],
              ["white_lead", ">", -2.5, "lead"], ["white_lead", "<", 2.5, "lead"], ["white_score_mean", ">", -3.5, "score"],
              ["white_score_mean", "<", 3.5, "score"]]
CANARIES = [
    ("opening-E16", GAME_A, 18, None, [["policy:E16", ">=", 0.95, None], ["policy:pass", "<=", 0.005, None]] + EVEN_VALUE),
    ("opening-P15", GAME_A, 36, None, [["policy:P15", ">=", 0.85, "policy"], ["policy:pass", "<=", 0.005, None]] + EVEN_VALUE),
    ("corner-Q2", GAME_B, 23, None, [["policy:Q2", ">=", 0.95, None], ["policy:pass", "<=", 0.005, None]] + EVEN_VALUE),
    ("corner-komi-7", GAME_B, 23, -7.0, [["white_win", "<", 0.1, "winrate"], ["white_lead", "<", -9.0, "lead"],
                                         ["white_lead", ">", -19.0, "lead"], ["white_score_mean", "<", -8.0, "score"],
                                         ["white_score_mean", ">", -22.0, "score"]]),
    ("corner-komi21", GAME_B, 23, 21.0, [["white_win", ">", 0.9, "winrate"], ["white_lead", ">", 9.0, "lead"],
                                         ["white_lead", "<", 19.0, "lead"], ["white_score_mean", ">", 8.0, "score"],
                                         ["white_score_mean", "<", 22.0, "score"]]),
    ("rect16x11-N3", GAME_C, 7, None, [["policy:N3", ">=", 0.80, "policy"], ["white_win", ">", 0.20, "winrate"],
                                       ["white_win", "<", 0.80, "winrate"], ["white_no_result", "<", 0.06, None],
                                       ["white_lead", ">", -2.5, "lead"], ["white_lead", "<", 2.5, "lead"],
                                       ["white_score_mean", ">", -3.5, "score"], ["white_score_mean", "<", 3.5, "score"]]),
]
# testnnevalcanary.cpp:27-32: nets of trunk spatial conv depth <= 21.
LENIENCE_SMALL_NET = {"policy": 0.05, "winrate": 0.12, "lead": 2.0, "score": 3.0}


def parse_sgf(text):
    size = re.search(r"SZ\[(\d+)(?::(\d+))?\]", text)
    xs = int(size.group(1))
    ys = int(size.group(2)) if size.group(2) else xs
    komi = float(re.search(r"KM\[([-\d.]+)\]", text).group(1))
    rules = re.search(r"RU\[(\w+)\]", text).group(1).lower()
    moves = [(c.lower(), ord(m[0]) - 97, ord(m[1]) - 97) for c, m in re.findall(r";([BW])\[([a-s]{2})\]", text)]
    return xs, ys, komi, rules, moves


def main():
    if not os.path.exists(DRIVER):
        sys.exit("oracle/_ref/ref_featurize is missing: build it with make -f oracle/Makefile.ref")
    records = []
    for name, game, turns, komi_override, checks in CANARIES:
        xs, ys, komi, rules, moves = parse_sgf(game)
        moves = moves[:turns]
        komi = komi if komi_override is None else komi_override
        cmd = f"moves {name} {xs} {ys} 19 19 {rules} {komi} {len(moves)} " + " ".join(f"{c} {x} {y}" for c, x, y in moves)
        out = subprocess.run([DRIVER], input=cmd + "\n", capture_output=True, text=True, check=True).stdout.splitlines()
        compare, row = json.loads(out[0]), json.loads(out[1])
        assert compare["differing"] == 0, compare
        records.append({"name": name, "x_size": xs, "y_size": ys, "rules": rules, "komi": komi, "turns": turns,
                        "pla": row["pla"], "no_result_disabled": row["no_result_disabled"], "spatial_nhwc": row["spatial_nhwc"],
                        "global": row["global"], "legal": row["legal"], "checks": checks})
    with gzip.open(OUT, "wt") as f:
        json.dump({"lenience_small_net": LENIENCE_SMALL_NET, "nnx": 19, "nny": 19, "canaries": records}, f)
    print("wrote", OUT, len(records), "canaries")


if __name__ == "__main__":
    main()
