"""The model-file parser (desc.cpp) and the featurizer (featurize.cpp) built
with AddressSanitizer + UndefinedBehaviorSanitizer (and the featurizer, whose
worker threads share the positions, with ThreadSanitizer), host code only
(g++), driven by tests/sanitize/parse_stress.cpp and
tests/sanitize/featurize_stress.cpp.

* Parser: every model file under tests/golden parsed as shipped, and about
  160 mutants of each of the two tiny nets (truncated at many lengths, single
  bytes overwritten in the header and anywhere): each must parse or be
  refused with an exception, with no sanitizer report.
* Featurizer: the 300 fixture positions featurized one at a time and in
  per-tensor-size batches on four threads; the rows must equal the fixture's
  expected bits (KataGo's own fillRowV7, nninputs.cpp:2273-2720) and each
  other."""
import glob
import gzip
import json
import os
import subprocess

import numpy as np
import pytest

from helpers import GOLDEN

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN = (["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"], "ERROR: AddressSanitizer")
TSAN = (["-fsanitize=thread"], "WARNING: ThreadSanitizer")


def _build(tmp_path, name, sources, flags, libs=()):
    exe = str(tmp_path / name)
    build = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-pthread", *flags, "-o", exe, *sources, *libs],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if build.returncode != 0 and "sanitize" in build.stdout and ("cannot find" in build.stdout or "unrecognized" in build.stdout):
        pytest.skip("this g++ cannot build with " + " ".join(flags))
    assert build.returncode == 0, build.stdout
    return exe


def _run(cmd, marker, timeout=600):
    env = dict(os.environ, ASAN_OPTIONS="allocator_may_return_null=1:detect_leaks=1")
    run = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=timeout, env=env)
    assert marker not in run.stderr, run.stderr[-4000:]
    assert "runtime error" not in run.stderr, run.stderr[-4000:]
    assert run.returncode == 0, (run.stdout[-2000:], run.stderr[-4000:])
    return run.stdout


def test_parser_on_model_files_and_mutants_under_asan_ubsan(tmp_path):
    exe = _build(tmp_path, "parse", [
        os.path.join(ROOT, "tests", "sanitize", "parse_stress.cpp"),
        os.path.join(ROOT, "katago_amd", "host", "neuralnet", "desc.cpp"),
        os.path.join(ROOT, "katago_amd", "host", "core", "global.cpp"),
    ], ASAN[0], ["-lz"])
    models = sorted(glob.glob(os.path.join(GOLDEN, "*.bin.gz")) + glob.glob(os.path.join(GOLDEN, "*.txt.gz")))
    small = [m for m in models if os.path.getsize(m) < 1 << 20]
    assert small, "no small model fixtures"
    out = _run([exe, str(tmp_path), *small], ASAN[1])
    assert "mutants parsed" in out and out.rstrip().endswith("done"), out
    refused = int(out.split("refused")[-1].split()[0])
    assert refused > 0, out  # the truncations at least are refused
    # The larger files (transformer, text-format and older-version nets) are
    # parsed whole: their mutants would take minutes under the sanitizers.
    out = _run([exe, "--parse-only", str(tmp_path), *[m for m in models if m not in small]], ASAN[1], timeout=900)
    assert out.rstrip().endswith("done"), out


def _positions_text(fixtures):
    lines = []
    for fx in fixtures:
        n = fx["x_size"] * fx["y_size"]
        f = [fx["nnx"], fx["nny"], fx["x_size"], fx["y_size"], fx["next_player"]]
        for k in range(3):
            f += list(fx["colors"][k])
        f += list(fx["ko_point"])
        for k in range(3):
            f += list(fx["chain_head"][k]) + list(fx["chain_next"][k])
        for key in ("super_ko_banned", "ko_recap_blocked", "second_encore_start_colors"):
            v = fx.get(key)
            f += [0] if v is None else [1] + list(v)
            assert v is None or len(v) == n
        f += [fx["num_moves"], *fx["move_point"], *fx["move_player"]]
        f += [fx[k] for k in ("num_approx_valid_turns_this_phase", "encore_phase", "ko_rule", "scoring_rule", "tax_rule",
                              "multi_stone_suicide_legal", "has_button")]
        f += [repr(float(fx["self_komi"]))]
        f += [int(fx[k]) for k in ("pass_would_end_game", "pass_would_end_phase", "suppress_end_game_from_friendly_pass",
                                   "is_game_finished", "is_past_normal_phase_end", "conservative_pass_and_is_root",
                                   "enable_passing_hacks")]
        f += [repr(float(fx["playout_doubling_advantage"])), fx["max_history"]]
        lines.append(" ".join(str(v) for v in f))
    return "\n".join(lines) + "\n"


@pytest.mark.parametrize("flags,marker", [ASAN, TSAN], ids=["asan-ubsan", "tsan"])
def test_featurizer_on_fixture_positions_under_sanitizers(tmp_path, flags, marker):
    exe = _build(tmp_path, "featurize", [
        os.path.join(ROOT, "tests", "sanitize", "featurize_stress.cpp"),
        os.path.join(ROOT, "katago_amd", "host", "neuralnet", "featurize.cpp"),
    ], flags)
    with gzip.open(os.path.join(GOLDEN, "featurize_golden.json.gz"), "rt") as f:
        fixtures = json.load(f)["positions"]
    pos = tmp_path / "positions.txt"
    pos.write_text(_positions_text(fixtures))
    out_bin = tmp_path / "rows.bin"
    out = _run([exe, str(pos), str(out_bin)], marker)
    assert f"positions {len(fixtures)}" in out and "batch mismatches 0" in out, out
    rows = np.fromfile(out_bin, np.float32)
    at = 0
    for fx in fixtures:
        hw = fx["nnx"] * fx["nny"]
        digits = fx["spatial_nhwc_bits"]
        bits = np.unpackbits(np.frombuffer(bytes.fromhex(digits + ("0" if len(digits) % 2 else "")), np.uint8))
        want_sp = bits[: hw * 22].astype(np.float32)
        want_gl = np.asarray(fx["global"], np.float32)
        got_sp = rows[at:at + hw * 22]
        got_gl = rows[at + hw * 22:at + hw * 22 + 19]
        at += hw * 22 + 19
        assert np.array_equal(got_sp, want_sp), fx["fixture"]
        assert np.array_equal(got_gl, want_gl), fx["fixture"]
    assert at == rows.size
