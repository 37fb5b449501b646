"""The NNEvaluator batching server loop (nneval.cpp) built with
ThreadSanitizer, and with AddressSanitizer + UndefinedBehaviorSanitizer,
host code only (g++, no device code), and driven by tests/sanitize/serve_stress.cpp:
three server threads in debugSkipNeuralNet mode, twelve client threads,
servers killed and respawned between rounds. The reference's serve loop is
nneval.cpp:342-420, 549-750."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCES = [
    os.path.join(ROOT, "tests", "sanitize", "serve_stress.cpp"),
    os.path.join(ROOT, "tests", "sanitize", "nninterface_stub.cpp"),
    os.path.join(ROOT, "katago_amd", "host", "neuralnet", "nneval.cpp"),
    os.path.join(ROOT, "katago_amd", "host", "core", "global.cpp"),
]


@pytest.mark.parametrize("flags,marker", [
    (["-fsanitize=thread"], "WARNING: ThreadSanitizer"),
    (["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"], "ERROR: AddressSanitizer"),
], ids=["tsan", "asan-ubsan"])
def test_serve_loop_under_sanitizers(tmp_path, flags, marker):
    exe = str(tmp_path / "serve")
    build = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-pthread", *flags, "-o", exe, *SOURCES],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if build.returncode != 0 and "sanitize" in build.stdout and ("cannot find" in build.stdout or "unrecognized" in build.stdout):
        pytest.skip("this g++ cannot build with " + " ".join(flags))
    assert build.returncode == 0, build.stdout
    run = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
    assert marker not in run.stderr, run.stderr[-4000:]
    assert "runtime error" not in run.stderr, run.stderr[-4000:]
    assert run.returncode == 0, (run.stdout, run.stderr[-4000:])
    assert "bad 0" in run.stdout, run.stdout
