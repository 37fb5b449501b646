"""The backend file compiles unchanged inside KataGo's own source tree.

hipbackend.cpp is meant to be copied into cpp/neuralnet/ of a KataGo checkout
(next to eigenbackend.cpp, cudabackend.cpp, ...) and built against KataGo's
real headers (nninterface.h, nneval.h, desc.h, nninputs.h, core/*), not this
repository's mirrors of them. This test builds such a tree out of symlinks to
/root/reference/cpp with the backend file, the featurizer adapter and their
headers added to cpp/neuralnet/, and compiles the file there with g++ (object code, -Werror on
the file's own warnings). It is skipped where the reference tree is absent
(the GPU boxes).
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_CPP = "/root/reference/cpp"

needs_reference = pytest.mark.skipif(not os.path.isdir(os.path.join(REF_CPP, "neuralnet")),
                                     reason="needs the reference source tree")


def _katago_tree(tmp_path):
    cpp = tmp_path / "cpp"
    cpp.mkdir()
    for name in os.listdir(REF_CPP):
        if name != "neuralnet":
            os.symlink(os.path.join(REF_CPP, name), cpp / name)
    nn_dir = cpp / "neuralnet"
    nn_dir.mkdir()
    for name in os.listdir(os.path.join(REF_CPP, "neuralnet")):
        os.symlink(os.path.join(REF_CPP, "neuralnet", name), nn_dir / name)
    for f in ("hipbackend.cpp", "featurizeadapter.cpp", "featurizeadapter.h"):
        shutil.copy(os.path.join(ROOT, "katago_amd", "host", "neuralnet", f), nn_dir / f)
    for h in ("katago_hip.h", "katago_hip_backend.h", "katago_featurize.h"):
        shutil.copy(os.path.join(ROOT, "include", h), nn_dir / h)
    return cpp


@needs_reference
def test_hipbackend_compiles_inside_katago_tree(tmp_path):
    cpp = _katago_tree(tmp_path)
    src = cpp / "neuralnet" / "hipbackend.cpp"
    cmd = ["g++", "-std=c++17", "-c", "-O0", "-Wall", "-Wno-sign-compare", "-I", str(cpp / "external"),
           "-I", str(cpp / "external" / "tclap-1.2.2" / "include"), str(src), "-o", str(tmp_path / "hipbackend.o")]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, cwd=str(cpp))
    assert proc.returncode == 0, proc.stdout
    # Warnings the file itself raises (not KataGo's headers) are errors too.
    own = [l for l in proc.stdout.splitlines() if l.startswith(str(src)) and "warning" in l]
    assert not own, "\n".join(own)


@needs_reference
def test_featurize_adapter_compiles_inside_katago_tree(tmp_path):
    """The adapter from KataGo's Board / BoardHistory to kgn_position uses
    only what KataGo's game headers declare."""
    cpp = _katago_tree(tmp_path)
    src = cpp / "neuralnet" / "featurizeadapter.cpp"
    cmd = ["g++", "-std=c++17", "-c", "-O0", "-Wall", "-Wno-sign-compare", "-I", str(cpp / "external"), str(src), "-o",
           str(tmp_path / "featurizeadapter.o")]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, cwd=str(cpp))
    assert proc.returncode == 0, proc.stdout
    own = [l for l in proc.stdout.splitlines() if l.startswith(str(src)) and "warning" in l]
    assert not own, "\n".join(own)


@needs_reference
def test_hipbackend_resolves_katago_headers_not_mirrors(tmp_path):
    """The dependency list of that compile names KataGo's headers only: no
    file of this repository's host mirrors is pulled in."""
    cpp = _katago_tree(tmp_path)
    src = cpp / "neuralnet" / "hipbackend.cpp"
    proc = subprocess.run(["g++", "-std=c++17", "-MM", "-I", str(cpp / "external"), str(src)],
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, cwd=str(cpp))
    assert proc.returncode == 0, proc.stdout
    deps = proc.stdout.replace("\\\n", " ").split()
    assert any(d.endswith("neuralnet/nninterface.h") for d in deps)
    assert any(d.endswith("neuralnet/nneval.h") for d in deps)
    assert not any("katago_amd" in d for d in deps), deps
