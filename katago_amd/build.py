"""Builds the native libraries of this repository in-tree.

  katago_amd/lib/libkatago_hip.so   hipcc, gfx950: kernels + C ABI (include/katago_hip.h)
  katago_amd/lib/libkatago_host.so  g++: ModelDesc parser, NeuralNet::* backend
                                    (hipbackend.cpp) and its C shim (include/katago_nn.h)
  oracle/liboracle_eigen.so         g++: CPU oracle (test infrastructure)
  oracle/_ref/                      g++: KataGo's own featurizer and model parser
                                    built from the reference sources (checkers;
                                    only where /root/reference exists)

Every call recompiles (the driver uses it as the "does it build" check).
Objects go to katago_amd/_build/. Run as ``python -m katago_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import json
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "katago_amd")
LIB_DIR = os.path.join(PKG, "lib")
BUILD_DIR = os.path.join(PKG, "_build")
ORACLE_DIR = os.path.join(ROOT, "oracle")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

# Packed-FP32 instructions stay disabled in all device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result"]
# The oracle is also the timed CPU baseline; AVX2/FMA is available on every
# x86-64 server CPU these GPU hosts use.
ORACLE_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-mavx2", "-mfma", "-Wall"]

HIP_SOURCES = ["kgh_conv.hip", "kgh_kernels.hip", "kgh_transformer.hip", "kgh_api.hip"]
HOST_SOURCES = [
    "host/core/global.cpp",
    "host/neuralnet/desc.cpp",
    "host/neuralnet/nninputs.cpp",
    "host/neuralnet/hipbackend.cpp",
    "host/neuralnet/nneval.cpp",
    "host/neuralnet/capi.cpp",
    "host/neuralnet/featurize.cpp",
]
ORACLE_SOURCES = [
    os.path.join(ORACLE_DIR, "eigen_oracle.cpp"),
    os.path.join(PKG, "host/core/global.cpp"),
    os.path.join(PKG, "host/neuralnet/desc.cpp"),
    os.path.join(PKG, "host/neuralnet/nninputs.cpp"),
]


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|LDS Size \[bytes/block\]|"
                     r"VGPRs Spill|SGPRs Spill|Occupancy \[waves/SIMD\]):\s*(\S+)")
_FIELDS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch", "LDS Size [bytes/block]": "lds",
           "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill", "Occupancy [waves/SIMD]": "occupancy"}


def _resource_usage(compiler_output: str) -> dict:
    """Per-kernel registers, scratch and LDS from the compiler's
    kernel-resource-usage remarks."""
    kernels, cur = {}, None
    for key, val in _REMARK.findall(compiler_output):
        if key == "Function Name":
            cur = kernels.setdefault(val, {})
        elif cur is not None:
            cur[_FIELDS[key]] = int(val)
    return kernels


def build_hip(jobs: int = 8) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", os.path.join(PKG, "csrc", src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        outputs = list(ex.map(_run, cmds))
    usage = {}
    for o in outputs:
        usage.update(_resource_usage(o))
    with open(os.path.join(LIB_DIR, "kernel_resources.json"), "w") as f:
        json.dump(usage, f, indent=1, sort_keys=True)
    out = os.path.join(LIB_DIR, "libkatago_hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


def build_host() -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    out = os.path.join(LIB_DIR, "libkatago_host.so")
    tmp = out + ".tmp"
    _run([CXX, *HOST_FLAGS, "-shared", "-I", os.path.join(ROOT, "include"),
          *[os.path.join(PKG, s) for s in HOST_SOURCES],
          "-L", LIB_DIR, "-lkatago_hip", "-lz", "-Wl,-rpath,$ORIGIN", "-o", tmp])
    os.replace(tmp, out)
    return out


def build_oracle() -> str:
    out = os.path.join(ORACLE_DIR, "liboracle_eigen.so")
    tmp = out + ".tmp"
    _run([CXX, *ORACLE_FLAGS, "-shared", *ORACLE_SOURCES, "-lz", "-lpthread", "-o", tmp])
    os.replace(tmp, out)
    return out


REF_CPP = "/root/reference/cpp"


def build_ref() -> str | None:
    """oracle/_ref: KataGo's own featurizer and model parser compiled from the
    reference sources where they lie (oracle/Makefile.ref), as checkers for the
    tests' fixtures. Only where the reference tree exists (this container);
    the GPU boxes use what was built here."""
    if not os.path.isdir(REF_CPP):
        return None
    _run(["make", "-B", "-s", "-j8", "-f", os.path.join(ORACLE_DIR, "Makefile.ref"), f"REF={REF_CPP}"] + ["-C", ROOT])
    return os.path.join(ORACLE_DIR, "_ref")


def build_all(verbose: bool = True) -> None:
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        f_oracle = ex.submit(build_oracle)
        hip = build_hip()
        if verbose:
            print("built", hip, flush=True)
        oracle = f_oracle.result()
        if verbose:
            print("built", oracle, flush=True)
    host = build_host()
    if verbose:
        print("built", host, flush=True)
    ref = build_ref()
    if verbose and ref:
        print("built", ref, flush=True)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
