import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _libs_built() -> bool:
    return all(os.path.exists(p) for p in (
        os.path.join(ROOT, "katago_amd", "lib", "libkatago_hip.so"),
        os.path.join(ROOT, "katago_amd", "lib", "libkatago_host.so"),
        os.path.join(ROOT, "katago_amd", "lib", "kernel_resources.json"),
        os.path.join(ROOT, "oracle", "liboracle_eigen.so"),
    ))


@pytest.fixture(scope="session", autouse=True)
def built_libraries():
    """Builds the native libraries once if nothing is built yet."""
    if not _libs_built():
        from katago_amd import build
        build.build_all(verbose=False)
    return True


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return str(tmp_path_factory.mktemp("models"))


GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    try:
        from helpers import ARGMAX_ROWS, ARGMAX_TIES
    except ImportError:
        return
    if ARGMAX_ROWS[0] == 0:
        return
    terminalreporter.write_line(f"argmax tie allowance used on {len(ARGMAX_TIES)} of {ARGMAX_ROWS[0]} whole-net rows compared")
    for line in ARGMAX_TIES:
        terminalreporter.write_line("  " + line)
