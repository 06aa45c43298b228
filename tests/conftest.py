"""Shared fixtures: the oracle (checker), the reference harness (when built) and the
gfx950 library context.  GPU tests carry @pytest.mark.gpu."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gemma4-e2b-laptop-cpu_amd")
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


def load_g4v():
    spec = importlib.util.spec_from_file_location("g4v", os.path.join(PKG, "g4v.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import Ref, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return Ref()


@pytest.fixture(scope="session")
def g4v():
    return load_g4v()


@pytest.fixture(scope="session")
def dev(g4v):
    d = g4v.Device(0)
    yield d
    d.close()


def note(msg):
    """print the case about to run on the GPU (flushed, so a crash still names it)"""
    print(f"\n[case] {msg}", flush=True)


@pytest.fixture(scope="session")
def gemma_ckpt(orc, tmp_path_factory):
    """the synthetic Gemma-4-E2B-layout checkpoint and its drafter checkpoint, written once"""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import gemma_layout as gl
    d = str(tmp_path_factory.mktemp("gemma_ckpt"))
    note("writing the synthetic Gemma-layout checkpoint and drafter")
    E = gl.write_checkpoint(orc, d)
    gl.write_drafter(orc, d, E)
    return d
