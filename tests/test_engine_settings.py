"""g4v_engine's handling of reference settings it does not restate: the process ends with exit
code 2 and a message before it touches a device (runs on the CPU), instead of silently taking
another path than the reference engine (engine/gemma4_engine.cpp E:1211-1216, 1515)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "gemma4-e2b-laptop-cpu_amd", "g4v_engine")


@pytest.mark.parametrize("env,word", [
    ({"ENGINE_TAU": "0.3"}, "ENGINE_TAU"),            # E:1515, 1561, 1644: the chain's probability cut
    ({"ENGINE_NO_TILED": "1"}, "ENGINE_NO_TILED"),    # E:1213, 1328: run_mh where attn_tile runs
    ({"ENGINE_ATT_PAR": "64"}, "ENGINE_ATT_PAR"),     # E:1214
    ({"ENGINE_SPLITKV": "0"}, "ENGINE_SPLITKV"),      # E:1212
    ({"ENGINE_FAKE_CTX": "100", "ENGINE_SLOTS": "2"}, "ENGINE_FAKE_CTX"),  # E:1211 with E:1573 slots
    ({"ENGINE_FAKE_CTX": "5000"}, "ENGINE_FAKE_CTX"),  # beyond ENGINE_CTX (4096)
])
def test_unsupported_settings_end_the_process(env, word):
    if not os.path.exists(EXE):
        pytest.skip("g4v_engine not built")
    e = dict(os.environ)
    for k in ("ENGINE_TAU", "ENGINE_NO_TILED", "ENGINE_ATT_PAR", "ENGINE_SPLITKV", "ENGINE_FAKE_CTX", "ENGINE_SLOTS",
              "ENGINE_CTX"):
        e.pop(k, None)
    e.update(env)
    p = subprocess.run([EXE, "synth:1:4096:2:6144", "-", "-", "4"], env=e, capture_output=True, text=True, timeout=60)
    assert p.returncode == 2 and word in p.stderr, (p.returncode, p.stderr[-500:])


def test_tau_zero_is_the_default_path():
    """ENGINE_TAU=0 is the reference's default (every draft kept, E:1515): not refused"""
    if not os.path.exists(EXE):
        pytest.skip("g4v_engine not built")
    e = dict(os.environ, ENGINE_TAU="0")
    for k in ("ENGINE_NO_TILED", "ENGINE_ATT_PAR", "ENGINE_SPLITKV", "ENGINE_FAKE_CTX"):
        e.pop(k, None)
    # no device here: the process passes the settings check and fails at context creation instead
    p = subprocess.run([EXE, "synth:1:4096:2:6144", "-", "-", "4"], env=e, capture_output=True, text=True, timeout=120)
    assert "not supported" not in p.stderr, p.stderr[-500:]
