"""The C-ABI boundary on the host: libg4v.so loads without a GPU, exports every entry point
that include/g4v.h declares, the Python mirror binds exactly those, and the product path never
reaches the oracle or a CPU fallback.  No compute call is made here (these run without a GPU),
except the host-side self-test of the library's libm expf restatement."""
import ctypes as C
import os
import re

import pytest

from conftest import PKG, ROOT, load_g4v

HEADER = os.path.join(ROOT, "include", "g4v.h")
LIB = os.path.join(PKG, "libg4v.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(g4v_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("g4v_create", "g4v_w4_upload", "g4v_w4g32_gemm", "g4v_attn_splitkv", "g4v_head_build",
                 "g4v_head_argmax", "g4v_model_synth", "g4v_verify_step"):
        assert must in names


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.skip("libg4v.so not built (run __graft_entry__.build())")
    lib = C.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_mirror_binds_exactly_the_header():
    g4v = load_g4v()
    assert sorted(g4v.SIGNATURES) == declared()


def test_no_device_is_an_error_not_a_fallback():
    """without a HIP device the context cannot be created: the call fails loudly"""
    if not os.path.exists(LIB):
        pytest.skip("libg4v.so not built")
    if os.path.exists("/dev/kfd"):  # the ROCm kernel driver: this host has (or may have) a GPU
        pytest.skip("a GPU is present")
    g4v = load_g4v()
    with pytest.raises(RuntimeError):
        g4v.Device(0)


def test_missing_library_raises(tmp_path):
    g4v = load_g4v()
    with pytest.raises(FileNotFoundError):
        g4v.load(str(tmp_path / "libg4v.so"))


def test_product_sources_do_not_reach_the_oracle():
    """the package (HIP sources, C ABI, Python mirror) never loads the oracle or the reference"""
    for dirpath, _, files in os.walk(PKG):
        if "_build" in dirpath or "__pycache__" in dirpath:
            continue
        for f in files:
            if not f.endswith((".py", ".hip", ".h", ".cpp", "Makefile")):
                continue
            text = open(os.path.join(dirpath, f)).read()
            assert "liboracle" not in text and "libg4ref" not in text and "import oracle" not in text, f
            assert "/root/reference" not in text, f


def test_expf_restatement_matches_host_libm():
    """the split merge's expf (the reference merges with libm expf, E:1019-1059) restated in
    the library equals this host's libm bit for bit on a dense sample of x <= 0"""
    if not os.path.exists(LIB):
        pytest.skip("libg4v.so not built")
    lib = C.CDLL(LIB)
    lib.g4v_expf_selftest.restype = C.c_longlong
    lib.g4v_expf_selftest.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
    assert lib.g4v_expf_selftest(0x80000000, 0xFF800000, 97) == 0  # -0 .. -inf, every 97th pattern
    assert lib.g4v_expf_selftest(0xC2AE0000, 0xC2D00000, 1) == 0  # every pattern of the underflow edge
    assert lib.g4v_expf_selftest(0xBF800000, 0xBF900000, 1) == 0  # every pattern of [-1.125, -1]
