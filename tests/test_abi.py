"""The C-ABI library loads without a GPU and exports every entry point that
include/helrm_hip.h declares; error paths that need no device report through
GetLastError instead of aborting."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    src = open(os.path.join(ROOT, "include", "helrm_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b([A-Z]\w*)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_lattigo_surface():
    names = set(header_symbols())
    for n in ["NewScheme", "DeleteScheme", "Encode", "Decode", "Encrypt", "Decrypt", "Rotate", "RotateNew",
              "Rescale", "RescaleNew", "AddCiphertext", "AddPlaintext", "GenerateLinearTransform",
              "EvaluateLinearTransform", "GetLinearTransformRotationKeys", "GenerateLinearTransformRotationKey",
              "GetModuliChain", "FreeCArray", "DeleteCiphertext", "DeletePlaintext", "AddRotationKey"]:
        assert n in names, n


def test_library_exports_every_declared_symbol():
    from helrm_amd import library_path
    lib = ctypes.CDLL(library_path())
    missing = [n for n in header_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    from helrm_amd.backend import EXPORTED_SYMBOLS
    assert set(header_symbols()) <= set(EXPORTED_SYMBOLS) | {"FreeCArray"}


def test_error_without_scheme_is_reported_not_fatal():
    from helrm_amd.backend import HipLibrary, HipError
    lib = HipLibrary()
    with pytest.raises(HipError, match="no scheme"):
        lib.GetModuliChain()
    with pytest.raises(HipError, match="no scheme"):
        lib.EvaluateLinearTransform(0, 0)
    assert "no scheme" in lib.lib.GetLastError().decode()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import helrm_amd
    monkeypatch.setattr(helrm_amd, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        helrm_amd.library_path()
