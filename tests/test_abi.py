"""The C-ABI library loads and exports every entry point include/*.h declares (no GPU calls)."""
import ctypes
import glob
import os
import re

from tests.conftest import ROOT


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(mc_\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    names = declared_functions()
    assert {"mc_step", "mc_forward", "mc_ngram_propose", "mc_accept", "mc_batch_rollback"} <= names


def test_library_exports_every_declared_symbol():
    from mlxcat_amd import _lib
    assert os.path.exists(_lib.LIB_PATH), "build with python -m mlxcat_amd.build"
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the same set
    assert set(_lib.EXPORTS) == declared_functions()


def test_product_does_not_touch_the_oracle():
    """The product package never imports, links or loads anything under oracle/."""
    for path in glob.glob(os.path.join(ROOT, "mlxcat_amd", "**", "*"), recursive=True):
        if os.path.isdir(path) or path.endswith((".so", ".o", ".pyc")):
            continue
        text = open(path, errors="ignore").read()
        assert "pyoracle" not in text and "liboracle" not in text and "oracle.h" not in text, path


def test_missing_library_fails_loudly(tmp_path):
    from mlxcat_amd import _lib
    saved = _lib._lib
    try:
        _lib._lib = None
        try:
            _lib.load(str(tmp_path / "nope.so"))
        except ImportError as e:
            assert "no CPU fallback" in str(e)
        else:
            raise AssertionError("load() must raise without the HIP library")
    finally:
        _lib._lib = saved
