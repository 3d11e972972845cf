"""The C ABI of include/dj.h (CPU): libdj.so loads, exports every function the header declares, the
ctypes binding covers them all, and without a GPU dj_init fails with a decision.js error (no fallback)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    txt = open(os.path.join(ROOT, "include", "dj.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(dj_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_function(pkg):
    from decision_js_amd import _dj
    lib = ctypes.CDLL(_dj.LIB_PATH)
    names = declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(_dj.SIGNATURES) == names  # the binding covers exactly the header
    assert _dj.lib().dj_abi_version() == 1


def test_no_gpu_means_a_loud_error(pkg):
    from decision_js_amd import _dj
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    with pytest.raises(_dj.DJError, match="^decision.js: no HIP device"):
        _dj.Context(0)
    assert _dj.lib().dj_last_error().decode().startswith("decision.js:")


def test_missing_library_fails_loudly(pkg, monkeypatch):
    from decision_js_amd import _dj
    monkeypatch.setattr(_dj, "_lib", None)
    monkeypatch.setattr(_dj, "LIB_PATH", "/nonexistent/libdj.so")
    with pytest.raises(ImportError, match="libdj.so is missing"):
        _dj.lib()
