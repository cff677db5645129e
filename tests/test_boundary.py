"""The C-ABI library loads without a GPU and exports every function that
include/*.h declares, each with a ctypes signature in _native.SIGNATURES."""
import ctypes
import re
from pathlib import Path

from conftest import ROOT, load_package


def declared_functions():
    names = set()
    for header in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        text = re.sub(r"typedef[^;]*;", "", text)
        names.update(re.findall(r"\b(dmx_[a-z0-9_]+)\s*\(", text))
    return names


def test_every_declared_function_is_exported_and_bound():
    load_package()
    from demucs_wgpu_amd import _native
    declared = declared_functions()
    assert len(declared) > 40
    lib = ctypes.CDLL(str(_native.LIBRARY_PATH))
    missing = sorted(n for n in declared if not hasattr(lib, n))
    assert not missing, missing
    unbound = sorted(declared - set(_native.SIGNATURES))
    assert not unbound, unbound
    extra = sorted(set(_native.SIGNATURES) - declared)
    assert not extra, extra
    _native.load()  # binds every signature
