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


def test_unsupported_configurations_are_refused_before_any_device_work():
    """dmx_runner_create checks the config first (UnsupportedModel / Config
    kinds), so these errors need no GPU; the weights are never looked at."""
    import pytest
    pkg = load_package()
    cases = [dict(cac=0), dict(nfft=2048), dict(stride=2), dict(sources=6), dict(depth=6), dict(t_heads=4),
             dict(context=0)]
    for change in cases:
        cfg = pkg.Config(**change)
        with pytest.raises(pkg.DmxError) as e:
            pkg.Runner({}, cfg)
        assert e.value.kind == "UnsupportedModel", change
        assert "this backend needs" in str(e.value)
    with pytest.raises(pkg.DmxError) as e:
        pkg.Runner({}, pkg.Config(segment=0.0))
    assert e.value.kind == "Config"
