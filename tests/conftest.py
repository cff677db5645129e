import importlib.util
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PACKAGE_NAME = "demucs_wgpu_amd"


def load_package():
    """Import the `demucs-wgpu_amd/` package (its directory name is not an identifier)."""
    if PACKAGE_NAME in sys.modules:
        return sys.modules[PACKAGE_NAME]
    pkg_dir = ROOT / "demucs-wgpu_amd"
    spec = importlib.util.spec_from_file_location(PACKAGE_NAME, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PACKAGE_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (runs through the HIP C-ABI)")


@pytest.fixture(scope="session")
def dmx():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    load_package()
    from oracle import binding
    binding.lib()
    return binding


def snr_db(ref: np.ndarray, test: np.ndarray) -> float:
    """Energy SNR 10 log10(sum ref^2 / sum (ref - test)^2)."""
    ref = np.asarray(ref, np.float64)
    err = ref - np.asarray(test, np.float64)
    num = float(np.sum(ref * ref))
    den = float(np.sum(err * err))
    if den == 0.0:
        return float("inf")
    return 10.0 * np.log10(num / den)


def rms_relative_error(ref: np.ndarray, test: np.ndarray) -> float:
    """`rms_relative_error` of the reference's fixtures (crates/demucs-core/src/fixtures.rs:133-139)."""
    ref = np.asarray(ref, np.float64)
    err = ref - np.asarray(test, np.float64)
    return float(np.sqrt(np.mean(err * err)) / max(np.sqrt(np.mean(ref * ref)), 1e-30))


def small_config(dmx, segment_samples: int = 11025):
    """The real architecture with a short segment (0.25 s by default)."""
    cfg = dmx.Config()
    cfg.segment = segment_samples / cfg.samplerate
    assert cfg.training_length == segment_samples
    return cfg
