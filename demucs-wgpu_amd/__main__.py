"""`python demucs-wgpu_amd <command> ...`: the command line of cli.py.

The directory name is not an identifier, so the package is loaded from its
path under the name demucs_wgpu_amd before the command runs."""
import importlib.util
import sys
from pathlib import Path


def _package():
    name = "demucs_wgpu_amd"
    if name in sys.modules:
        return sys.modules[name]
    here = Path(__file__).resolve().parent
    spec = importlib.util.spec_from_file_location(name, here / "__init__.py", submodule_search_locations=[str(here)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


if __name__ == "__main__":
    _package()
    from demucs_wgpu_amd import cli

    sys.exit(cli.main())
