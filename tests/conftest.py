import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def _load_package():
    """Import the product package from the ``fusion-pcu_amd/`` directory as
    ``fusion_pcu_amd`` (a hyphenated directory is not importable by name)."""
    if "fusion_pcu_amd" in sys.modules:
        return sys.modules["fusion_pcu_amd"]
    pkg_dir = os.path.join(ROOT, "fusion-pcu_amd")
    spec = importlib.util.spec_from_file_location(
        "fusion_pcu_amd", os.path.join(pkg_dir, "__init__.py"),
        submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["fusion_pcu_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: full-size configuration (GPU box only)")


@pytest.fixture(scope="session")
def pcu_pkg():
    return _load_package()


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    return oracle
