"""Test configuration: the `gpu` marker, and loaders for the package (whose
directory name, swin2sr-rs_amd, is not an identifier) and the oracle."""
import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def load_package():
    if "swin2sr_rs_amd" in sys.modules:
        return sys.modules["swin2sr_rs_amd"]
    pkgdir = ROOT / "swin2sr-rs_amd"
    spec = importlib.util.spec_from_file_location(
        "swin2sr_rs_amd", pkgdir / "__init__.py", submodule_search_locations=[str(pkgdir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["swin2sr_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_oracle():
    if "s2s_oracle_py" in sys.modules:
        return sys.modules["s2s_oracle_py"]
    load_package()
    spec = importlib.util.spec_from_file_location("s2s_oracle_py", ROOT / "oracle" / "oracle.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["s2s_oracle_py"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def orc():
    return load_oracle()
