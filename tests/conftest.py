"""Shared fixtures: the `gpu` marker, the package loader, the oracle module and the reference's LCG streams."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the HIP library through its C-ABI)")


def load_package():
    """The package directory is `pyodide-llm_amd/` (not an identifier): load it as `pyodide_llm_amd`."""
    if "pyodide_llm_amd" in sys.modules:
        return sys.modules["pyodide_llm_amd"]
    where = os.path.join(ROOT, "pyodide-llm_amd")
    spec = importlib.util.spec_from_file_location("pyodide_llm_amd", os.path.join(where, "__init__.py"),
                                                  submodule_search_locations=[where])
    module = importlib.util.module_from_spec(spec)
    sys.modules["pyodide_llm_amd"] = module
    spec.loader.exec_module(module)
    return module


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o
