import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """The product package (its directory name is not an identifier)."""
    name = "power_cpu_llm_amd"
    if name in sys.modules:
        return sys.modules[name]
    path = os.path.join(ROOT, "power-cpu-llm_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pcl():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    from oracle import binding
    binding.load()
    return binding
