import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs libmx kernels on device 0)")


def load_mx():
    name = "speech_cpp_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg = ROOT / "speech.cpp_amd"
    spec = importlib.util.spec_from_file_location(name, pkg / "__init__.py", submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def mx():
    return load_mx()


@pytest.fixture(scope="session")
def be(mx):
    if mx.device_count() < 1:
        pytest.fail("the gpu tests need a GPU visible to libmx")
    b = mx.Backend(0)
    yield b
    b.close()
