import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """Import hy-mt-rs_amd/ (a directory name that is not an identifier)."""
    if "hy_mt_rs_amd" in sys.modules:
        return sys.modules["hy_mt_rs_amd"]
    pkg_dir = os.path.join(ROOT, "hy-mt-rs_amd")
    spec = importlib.util.spec_from_file_location(
        "hy_mt_rs_amd", os.path.join(pkg_dir, "__init__.py"),
        submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["hy_mt_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def hyq():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def gpu_ctx(hyq):
    """One device context for the whole GPU session (device 0)."""
    ctx = hyq.Context(0)
    yield ctx
    ctx.close()
