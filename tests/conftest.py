import os
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")
    config.addinivalue_line("markers", "slow: minutes of CPU time")


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def model_root():
    d = os.environ.get("L98_MODEL_DIR") or os.path.join(tempfile.gettempdir(), "l98_models")
    os.makedirs(d, exist_ok=True)
    return d


@pytest.fixture(scope="session")
def micro(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "micro"), 10, seed=1234)


@pytest.fixture(scope="session")
def tiny(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "tiny"), 0, seed=1234)


@pytest.fixture(scope="session")
def server(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "server"), 4, seed=1234)


@pytest.fixture(scope="session")
def micro_subln(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "micro_subln"), 12, seed=1234)


@pytest.fixture(scope="session")
def subln(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "subln"), 5, seed=1234)


# DSpark heads (mtp_n_draft > 1): micro, echo, tiny (v7, groups of 64, BF16)
# and micro-subln shapes
@pytest.fixture(scope="session")
def ds_micro(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "ds_micro"), 18, seed=1234)


@pytest.fixture(scope="session")
def ds_echo(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "ds_echo"), 19, seed=1234)


@pytest.fixture(scope="session")
def ds_tiny(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "ds_tiny"), 20, seed=1234)


@pytest.fixture(scope="session")
def ds_subln(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "ds_subln"), 21, seed=1234)
