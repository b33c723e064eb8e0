"""pytest configuration: the `gpu` marker (tests that need an MI355X: run with -m gpu on the GPU box), shared paths and
session fixtures (synthetic models written once per session)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def workdir(tmp_path_factory):
    return str(tmp_path_factory.mktemp("gw"))


@pytest.fixture(scope="session")
def synth_models(workdir):
    """Paths of the small synthetic GGUF files (written on first use)."""
    from gwenedeg_amd import synth
    cache = {}

    def get(shape: str, seed: int = 1):
        key = (shape, seed)
        if key not in cache:
            cache[key] = synth.write_gguf(os.path.join(workdir, f"{shape}_{seed}.gguf"), shape, seed=seed)
        return cache[key]
    return get
