import os
import sys
import tempfile

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "odin-infer_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def model_dir():
    d = tempfile.mkdtemp(prefix="oi_models_")
    yield d
    for f in os.listdir(d):
        try:
            os.remove(os.path.join(d, f))
        except OSError:
            pass
    try:
        os.rmdir(d)
    except OSError:
        pass


@pytest.fixture(scope="session")
def make_model(model_dir):
    from oi import synth
    cache = {}

    def make(name, **overrides):
        key = (name, tuple(sorted(overrides.items())))
        if key not in cache:
            path = os.path.join(model_dir, "%s_%d.gguf" % (name, len(cache)))
            synth.write_gguf(path, name, **overrides)
            cache[key] = path
        return cache[key]

    return make
